// thunderfft.cuh -- drop-in include name of the reference's public header
// (mcrl/thunderfft include/thunderfft/thunderfft.cuh).  On MI355X the host
// API lives in thunderfft.hpp and the device-side fusion API in
// thunderfft_device.hpp; this file includes both so that existing
// `#include <thunderfft/thunderfft.cuh>` lines keep compiling under hipcc.
#pragma once
#include "thunderfft/thunderfft.hpp"
#include "thunderfft/thunderfft_device.hpp"
