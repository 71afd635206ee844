// thunderfft.cuh -- drop-in include name of the reference's public header
// (mcrl/thunderfft include/thunderfft/thunderfft.cuh).  On MI355X the API
// lives in thunderfft.hpp; this file only forwards to it so that existing
// `#include <thunderfft/thunderfft.cuh>` lines keep compiling under hipcc.
#pragma once
#include "thunderfft/thunderfft.hpp"
