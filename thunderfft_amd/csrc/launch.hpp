// launch.hpp -- internal launch entry points shared by the C ABI (capi.cpp)
// and the per-length kernel translation units (c2c_n*.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace thff {

// Enqueue the batched C2C kernel for length N.  precision: 0 float2, 1 half2.
// tw: the device's fp32 table of N values (cos, sin)(2*pi*m/N).
template <int N>
hipError_t launch_c2c(int precision, bool forward, const void* in, void* out, int batch,
                      const float2* tw, hipStream_t stream);

// Transforms per workgroup (256 lanes) for length N; sizes the grid.
int c2c_transforms_per_block(int n);

hipError_t launch_fill_uniform(int precision, void* out, long long count, unsigned long long seed,
                               long long first_element, hipStream_t stream);

}  // namespace thff
