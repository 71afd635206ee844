// launch.hpp -- internal launch entry points shared by the C ABI (capi.cpp)
// and the per-length kernel translation units (c2c_n*.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace thff {

// Enqueue the batched C2C kernel for length N.  precision: 0 float2, 1 half2.
// aligned16: both buffers start on a 16-byte boundary (otherwise they need
// only the element's alignment, and tiles move value by value).  tw: the
// device's fp32 table of N values (cos, sin)(2*pi*m/N); num_cus: the
// device's compute-unit count (sizes the grid).
template <int N>
hipError_t launch_c2c(int precision, bool forward, bool aligned16, const void* in, void* out,
                      int batch, const float2* tw, int num_cus, hipStream_t stream);

// Enqueue the fused circular convolution of `batch` signals of length N:
// y[b] = IFFT(FFT(x[b]) * FFT(h[per_signal_filter ? b : 0])) / N.
template <int N>
hipError_t launch_conv1d(int precision, bool per_signal_filter, const void* x, const void* h,
                         void* y, int batch, const float2* tw, int num_cus, hipStream_t stream);

// Enqueue the spectra of `channels` real fp32 filters h[d] (N taps each):
// spectrum[d][k] = scale * FFT(h[d])[k], fp32 complex.
template <int N>
hipError_t launch_conv1d_real_filter(const float* h, float2* spectrum, int channels, float scale,
                                     const float2* tw, hipStream_t stream);

// Enqueue the fused real convolution of x[batch][channels][N] (float or half)
// with the channel spectra: y[b][d] = IFFT(FFT(x[b][d]) * spectrum[d]), real.
template <int N>
hipError_t launch_conv1d_real(int precision, const void* x, const float2* spectrum, void* y,
                              int batch, int channels, const float2* tw, int num_cus,
                              hipStream_t stream);

// Enqueue the tiled valid correlation y[b][i] = sum_{k < ntaps} x[b][i + k] * taps[k]
// (i < len - ntaps + 1, 1 <= ntaps <= 64) with 64-point FFT windows (tw: the
// N = 64 table); taps are fp32 complex.
hipError_t launch_conv1d_valid(int precision, const void* x, long long len, const float2* taps,
                               int ntaps, void* y, int batch, const float2* tw, int num_cus,
                               hipStream_t stream);

// Enqueue the fused 2-D circular convolution of `batch` 64 x 64 images with
// one shared 64 x 64 filter h (tw: the N = 64 table).
hipError_t launch_conv2d64(int precision, const void* x, const void* h, void* y, int batch,
                           const float2* tw, int num_cus, hipStream_t stream);

// Enqueue the fused 2-D circular convolution of `batch` 128 x 128 images with
// one shared 128 x 128 filter h (tw: the N = 128 table).
hipError_t launch_conv2d128(int precision, const void* x, const void* h, void* y, int batch,
                            const float2* tw, int num_cus, hipStream_t stream);

// Enqueue the column pass of the multi-pass 2-D convolution over `images`
// 1024-row images with `cols` columns (tw: the N = 1024 table).  conv:
// out = IFFT_col(FFT_col(in) * H) (in, out: the precision's storage, may be
// the same buffer; H fp32 rows x cols); otherwise out = scale * FFT_col(in)
// with out fp32 complex.
hipError_t launch_conv2d_cols(int precision, bool conv, const void* in, void* out,
                              const float2* H, int cols, long long images, float scale,
                              const float2* tw, int num_cus, hipStream_t stream);

// Transforms per tile (4096 complex values, one workgroup pass) for length N.// Transforms per tile (4096 complex values, one workgroup pass) for length N.
int c2c_transforms_per_block(int n);


hipError_t launch_fill_uniform(int precision, void* out, long long count, unsigned long long seed,
                               long long first_element, hipStream_t stream);
hipError_t launch_copy_nt(void* dst, const void* src, long long bytes, hipStream_t stream);

}  // namespace thff
