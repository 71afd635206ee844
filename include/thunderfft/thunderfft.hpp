// thunderfft.hpp -- the reference's C++ host API on MI355X (gfx950).
//
// Same names, template parameters, argument order, synchronous semantics and
// exception contract as mcrl/thunderfft's include/thunderfft/thunderfft.cuh
// (:55-56 ThunderFFTInitialize, :62-63 ThunderFFTFinalize, :150-154
// ThunderFFT_global) and detail/util_cuda.h:46-49 (vec2_t).  Each call
// forwards to the C ABI of libthunderfft_amd.so (thunderfft/thunderfft.h) and
// turns its return code into the reference's exception:
//   THFF_EINVAL -> std::invalid_argument (raised before any HIP call)
//   THFF_EIO    -> std::runtime_error("[ThunderFFT] <context>: <hip error>")
// Differences from the reference: the stream is a hipStream_t, and a
// ThunderFFT_global<T,N> call on a device whose twiddle cache for T does not
// hold N throws std::runtime_error instead of running without it.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>
#include <type_traits>

#include "thunderfft/thunderfft.h"

template <class T>
using vec2_t = typename std::conditional_t<std::is_same_v<std::remove_cv_t<T>, float>, float2,
                                           half2>;

namespace thunderfft {

namespace detail {

template <class T>
constexpr int precision_code() {
    static_assert(std::is_same_v<T, float> || std::is_same_v<T, half>,
                  "ThunderFFT supports float and half only");
    return std::is_same_v<T, float> ? THFF_FLOAT : THFF_HALF;
}

inline void check(int rc) {
    if (rc == THFF_OK) return;
    if (rc == THFF_EINVAL) throw std::invalid_argument(thff_last_error());
    throw std::runtime_error(thff_last_error());
}

}  // namespace detail

// Supported transform lengths (include/thunderfft/thunderfft.cuh:20-23,145).
template <int N>
inline constexpr bool is_supported_length =
    N == 64 || N == 128 || N == 256 || N == 512 || N == 1024 || N == 2048 || N == 4096;

// Transforms per workgroup of the global kernel (the reference's
// batch_per_block<N>, detail/thunderfft_impl.cuh:14-22; wave64 values).
template <int N>
inline constexpr int batch_per_block = is_supported_length<N> ? 4096 / N : 0;

// Lanes per wavefront on gfx950 (the reference's threads_per_warp = 32).
inline constexpr int threads_per_warp = 64;

// Initialise the current device's twiddle table for (T, N).  Unsupported N
// throws std::invalid_argument before any HIP call; one N per (device, T).
template <typename T>
void ThunderFFTInitialize(int N) {
    detail::check(thff_initialize(detail::precision_code<T>(), N));
}

// Release the current device's twiddle table for T (repeat calls are fine).
template <typename T>
void ThunderFFTFinalize() {
    detail::check(thff_finalize(detail::precision_code<T>()));
}

// Device pointer of the current device's twiddle table for T (the table
// ThunderFFT_kernel_reg / ThunderFFT_load_twiddles read), nullptr when
// released.  The reference exposes the same state through its device symbols
// d_twiddle_{f,h} (detail/thunderfft_impl_twiddle.cuh:44-68).
template <typename T>
inline const float2* ThunderFFT_twiddle_table() {
    const void* table = nullptr;
    int n = 0;
    detail::check(thff_twiddle_info(detail::precision_code<T>(), &table, &n));
    return static_cast<const float2*>(table);
}

// Batched unnormalized out-of-place C2C FFT of `batch` natural-order signals
// of N values (signal j at offset j*N).  forward = exp(-2*pi*i*k/N).
// batch < 0, null or identical pointers, and pointers not aligned to their
// element (8 bytes for float2, 4 for half2) throw std::invalid_argument;
// batch 0 is a no-op.  Any element-aligned buffer is accepted, as in the
// reference; 16-byte aligned ones take the vectorised kernels.  Synchronises
// `stream` before returning.
template <typename T, int N, bool forward = true>
inline void ThunderFFT_global(vec2_t<T>* d_input, vec2_t<T>* d_output, int batch,
                              hipStream_t stream = 0) {
    static_assert(std::is_same_v<T, float> || std::is_same_v<T, half>,
                  "ThunderFFT_global supports float and half only");
    static_assert(is_supported_length<N>, "Unsupported ThunderFFT length");
    detail::check(thff_global(detail::precision_code<T>(), N, forward ? 1 : 0, d_input, d_output,
                              batch, static_cast<void*>(stream)));
}

// Fused circular convolution y[b] = IFFT(FFT(x[b]) * FFT(h[b or 0])) / N of
// `batch` signals of N values (per-signal filters, or one shared filter).
// No counterpart in the reference's library API; the reference ships the
// fused convolution as a sample kernel
// (sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331).  Same argument
// checks and synchronous semantics as ThunderFFT_global; Initialize<T>(N) first.
template <typename T, int N>
inline void ThunderFFT_conv1d(const vec2_t<T>* d_x, const vec2_t<T>* d_h, vec2_t<T>* d_y,
                              int batch, bool per_signal_filter = true, hipStream_t stream = 0) {
    static_assert(is_supported_length<N>, "Unsupported ThunderFFT length");
    detail::check(thff_conv1d(detail::precision_code<T>(), N, d_x, d_h, d_y, batch,
                              per_signal_filter ? 1 : 0, static_cast<void*>(stream)));
}

// Spectra of `channels` real fp32 filters h[d] (N taps each) for
// ThunderFFT_conv1d_real<T, N>: spectrum[d][k] = scale * FFT(h[d])[k], fp32
// complex.  Replaces the reference's filter_fft_once
// (sample/conv1d/conv1d_fullfft_l4096_thunder.cu:475-497); Initialize<T>(N) first.
template <typename T, int N>
inline void ThunderFFT_conv1d_real_filter(const float* d_h, float2* d_spectrum, int channels,
                                          float scale = 1.0f, hipStream_t stream = 0) {
    static_assert(is_supported_length<N>, "Unsupported ThunderFFT length");
    detail::check(thff_conv1d_real_filter(detail::precision_code<T>(), N, d_h, d_spectrum,
                                          channels, scale, static_cast<void*>(stream)));
}

// Fused real convolution of x[batch][channels][N] with one filter per channel:
// y[b][d] = Re IFFT(FFT(x[b][d]) * spectrum[d]), unnormalized (the reference's
// thunder_convN_block_kernel_realin_realout,
// sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331).
template <typename T, int N>
inline void ThunderFFT_conv1d_real(const T* d_x, const float2* d_spectrum, T* d_y, int batch,
                                   int channels, hipStream_t stream = 0) {
    static_assert(is_supported_length<N>, "Unsupported ThunderFFT length");
    detail::check(thff_conv1d_real(detail::precision_code<T>(), N, d_x, d_spectrum, d_y, batch,
                                   channels, static_cast<void*>(stream)));
}

// Tiled valid 1-D correlation y[b][i] = sum_k x[b][i + k] * taps[k] of `batch`
// signals of input_len values with 1 <= filter_len <= 64 fp32 complex taps,
// through 64-point FFT windows (the reference's sample/conv1d/main.cu:38-174).
// y holds batch * (input_len - filter_len + 1) values; Initialize<T>(64) first.
template <typename T>
inline void ThunderFFT_conv1d_valid(const vec2_t<T>* d_x, long long input_len,
                                    const float2* d_taps, int filter_len, vec2_t<T>* d_y,
                                    int batch = 1, hipStream_t stream = 0) {
    detail::check(thff_conv1d_valid(detail::precision_code<T>(), d_x, input_len, d_taps,
                                    filter_len, d_y, batch, static_cast<void*>(stream)));
}

// 2-D circular convolution of `batch` Rows x Cols images with one shared
// filter: y[b] = IFFT2(FFT2(x[b]) * FFT2(h)) / (Rows*Cols).  Rows = Cols = 64
// or 128 (one fused kernel per image), or 1024 (the reference's built sample
// shape: row pass, fused column pass, inverse row pass); Initialize<T>(Rows)
// first.  No counterpart in the reference's library API (its 2-D convolution
// is sample/conv2d/thunder.cu).
template <typename T, int Rows, int Cols>
inline void ThunderFFT_conv2d(const vec2_t<T>* d_x, const vec2_t<T>* d_h, vec2_t<T>* d_y, int batch,
                              hipStream_t stream = 0) {
    static_assert(Rows == Cols && (Rows == 64 || Rows == 128 || Rows == 1024),
                  "ThunderFFT_conv2d supports 64 x 64, 128 x 128 and 1024 x 1024 images");
    detail::check(thff_conv2d(detail::precision_code<T>(), Rows, Cols, d_x, d_h, d_y, batch,
                              static_cast<void*>(stream)));
}

}  // namespace thunderfft
