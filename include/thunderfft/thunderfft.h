/*
 * thunderfft.h -- C ABI of the MI355X (gfx950) ThunderFFT library
 * (libthunderfft_amd.so).
 *
 * The reference (mcrl/thunderfft) is a header-only CUDA C++ template API with
 * no C ABI.  Each entry point below is the plain-pointer form of one
 * reference interface, cited as path:line in the reference tree; the C++
 * template API of the reference is restated on top of these entry points in
 * <thunderfft/thunderfft.hpp>.  No PyTorch or HIP types appear in the
 * signatures: streams are passed as `void*` (a hipStream_t, NULL = the null
 * stream) and buffers as device pointers.
 *
 * Return codes: THFF_OK on success; THFF_EINVAL where the reference throws
 * std::invalid_argument (always before any HIP call); THFF_EIO where it
 * throws std::runtime_error("[ThunderFFT] ...").  thff_last_error() returns
 * the message of the calling thread's last failure.
 */
#ifndef THUNDERFFT_AMD_THUNDERFFT_H
#define THUNDERFFT_AMD_THUNDERFFT_H

#ifdef __cplusplus
extern "C" {
#endif

#define THFF_OK 0
#define THFF_EINVAL (-22)
#define THFF_EIO (-5)

/* Component type T of the reference templates: float (float2 storage) or
 * half (__half2 storage, low = real, high = imaginary). */
#define THFF_FLOAT 0
#define THFF_HALF 1

/* Library version, major*10000 + minor*100 + patch. */
int thff_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* thff_last_error(void);

/* ThunderFFTInitialize<T>(N)
 *   reference: include/thunderfft/thunderfft.cuh:55-56,
 *              include/thunderfft/detail/thunderfft_impl_twiddle.cuh:279-327.
 * Builds (or keeps, if it already holds N) the current device's twiddle table
 * for `precision`: N fp32 complex values W[m] = (cos, sin)(2*pi*m/N), computed
 * in fp64 and rounded once.  One N per (device, precision); another N
 * replaces it.  N outside {64,...,4096} (powers of two) -> THFF_EINVAL before
 * any HIP call.  Serialised per precision; not stream ordered: finish every
 * transform that uses the old table before replacing it. */
int thff_initialize(int precision, int n);

/* ThunderFFTFinalize<T>()
 *   reference: include/thunderfft/thunderfft.cuh:62-63,
 *              include/thunderfft/detail/thunderfft_impl_twiddle.cuh:358-378.
 * Frees the current device's table for `precision`; a second call is a no-op.
 * Other devices' tables are untouched. */
int thff_finalize(int precision);

/* ThunderFFT_global<T,N,forward>(d_input, d_output, batch, stream)
 *   reference: include/thunderfft/thunderfft.cuh:150-154,
 *              include/thunderfft/detail/thunderfft_impl_kernel.cuh:6-41.
 * Batched, unnormalized, out-of-place C2C transforms of `batch` contiguous
 * natural-order signals of n complex values (signal b at offset b*n).
 * forward != 0 uses exp(-2*pi*i*n*k/N), forward == 0 exp(+...).
 * Argument checks in the reference's order, all before any HIP call:
 *   unsupported precision or n -> THFF_EINVAL (a static_assert there);
 *   batch < 0 -> THFF_EINVAL; batch == 0 -> THFF_OK without touching the
 *   pointers; null d_input or d_output, or d_input == d_output -> THFF_EINVAL;
 *   a buffer not aligned to its element (8 bytes for float2, 4 bytes for
 *   half2) -> THFF_EINVAL, since no kernel can read a split element.
 * Any element-aligned buffer is accepted, as in the reference: buffers on a
 * 16-byte boundary (every hipMalloc pointer, and every offset of whole
 * transforms of >= 2 values) take the vectorised kernels; others take a
 * kernel that moves single elements.
 * Requires thff_initialize(precision, n) on the current device (THFF_EIO
 * otherwise).  Synchronises `stream` before returning, like the reference. */
int thff_global(int precision, int n, int forward, const void* d_input, void* d_output,
                int batch, void* stream);

/* Same as thff_global without the final stream synchronisation: the launch is
 * enqueued on `stream` and the call returns.  No counterpart in the
 * reference (whose wrapper always synchronises); for callers that time or
 * pipeline transforms.  Same checks and return codes. */
int thff_global_async(int precision, int n, int forward, const void* d_input, void* d_output,
                      int batch, void* stream);

/* Fused circular convolution (no function counterpart in the reference
 * library; the reference ships it as the sample kernel
 * thunder_convN_block_kernel_realin_realout,
 * sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331, which this
 * generalises to complex signals, all seven lengths and per-signal filters):
 *   y[b][k] = sum_m x[b][m] * h[f][(k - m) mod n],  f = per_signal_filter ? b : 0,
 * computed as IFFT(FFT(x[b]) * FFT(h[f])) / n in one kernel (forward FFT,
 * pointwise product, inverse FFT and the 1/n scale; the spectra stay on chip).
 * x and y hold batch*n complex values, h holds batch*n (per-signal) or n
 * (shared) values, all in `precision` storage, natural order.  Same checks and
 * return codes as thff_global (y may alias neither x nor h), except that x, h
 * and y must start on a 16-byte boundary (THFF_EINVAL otherwise: the fused
 * kernels move 16-byte vectors only; every offset of whole signals meets it).
 * Requires thff_initialize(precision, n), synchronises `stream` before
 * returning. */
int thff_conv1d(int precision, int n, const void* d_x, const void* d_h, void* d_y, int batch,
                int per_signal_filter, void* stream);

/* thff_conv1d without the final stream synchronisation. */
int thff_conv1d_async(int precision, int n, const void* d_x, const void* d_h, void* d_y,
                      int batch, int per_signal_filter, void* stream);

/* Spectra of `channels` real filters for thff_conv1d_real: for every channel
 * d, spectrum[d][k] = scale * FFT(h[d])[k], k < n, as fp32 complex (8 bytes per
 * value, natural order).  h holds channels*n real fp32 taps, zero-padded to n,
 * for both precisions; `precision` names the convolution the spectra are for
 * (its twiddle table is used).  Replaces the reference's filter-spectrum
 * preparation filter_fft_once (cuFFT C2C + f32_to_h2 + permute_filter_layout*,
 * sample/conv1d/conv1d_fullfft_l4096_thunder.cu:475-497,154-226); scale = 1
 * gives its spectra, scale = 1/n folds the inverse's normalisation in.
 * Requires thff_initialize(precision, n); THFF_EINVAL for a bad precision or
 * length, channels < 0, null or aliased pointers; channels = 0 is a no-op.
 * Synchronises `stream` before returning. */
int thff_conv1d_real_filter(int precision, int n, const void* d_h, void* d_spectrum,
                            int channels, float scale, void* stream);

/* thff_conv1d_real_filter without the final stream synchronisation. */
int thff_conv1d_real_filter_async(int precision, int n, const void* d_h, void* d_spectrum,
                                  int channels, float scale, void* stream);

/* Fused real-input, real-output convolution with one filter per channel (the
 * reference's thunder_convN_block_kernel_realin_realout,
 * sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331, launched by run_case
 * :508-515; the reference instantiates n = 256, 1024, 4096 in half, this
 * takes all seven lengths in float or half):
 *   y[b][d] = Re IFFT(FFT(x[b][d]) * spectrum[d])   (unnormalized inverse),
 * x and y real [batch][channels][n] in `precision` storage, spectrum from
 * thff_conv1d_real_filter(precision, n, ...) for the same channels.  With
 * scale = 1 the output is n * (x (*) h), as the reference writes it; with
 * scale = 1/n it is the circular convolution x (*) h.  x and y must be
 * 16-byte aligned.  Same checks and return codes as thff_conv1d (y may alias
 * neither x nor spectrum; channels <= 0 is THFF_EINVAL when batch > 0).
 * Synchronises `stream` before returning. */
int thff_conv1d_real(int precision, int n, const void* d_x, const void* d_spectrum, void* d_y,
                     int batch, int channels, void* stream);

/* thff_conv1d_real without the final stream synchronisation. */
int thff_conv1d_real_async(int precision, int n, const void* d_x, const void* d_spectrum,
                           void* d_y, int batch, int channels, void* stream);

/* Tiled valid 1-D correlation with 64-point FFT windows (overlap-save), the
 * reference's conv1d_direct_fft_kernel (sample/conv1d/main.cu:38-128, driven
 * by main :207-336 with the definition of :156-174):
 *   y[b][i] = sum_{k < filter_len} x[b][i + k] * taps[k],  i < input_len - filter_len + 1,
 * complex, no conjugation.  x holds batch signals of input_len values and y
 * batch outputs of input_len - filter_len + 1 values, both in `precision`
 * storage; taps are filter_len fp32 complex values (float2) for both
 * precisions.  1 <= filter_len <= 64 and input_len >= filter_len (the
 * sample's checks, main.cu:223-230), THFF_EINVAL otherwise; batch < 0, null,
 * aliased or misaligned pointers are THFF_EINVAL, batch = 0 is a no-op.
 * Requires thff_initialize(precision, 64) (the windows are 64-point
 * transforms).  Synchronises `stream` before returning. */
int thff_conv1d_valid(int precision, const void* d_x, long long input_len, const void* d_taps,
                      int filter_len, void* d_y, int batch, void* stream);

/* thff_conv1d_valid without the final stream synchronisation. */
int thff_conv1d_valid_async(int precision, const void* d_x, long long input_len,
                            const void* d_taps, int filter_len, void* d_y, int batch,
                            void* stream);

/* Fused 2-D circular convolution of `batch` rows x cols row-major images with
 * one shared rows x cols filter (no function counterpart in the reference
 * library; the reference's 2-D convolution is the sample
 * sample/conv2d/thunder.cu:70-207,556-565, row FFT -> column FFT x H ->
 * column IFFT -> row IFFT over one 1024 x 1024 image, and the unbuilt 64 x 64
 * tile sketch sample/conv2d/thunder_tile64.cu:33-208):
 *   y[b][r][c] = sum_{r',c'} x[b][r'][c'] * h[(r - r') mod rows][(c - c') mod cols],
 * computed as IFFT2(FFT2(x[b]) * FFT2(h)) / (rows*cols).  rows = cols = 64 or
 * 128: one fused kernel (forward 2-D FFT, product, inverse) per image, the
 * image on chip.  rows = cols = 1024 (the reference's sample shape): the
 * filter's spectrum goes to a workspace the call allocates stream-ordered
 * (hipMallocAsync, 8 MiB) and frees the same way, then row FFTs x -> y, a
 * column pass (FFT, product, inverse FFT) and inverse row FFTs in place in
 * y.  Other shapes -> THFF_EINVAL; requires thff_initialize(precision, rows).
 * x and y hold batch*rows*cols complex values, h rows*cols.  Same checks,
 * return codes and synchronisation as thff_conv1d. */
int thff_conv2d(int precision, int rows, int cols, const void* d_x, const void* d_h, void* d_y,
                int batch, void* stream);

/* thff_conv2d without the final stream synchronisation. */
int thff_conv2d_async(int precision, int rows, int cols, const void* d_x, const void* d_h,
                      void* d_y, int batch, void* stream);

/* thff_conv2d_async that allocates nothing.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, checks, results and return codes as thff_conv2d_async
 * (enqueued on `stream`, no synchronisation); the 1024 x 1024 form keeps the
 * filter's spectrum in a device array of the library (8 MiB per GPU, held
 * until the process ends) instead of a stream-ordered allocation, so images
 * larger than 1024 x 1024 are THFF_EINVAL.  Every call on one GPU shares
 * that array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller.  Requires
 * thff_initialize(precision, rows) on the current device, as thff_conv2d. */
int thff_conv2d_noalloc(int precision, int rows, int cols, const void* d_x, const void* d_h,
                        void* d_y, int batch, void* stream);

/* Snapshot of the current device's twiddle cache for `precision`: the device
 * pointer (NULL when released) and its length (0 when released).  The
 * reference exposes the same state through its device symbols
 * d_twiddle_{f,h} / d_twiddle_N_{f,h}
 * (include/thunderfft/detail/thunderfft_impl_twiddle.cuh:44-68), read by
 * sample/validation/cache_validation.cu:36-50.  Entries are fp32 complex
 * (8 bytes) for both precisions. */
int thff_twiddle_info(int precision, const void** d_table, int* n);

/* Benchmark/test input generator (no reference counterpart; the reference
 * seeds its inputs on the host or with an LCG kernel,
 * sample/bench/paper_fft.cu:27-43).  Writes `count` complex values to
 * d_out in `precision` storage: component c (real of element e is
 * c = 2*(first_element + e), imaginary c + 1) is
 * 2 * (splitmix64(seed ^ c) >> 40) * 2^-24 - 1, exact in fp32, rounded to
 * nearest-even for half.  Asynchronous on `stream`. */
int thff_fill_uniform(int precision, void* d_out, long long count, unsigned long long seed,
                      long long first_element, void* stream);

/* Benchmark helper (no reference counterpart): copies `bytes` (a multiple
 * of 16) from d_src to d_dst with one 16-byte non-temporal load and store per
 * lane, the fastest streaming copy measured on MI355X.  It gives the device's
 * read-plus-write ceiling beside the transforms (bench.py).  Null,
 * misaligned or overlapping buffers and bad sizes -> THFF_EINVAL before any
 * HIP call; bytes = 0 is a no-op.  Asynchronous on `stream`. */
int thff_copy_nt(void* d_dst, const void* d_src, long long bytes, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* THUNDERFFT_AMD_THUNDERFFT_H */
