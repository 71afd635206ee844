// c2c_instance.hip -- instantiates the C2C kernels of one length THFF_N
// (compiled once per length, -DTHFF_N=64 ... 4096, so the lengths build in
// parallel).
#include "thunderfft/detail/fft_c2c.hpp"
#include "thunderfft/detail/fft_conv.hpp"
#include "thunderfft/detail/fft_conv_mfma.hpp"
#include "thunderfft/detail/fft_mfma.hpp"
#include "launch.hpp"

#include <type_traits>

#ifndef THFF_N
#error "compile with -DTHFF_N=<transform length>"
#endif

namespace thff {

// Launch shape per (N, precision), from sweeps on MI355X at batch = 2^26/N
// with random inputs: tiles each workgroup walks, and whether the next
// tile's loads are issued before the current tile is transformed.
struct LaunchShape {
    int tiles;
    bool prefetch;
};

template <int N>
constexpr LaunchShape launch_shape(int precision) {
    if (precision == 0) return N == 2048 ? LaunchShape{2, true} : LaunchShape{1, false};
    if (N <= 128) return {1, false};
    if (N == 2048) return {2, true};  // N = 256 ... 4096 run MFMA kernels
    if (N == 4096) return {0, false};  // the three-stage kernel: grid sized to the device
    return {2, N == 1024};
}

// half2 lengths whose radix-16 stages run on MFMA (fft_mfma.hpp): N = 256*C
// (two stages) and N = 4096 (three stages).
template <int N>
inline constexpr bool kHalfOnMfma = N >= 256 && N <= 2048;
template <int N>
inline constexpr bool kHalfOnMfma3 = N == 4096;

// Only the launch shape in use is instantiated.
template <class IO, int N, bool FWD>
void enqueue(unsigned grid, const IO* x, IO* y, int batch, const float2* tw, int tpb,
             hipStream_t stream) {
    constexpr bool kPf = launch_shape<N>(std::is_same_v<IO, float2> ? 0 : 1).prefetch;
    c2c_kernel<IO, N, FWD, kPf><<<grid, 256, 0, stream>>>(x, y, batch, tw, tpb);
}

template <int N, bool FWD>
void enqueue_mfma(unsigned grid, const __half2* x, __half2* y, int batch, const float2* tw,
                  int tpb, hipStream_t stream) {
    constexpr bool kPf = launch_shape<N>(1).prefetch;
    c2c_mfma_kernel<N / 256, FWD, kPf><<<grid, 256, 0, stream>>>(x, y, batch, tw, tpb);
}

template <bool FWD>
void enqueue_mfma4096(unsigned grid, const __half2* x, __half2* y, int batch, const float2* tw,
                      int tpb, hipStream_t stream) {
    constexpr bool kPf = launch_shape<4096>(1).prefetch;
    c2c_mfma4096_kernel<FWD, kPf><<<grid, 256, 0, stream>>>(x, y, batch, tw, tpb);
}

template <int N>
hipError_t launch_c2c(int precision, bool forward, const void* in, void* out, int batch,
                      const float2* tw, int num_cus, hipStream_t stream) {
    const LaunchShape shape = launch_shape<N>(precision);
    const bool mfma = precision != 0 && kHalfOnMfma<N>;
    long long fpb = C2CPlan<N>::kFPB;  // 1 for N = 4096 on either kernel
    if constexpr (kHalfOnMfma<N>)
        if (mfma) fpb = MfmaPlan<N / 256>::kFPB;
    const long long ntiles = (static_cast<long long>(batch) + fpb - 1) / fpb;
    // Small batches spread one tile per workgroup over the whole device.
    int tpb = ntiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? shape.tiles : 1;
    unsigned grid = static_cast<unsigned>((ntiles + tpb - 1) / tpb);
    if constexpr (kHalfOnMfma3<N>) {
        // The three-stage kernel: 2 workgroups per CU sharing the batch evenly
        // (tpb = 0) measured 99 us against 105-107 us for 4, 8 or 16 tiles per
        // workgroup (2^26 values, MI355X); its set-up is the heaviest.
        if (precision != 0) {
            const long long cap = 2LL * (num_cus > 0 ? num_cus : 256);
            grid = static_cast<unsigned>(ntiles < cap ? ntiles : cap);
            tpb = 0;
        }
    }
    if (precision == 0) {
        const auto* x = static_cast<const float2*>(in);
        auto* y = static_cast<float2*>(out);
        if (forward)
            enqueue<float2, N, true>(grid, x, y, batch, tw, tpb, stream);
        else
            enqueue<float2, N, false>(grid, x, y, batch, tw, tpb, stream);
    } else {
        const auto* x = static_cast<const __half2*>(in);
        auto* y = static_cast<__half2*>(out);
        if constexpr (kHalfOnMfma<N>) {
            if (forward)
                enqueue_mfma<N, true>(grid, x, y, batch, tw, tpb, stream);
            else
                enqueue_mfma<N, false>(grid, x, y, batch, tw, tpb, stream);
        } else if constexpr (kHalfOnMfma3<N>) {
            if (forward)
                enqueue_mfma4096<true>(grid, x, y, batch, tw, tpb, stream);
            else
                enqueue_mfma4096<false>(grid, x, y, batch, tw, tpb, stream);
        } else if (forward) {
            enqueue<__half2, N, true>(grid, x, y, batch, tw, tpb, stream);
        } else {
            enqueue<__half2, N, false>(grid, x, y, batch, tw, tpb, stream);
        }
    }
    return hipGetLastError();
}

template <class IO, int N>
void enqueue_conv1d(bool per_signal, unsigned grid, const IO* x, const IO* h, IO* y, int batch,
                    const float2* tw, int tpb, hipStream_t stream) {
    if (per_signal)
        conv1d_kernel<IO, N, true><<<grid, 256, 0, stream>>>(x, h, y, batch, tw, tpb);
    else
        conv1d_kernel<IO, N, false><<<grid, 256, 0, stream>>>(x, h, y, batch, tw, tpb);
}

template <int N>
hipError_t launch_conv1d(int precision, bool per_signal_filter, const void* x, const void* h,
                         void* y, int batch, const float2* tw, int num_cus, hipStream_t stream) {
    // fp16 N = 256 ... 2048: all three transforms on MFMA (fft_conv_mfma.hpp);
    // per-signal filters, 2^25 values, against the VALU path on MI355X:
    // 78 vs 90 us (N=256), 84 vs 116 (512), 93 vs 122 (1024), 106 vs 138 (2048).
    if constexpr (N >= 256 && N <= 2048) {
        if (precision != 0) {
            constexpr int C = N / 256;
            using M = MfmaPlan<C>;
            const long long ntiles = (static_cast<long long>(batch) + M::kFPB - 1) / M::kFPB;
            const int tpb = ntiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? (C == 8 ? 8 : 4) : 1;
            const unsigned grid = static_cast<unsigned>((ntiles + tpb - 1) / tpb);
            const auto* xx = static_cast<const __half2*>(x);
            const auto* hh = static_cast<const __half2*>(h);
            auto* yy = static_cast<__half2*>(y);
            if (per_signal_filter)
                conv1d_mfma_kernel<C, true><<<grid, 256, 0, stream>>>(xx, hh, yy, batch, tw, tpb);
            else
                conv1d_mfma_kernel<C, false><<<grid, 256, 0, stream>>>(xx, hh, yy, batch, tw, tpb);
            return hipGetLastError();
        }
    }
    // fp16 N = 4096: the three-stage MFMA transform, one signal per tile, the
    // grid sized to the kernel's occupancy (per-signal filters: 167 VGPRs, 3
    // workgroups per CU; a shared filter keeps its spectrum live across the
    // loop: 229 VGPRs, 2 per CU) with the signals shared out evenly.  2^25
    // values on MI355X: 109 vs 162 us per-signal, 76 vs 125 us shared,
    // against the VALU path.
    if constexpr (N == 4096) {
        if (precision != 0) {
            const long long cap = (per_signal_filter ? 3LL : 2LL) * (num_cus > 0 ? num_cus : 256);
            const unsigned grid = static_cast<unsigned>(batch < cap ? batch : cap);
            const auto* xx = static_cast<const __half2*>(x);
            const auto* hh = static_cast<const __half2*>(h);
            auto* yy = static_cast<__half2*>(y);
            if (per_signal_filter)
                conv1d_mfma4096_kernel<N, true><<<grid, 256, 0, stream>>>(xx, hh, yy, batch, tw);
            else
                conv1d_mfma4096_kernel<N, false><<<grid, 256, 0, stream>>>(xx, hh, yy, batch, tw);
            return hipGetLastError();
        }
    }
    using P = C2CPlan<N>;
    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    const int tpb = ntiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? 2 : 1;
    const unsigned grid = static_cast<unsigned>((ntiles + tpb - 1) / tpb);
    if (precision == 0)
        enqueue_conv1d<float2, N>(per_signal_filter, grid, static_cast<const float2*>(x),
                                  static_cast<const float2*>(h), static_cast<float2*>(y), batch, tw,
                                  tpb, stream);
    else
        enqueue_conv1d<__half2, N>(per_signal_filter, grid, static_cast<const __half2*>(x),
                                   static_cast<const __half2*>(h), static_cast<__half2*>(y), batch,
                                   tw, tpb, stream);
    return hipGetLastError();
}

template <int N>
hipError_t launch_conv1d_real_filter(const float* h, float2* spectrum, int channels, float scale,
                                     const float2* tw, hipStream_t stream) {
    const unsigned grid =
        static_cast<unsigned>((channels + C2CPlan<N>::kFPB - 1) / C2CPlan<N>::kFPB);
    conv1d_real_filter_kernel<N><<<grid, 256, 0, stream>>>(h, spectrum, channels, scale, tw);
    return hipGetLastError();
}

template <int N>
hipError_t launch_conv1d_real(int precision, const void* x, const float2* spectrum, void* y,
                              int batch, int channels, const float2* tw, int num_cus,
                              hipStream_t stream) {
    using P = C2CPlan<N>;
    const long long transforms = (static_cast<long long>(batch) + 1) / 2 * channels;
    // fp16 N = 256 ... 1024: both transforms on MFMA (fft_conv_mfma.hpp);
    // measured against this VALU path at 2^26 samples: 64 vs 68 us (N=256),
    // 68 vs 87 (512), 74 vs 87 (1024).
    if constexpr (N >= 256 && N <= 1024) {
        if (precision != 0) {
            // 4 tiles per workgroup amortise the set-up (twiddle table, three
            // operand sets): 16-20% faster than 1 or 2 on MI355X.
            using M = MfmaPlan<N / 256>;
            const long long ntiles = (transforms + M::kFPB - 1) / M::kFPB;
            const int tpb = ntiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? 4 : 1;
            const unsigned grid = static_cast<unsigned>((ntiles + tpb - 1) / tpb);
            conv1d_real_mfma_kernel<N / 256><<<grid, 256, 0, stream>>>(
                static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch, channels,
                tw, tpb);
            return hipGetLastError();
        }
    }
    // fp16 N = 4096: the three-stage MFMA transform, both directions.
    if constexpr (N == 4096) {
        if (precision != 0) {
            // 2 workgroups per CU sharing the transforms evenly: 87-90 us
            // against 107 us for 4 tiles per workgroup (2^26 samples, MI355X).
            const long long cap = 2LL * (num_cus > 0 ? num_cus : 256);
            const unsigned grid = static_cast<unsigned>(transforms < cap ? transforms : cap);
            conv1d_real_mfma4096_kernel<N><<<grid, 256, 0, stream>>>(
                static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch, channels,
                tw, 0);
            return hipGetLastError();
        }
    }
    const long long ntiles = (transforms + P::kFPB - 1) / P::kFPB;
    const int tpb = ntiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? 2 : 1;
    const unsigned grid = static_cast<unsigned>((ntiles + tpb - 1) / tpb);
    if (precision == 0)
        conv1d_real_kernel<float2, N><<<grid, 256, 0, stream>>>(
            static_cast<const float*>(x), spectrum, static_cast<float*>(y), batch, channels, tw,
            tpb);
    else
        conv1d_real_kernel<__half2, N><<<grid, 256, 0, stream>>>(
            static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch, channels, tw,
            tpb);
    return hipGetLastError();
}

#if THFF_N == 64
hipError_t launch_conv1d_valid(int precision, const void* x, long long len, const float2* taps,
                               int ntaps, void* y, int batch, const float2* tw, int num_cus,
                               hipStream_t stream) {
    // A group is the 64 windows (one per transform slot) of one workgroup
    // pass; a workgroup walks several when there are many, so its filter
    // transform is shared.
    const long long valid = 65 - ntaps;
    const long long windows = (len - ntaps + 1 + valid - 1) / valid;
    const long long groups = (windows + 63) / 64 * batch;
    const int gpb = groups >= 16LL * (num_cus > 0 ? num_cus : 256) ? 4 : 1;
    const unsigned grid = static_cast<unsigned>((groups + gpb - 1) / gpb);
    if (precision == 0)
        conv1d_valid_kernel<float2><<<grid, 256, 0, stream>>>(
            static_cast<const float2*>(x), taps, static_cast<float2*>(y), len, ntaps, batch, tw,
            gpb);
    else
        conv1d_valid_kernel<__half2><<<grid, 256, 0, stream>>>(
            static_cast<const __half2*>(x), taps, static_cast<__half2*>(y), len, ntaps, batch, tw,
            gpb);
    return hipGetLastError();
}

hipError_t launch_conv2d64(int precision, const void* x, const void* h, void* y, int batch,
                           const float2* tw, int num_cus, hipStream_t stream) {
    // One image per tile; a workgroup transforms the filter once, so it
    // walks several images when the batch is large.
    const long long tiles = batch;
    const int tpb = tiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? 8 : 1;
    const unsigned grid = static_cast<unsigned>((tiles + tpb - 1) / tpb);
    if (precision == 0)
        conv2d64_kernel<float2><<<grid, 256, 0, stream>>>(static_cast<const float2*>(x),
                                                          static_cast<const float2*>(h),
                                                          static_cast<float2*>(y), batch, tw, tpb);
    else
        conv2d64_kernel<__half2><<<grid, 256, 0, stream>>>(static_cast<const __half2*>(x),
                                                           static_cast<const __half2*>(h),
                                                           static_cast<__half2*>(y), batch, tw, tpb);
    return hipGetLastError();
}
#endif

template hipError_t launch_c2c<THFF_N>(int, bool, const void*, void*, int, const float2*, int,
                                       hipStream_t);
template hipError_t launch_conv1d<THFF_N>(int, bool, const void*, const void*, void*, int,
                                          const float2*, int, hipStream_t);
template hipError_t launch_conv1d_real_filter<THFF_N>(const float*, float2*, int, float,
                                                      const float2*, hipStream_t);
template hipError_t launch_conv1d_real<THFF_N>(int, const void*, const float2*, void*, int, int,
                                               const float2*, int, hipStream_t);

}  // namespace thff
