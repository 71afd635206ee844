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

// Grids.  per_cu = 0: one workgroup per tile.  per_cu = k: min(ntiles, k x
// CUs) workgroups walking the tiles grid-stride (tiles_per_block = 0,
// tile_walk in fft_tile.hpp), so the workgroups resident at any moment work
// on neighbouring tiles and one workgroup's set-up (twiddles, DFT operands, a
// shared filter's transform) serves many tiles.  The k of each kernel below
// is the fastest of 1, 2, 3, 4, 6, 8 and 16 on MI355X at 2^25-2^26 values
// per array (usually the kernel's occupancy in workgroups per CU).
struct Grid {
    unsigned blocks;
    int tiles_per_block;
};

inline Grid make_grid(long long ntiles, int per_cu, int num_cus) {
    if (per_cu <= 0) return {static_cast<unsigned>(ntiles), 1};
    const long long g = static_cast<long long>(per_cu) * (num_cus > 0 ? num_cus : 256);
    return {static_cast<unsigned>(ntiles < g ? ntiles : g), 0};
}

// C2C launch shape per (N, precision): workgroups per CU (make_grid) and
// whether the next tile's loads are issued before the current tile is
// transformed.  Measured at batch = 2^26/N:
//   fp32 N <= 1024: one tile per workgroup, 172-177 us (device grids: 181+).
//   fp32 N = 2048, 4096: 16 per CU with prefetch, 184 us (one or two tiles
//     per workgroup: 188-194 us); with direct movement, same box: 178 / 180 us
//     against 12 per CU 181 / 179, 8 per CU 184 / 180, 4 per CU 189 / 181,
//     8 per CU without prefetch 186 / 186, one tile per workgroup 181 / 186.
//     fp32 N = 2048 as one transform per 128-lane workgroup (each pass
//     barrier then spans the transform's 2 waves, not 4): 172.6 us at 32
//     per CU, 180.8 at 16, against 173.3 us (same box).
//   fp16 N = 2048 (three-stage MFMA, two transforms per tile): 2 per CU with
//     prefetch 88.2-88.5 us, against 90.6 at 3 per CU and 105.6 without
//     prefetch (the two-stage one-transform-per-wave kernel it replaced:
//     93-95 us at 2 per CU).
//   fp16 N = 64 (VALU): one tile per workgroup.
//   fp16 N = 128 (MFMA, c2c_mfma128_kernel): 2 per CU with prefetch 87.3 us,
//     against 90.0 at 3 per CU, 99.5 with one tile per workgroup and 90.3-91.1
//     for the VALU kernel (one tile per workgroup; device grids 93).
//   fp16 N = 256 ... 1024: the one-shot kernel (kHalfOneShot below), whose
//     shape is fixed there.  Before it, with the table-based kernel: N = 256
//     one tile per workgroup, 86.0-88.7 us wherever the output lies; the
//     2-per-CU grid-stride walk with prefetch as fast only for some output
//     placements (86.3-103 us over 12 offsets of y from x, one box); N = 512,
//     1024 on the walk (one tile per workgroup took 98-114 us for them, the
//     per-tile table set-up included).
//   fp16 MFMA (the walk): 2 per CU with prefetch, 86-91 us.  Runs
//     of contiguous tiles per workgroup, which leave the balancing to the
//     dispatcher, are slower: 2 tiles 87-98 us, 4-32 tiles 93-110 us (the
//     grid-stride walk keeps all workgroups on neighbouring tiles).
// `direct` (VALU kernel): tiles move between HBM and the first pass's
// registers with no LDS staging (DirectIO, fft_tile.hpp).  fp32, same box:
// N = 256 170 vs 175 us, 512 172 vs 174, 2048 180 vs 184, 4096 179 vs 183;
// 1024 174 vs 173; 64 and 128 244 / 192 vs 172 us (a wave instruction then
// covers 16 or 8 transforms with 32- or 64-byte pieces).
struct LaunchShape {
    int per_cu;
    bool prefetch;
    bool direct = false;
};

template <int N>
constexpr LaunchShape launch_shape(int precision) {
    if (precision == 0)
        return N <= 1024 ? LaunchShape{0, false, N == 256 || N == 512}
                         : LaunchShape{16, true, true};
    if (N == 128) return {2, true};
    if (N <= 128 || N == 256) return {0, false};
    return {2, true};
}

// half2 lengths whose radix-16 stages run on MFMA (fft_mfma.hpp): N = 256*C
// (two stages), N = 2048, 4096 (three stages across a workgroup) and N = 128
// (a DFT16 and a DFT8 pair within a wave).
template <int N>
inline constexpr bool kHalfOnMfma = N >= 256 && N <= 1024;
template <int N>
inline constexpr bool kHalfOnMfma3 = N == 2048 || N == 4096;
template <int N>
inline constexpr bool kHalfOnMfma128 = N == 128;

// Only the launch shape in use is instantiated.
template <class IO, int N, bool FWD>
void enqueue(Grid g, const IO* x, IO* y, int batch, const float2* tw, hipStream_t stream) {
    constexpr LaunchShape kShape = launch_shape<N>(std::is_same_v<IO, float2> ? 0 : 1);
    c2c_kernel<IO, N, FWD, kShape.prefetch, kShape.direct><<<g.blocks, 256, 0, stream>>>(
        x, y, batch, tw, g.tiles_per_block);
}

// fp16 N = 256 ... 1024 run the one-shot kernel (c2c_mfma_wave_kernel: one
// tile per wave, the wave's twiddles computed in the kernel, no LDS table,
// no workgroup barrier) instead of the persistent 2-per-CU grid-stride
// kernel (c2c_mfma_kernel, whose workgroups build LDS tables once and walk
// many tiles).  2^26 values, same output buffer, alternating (MI355X):
// N = 1024 86.6-87.0 against 88.4-89.1 us, 512 86.4-87.0 against 86.8-87.6,
// 256 85.7-86.4 against 86.5-87.6; over 8 output placements (bench.py's
// placement leg) 86.9-88.4 us against 90.0-102.0 us at N = 1024: the
// dispatcher keeps the CUs evenly fed, as for a streaming copy, and the
// time no longer depends on where the output lies.  Workgroups of 1 or 2
// such waves: 86.4-87.0 and 87.1-87.2 us at N = 1024, slower at 256 and 512.
// The three-stage kernels (N = 2048, 4096) as one tile per workgroup with
// computed twiddles took 128.3-128.8 and 94.7-95.1 us against 89.3-89.9 and
// 89.5-89.9 us, so they keep the persistent walk.
template <int N>
inline constexpr bool kHalfOneShot = N >= 256 && N <= 1024;
inline constexpr int kHalfOneShotWaves = 4;  // waves (tiles) per workgroup

template <int N, bool FWD>
void enqueue_mfma(Grid g, const __half2* x, __half2* y, int batch, const float2* tw,
                  hipStream_t stream) {
    if constexpr (kHalfOneShot<N>) {
        constexpr int kW = kHalfOneShotWaves;
        constexpr long long kPerBlock = static_cast<long long>(kW) * MfmaPlan<N / 256>::kFPW;
        const long long blocks = (static_cast<long long>(batch) + kPerBlock - 1) / kPerBlock;
        if (blocks <= 0) return;
        c2c_mfma_wave_kernel<N / 256, FWD, kW><<<static_cast<unsigned>(blocks), 64 * kW, 0, stream>>>(
            x, y, batch);
        (void)g;
        (void)tw;
    } else {
        constexpr bool kPf = launch_shape<N>(1).prefetch;
        c2c_mfma_kernel<N / 256, FWD, kPf><<<g.blocks, 256, 0, stream>>>(x, y, batch, tw,
                                                                         g.tiles_per_block);
    }
}

template <bool FWD>
void enqueue_mfma128(Grid g, const __half2* x, __half2* y, int batch, const float2* tw,
                     hipStream_t stream) {
    constexpr bool kPf = launch_shape<128>(1).prefetch;
    c2c_mfma128_kernel<FWD, kPf><<<g.blocks, 256, 0, stream>>>(x, y, batch, tw, g.tiles_per_block);
}

template <int N, bool FWD>
void enqueue_mfma3(Grid g, const __half2* x, __half2* y, int batch, const float2* tw,
                   hipStream_t stream) {
    constexpr bool kPf = launch_shape<N>(1).prefetch;
    if constexpr (N == 2048)
        c2c_mfma2048_kernel<FWD, kPf><<<g.blocks, 256, 0, stream>>>(x, y, batch, tw,
                                                                    g.tiles_per_block);
    else
        c2c_mfma4096_kernel<FWD, kPf><<<g.blocks, 256, 0, stream>>>(x, y, batch, tw,
                                                                    g.tiles_per_block);
}

// Buffers that are element-aligned but not 16-byte aligned (any vec2_t<T>
// pointer, the reference's contract): the VALU kernel with direct movement
// (DirectIO, fft_tile.hpp), whose accesses are one element each, one tile
// per workgroup.
template <class IO, int N>
void enqueue_unaligned(bool forward, const IO* x, IO* y, int batch, const float2* tw,
                       hipStream_t stream) {
    const unsigned blocks =
        static_cast<unsigned>((static_cast<long long>(batch) + C2CPlan<N>::kFPB - 1) /
                              C2CPlan<N>::kFPB);
    if (forward)
        c2c_kernel<IO, N, true, false, true><<<blocks, 256, 0, stream>>>(x, y, batch, tw, 1);
    else
        c2c_kernel<IO, N, false, false, true><<<blocks, 256, 0, stream>>>(x, y, batch, tw, 1);
}

template <int N>
hipError_t launch_c2c(int precision, bool forward, bool aligned16, const void* in, void* out,
                      int batch, const float2* tw, int num_cus, hipStream_t stream) {
    if (!aligned16) {
        if (precision == 0)
            enqueue_unaligned<float2, N>(forward, static_cast<const float2*>(in),
                                         static_cast<float2*>(out), batch, tw, stream);
        else
            enqueue_unaligned<__half2, N>(forward, static_cast<const __half2*>(in),
                                          static_cast<__half2*>(out), batch, tw, stream);
        return hipGetLastError();
    }
    const bool mfma = precision != 0 && kHalfOnMfma<N>;
    long long fpb = C2CPlan<N>::kFPB;  // 2 for N = 2048 and 1 for N = 4096 on either kernel
    if constexpr (kHalfOnMfma<N>)
        if (mfma) fpb = MfmaPlan<N / 256>::kFPB;
    const long long ntiles = (static_cast<long long>(batch) + fpb - 1) / fpb;
    const Grid g = make_grid(ntiles, launch_shape<N>(precision).per_cu, num_cus);
    if (precision == 0) {
        const auto* x = static_cast<const float2*>(in);
        auto* y = static_cast<float2*>(out);
        if (forward)
            enqueue<float2, N, true>(g, x, y, batch, tw, stream);
        else
            enqueue<float2, N, false>(g, x, y, batch, tw, stream);
    } else {
        const auto* x = static_cast<const __half2*>(in);
        auto* y = static_cast<__half2*>(out);
        if constexpr (kHalfOnMfma<N>) {
            if (forward)
                enqueue_mfma<N, true>(g, x, y, batch, tw, stream);
            else
                enqueue_mfma<N, false>(g, x, y, batch, tw, stream);
        } else if constexpr (kHalfOnMfma3<N>) {
            if (forward)
                enqueue_mfma3<N, true>(g, x, y, batch, tw, stream);
            else
                enqueue_mfma3<N, false>(g, x, y, batch, tw, stream);
        } else if constexpr (kHalfOnMfma128<N>) {
            if (forward)
                enqueue_mfma128<true>(g, x, y, batch, tw, stream);
            else
                enqueue_mfma128<false>(g, x, y, batch, tw, stream);
        } else if (forward) {
            enqueue<__half2, N, true>(g, x, y, batch, tw, stream);
        } else {
            enqueue<__half2, N, false>(g, x, y, batch, tw, stream);
        }
    }
    return hipGetLastError();
}

// Launch shapes of the VALU convolutions (conv1d_kernel, conv1d_real_kernel):
// workgroups per CU (make_grid; 0 = one tile per workgroup) and next-tile
// prefetch.  Measured on MI355X (complex: 2^25 values per array; real: 2^26
// samples, 64 channels):
//   complex fp32, per-signal filters: one tile per workgroup up to N = 1024
//     (127-144 us against 134-181 us for device grids, prefetch 138-152);
//     N = 2048 3 per CU (160 us; 2 tiles per workgroup 172, prefetch 163);
//     N = 4096 2 per CU (167 us; prefetch 192).
//   complex fp32, shared filter (transformed once per workgroup): one tile
//     per workgroup up to N = 256 (92-96 us, equal to prefetch); N = 512 2
//     per CU with early prefetch (101 us, one tile per workgroup 122);
//     N = 1024, 2048 3 per CU (102 and 107 us; one tile per workgroup 127);
//     N = 4096 2 per CU with early prefetch (113 us against 121).
//   real fp32: 2 per CU with prefetch, late up to N = 512 and early above:
//     97-116 us for N = 64 ... 512 (one tile per workgroup 110-153) and
//     112/121/115 us for N = 1024/2048/4096 (168-176 without prefetch).
//   fp16 on VALU (N = 64, 128 only): real 4 per CU (62-64 us; prefetch
//     62-74), complex 16 per CU (conv1d 78-87 us against 85-91).
struct ConvShape {
    int per_cu;
    Prefetch prefetch;
};

template <int N>
constexpr ConvShape valu_conv_shape(int precision, bool real, bool per_signal) {
    if (precision != 0) return {real ? 4 : 16, Prefetch::kNone};
    if (real) return {2, N <= 512 ? Prefetch::kLate : Prefetch::kEarly};
    if (per_signal) return {N <= 1024 ? 0 : N == 2048 ? 3 : 2, Prefetch::kNone};
    if (N <= 256) return {0, Prefetch::kNone};
    if (N == 512 || N == 4096) return {2, Prefetch::kEarly};
    return {3, Prefetch::kNone};
}

template <class IO, int N>
void enqueue_conv1d(bool per_signal, Grid g, Prefetch pf, const IO* x, const IO* h, IO* y,
                    int batch, const float2* tw, hipStream_t stream) {
    if (per_signal)
        conv1d_kernel<IO, N, true, Prefetch::kNone, (N >= 256)><<<g.blocks, 256, 0, stream>>>(
            x, h, y, batch, tw, g.tiles_per_block);
    else if (pf == Prefetch::kEarly)
        conv1d_kernel<IO, N, false, Prefetch::kEarly><<<g.blocks, 256, 0, stream>>>(
            x, h, y, batch, tw, g.tiles_per_block);
    else
        conv1d_kernel<IO, N, false><<<g.blocks, 256, 0, stream>>>(x, h, y, batch, tw,
                                                                  g.tiles_per_block);
}

template <int N>
hipError_t launch_conv1d(int precision, bool per_signal_filter, const void* x, const void* h,
                         void* y, int batch, const float2* tw, int num_cus, hipStream_t stream) {
    // fp16 N = 256 ... 2048: all three transforms on MFMA (fft_conv_mfma.hpp);
    // per-signal filters, 2^25 values, against the VALU path on MI355X:
    // 77 vs 90 us (N=256), 83 vs 116 (512), 91 vs 122 (1024), 107 vs 138 (2048).
    // Grid: the occupancy, 3 workgroups per CU (2 for N = 2048), 6% faster
    // than 4 tiles per workgroup.
    if constexpr (N >= 256 && N <= 2048) {
        if (precision != 0) {
            constexpr int C = N / 256;
            using M = MfmaPlan<C>;
            const long long ntiles = (static_cast<long long>(batch) + M::kFPB - 1) / M::kFPB;
            const Grid g = make_grid(ntiles, C == 8 ? 2 : 3, num_cus);
            const auto* xx = static_cast<const __half2*>(x);
            const auto* hh = static_cast<const __half2*>(h);
            auto* yy = static_cast<__half2*>(y);
            if (per_signal_filter)
                conv1d_mfma_kernel<C, true><<<g.blocks, 256, 0, stream>>>(xx, hh, yy, batch, tw,
                                                                          g.tiles_per_block);
            else
                conv1d_mfma_kernel<C, false><<<g.blocks, 256, 0, stream>>>(xx, hh, yy, batch, tw,
                                                                           g.tiles_per_block);
            return hipGetLastError();
        }
    }
    // fp16 N = 4096: the three-stage MFMA transform, one signal per tile, the
    // grid at the kernel's occupancy (per-signal filters: 3 workgroups per CU;
    // a shared filter keeps its spectrum live across the loop, 2 per CU).
    // 2^25 values on MI355X: 103 vs 162 us per-signal, 76 vs 125 us shared,
    // against the VALU path.
    if constexpr (N == 4096) {
        if (precision != 0) {
            const Grid g = make_grid(batch, per_signal_filter ? 3 : 2, num_cus);
            const auto* xx = static_cast<const __half2*>(x);
            const auto* hh = static_cast<const __half2*>(h);
            auto* yy = static_cast<__half2*>(y);
            if (per_signal_filter)
                conv1d_mfma4096_kernel<N, true><<<g.blocks, 256, 0, stream>>>(xx, hh, yy, batch, tw);
            else
                conv1d_mfma4096_kernel<N, false><<<g.blocks, 256, 0, stream>>>(xx, hh, yy, batch,
                                                                               tw);
            return hipGetLastError();
        }
    }
    using P = C2CPlan<N>;
    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    const ConvShape shape = valu_conv_shape<N>(precision, false, per_signal_filter);
    const Grid g = make_grid(ntiles, shape.per_cu, num_cus);
    if (precision == 0)
        enqueue_conv1d<float2, N>(per_signal_filter, g, shape.prefetch,
                                  static_cast<const float2*>(x), static_cast<const float2*>(h),
                                  static_cast<float2*>(y), batch, tw, stream);
    else if constexpr (N < 256)  // fp16 N >= 256 returned above (MFMA)
        enqueue_conv1d<__half2, N>(per_signal_filter, g, Prefetch::kNone,
                                   static_cast<const __half2*>(x), static_cast<const __half2*>(h),
                                   static_cast<__half2*>(y), batch, tw, stream);
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
    // fp16 N = 256 ... 2048: both transforms on MFMA (fft_conv_mfma.hpp);
    // measured against this VALU path at 2^26 samples: 61 vs 68 us (N=256),
    // 60 vs 87 (512), 64 vs 87 (1024).  Grid: the occupancy (2 workgroups per
    // CU for N = 256 and 2048, else 3); up to N = 1024 the channels' spectra
    // stay in registers (5-9% over reloading them per tile).
    if constexpr (N >= 256 && N <= 2048) {
        if (precision != 0) {
            using M = MfmaPlan<N / 256>;
            const long long ntiles = (transforms + M::kFPB - 1) / M::kFPB;
            const Grid g = make_grid(ntiles, N == 256 || N == 2048 ? 2 : 3, num_cus);
            if (real_buffer_fits<N / 256>(channels))
                conv1d_real_mfma_kernel<N / 256, true><<<g.blocks, 256, 0, stream>>>(
                    static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch,
                    channels, tw, g.tiles_per_block);
            else
                conv1d_real_mfma_kernel<N / 256, false><<<g.blocks, 256, 0, stream>>>(
                    static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch,
                    channels, tw, g.tiles_per_block);
            return hipGetLastError();
        }
    }
    // fp16 N = 4096: the three-stage MFMA transform, both directions; 2
    // workgroups per CU: 77 us against 87-84 us for 3 or 4 (2^26 samples);
    // the channel's spectrum stays in registers (84 us reloading it per tile).
    if constexpr (N == 4096) {
        if (precision != 0) {
            const Grid g = make_grid(transforms, 2, num_cus);
            if (channels <= kReal4096BufferMaxChannels)
                conv1d_real_mfma4096_kernel<N, true><<<g.blocks, 256, 0, stream>>>(
                    static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch,
                    channels, tw, g.tiles_per_block);
            else
                conv1d_real_mfma4096_kernel<N, false><<<g.blocks, 256, 0, stream>>>(
                    static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch,
                    channels, tw, g.tiles_per_block);
            return hipGetLastError();
        }
    }
    const long long ntiles = (transforms + P::kFPB - 1) / P::kFPB;
    const ConvShape shape = valu_conv_shape<N>(precision, true, false);
    const Grid g = make_grid(ntiles, shape.per_cu, num_cus);
    constexpr Prefetch kF32 = valu_conv_shape<N>(0, true, false).prefetch;
    // fp32 N >= 2048 moves samples straight between HBM and registers
    // (conv1d_real_kernel's kDirect): N = 4096 108-114 us against 115-117,
    // 2048 115-119 against 120-123; at N = 1024 it measured slower (125 vs 113).
    if (precision == 0)
        conv1d_real_kernel<float2, N, kF32, (N >= 2048)><<<g.blocks, 256, 0, stream>>>(
            static_cast<const float*>(x), spectrum, static_cast<float*>(y), batch, channels, tw,
            g.tiles_per_block);
    else if constexpr (N < 256)  // fp16 N >= 256 returned above (MFMA)
        conv1d_real_kernel<__half2, N><<<g.blocks, 256, 0, stream>>>(
            static_cast<const __half*>(x), spectrum, static_cast<__half*>(y), batch, channels, tw,
            g.tiles_per_block);
    return hipGetLastError();
}

#if THFF_N == 64
hipError_t launch_conv1d_valid(int precision, const void* x, long long len, const float2* taps,
                               int ntaps, void* y, int batch, const float2* tw, int num_cus,
                               hipStream_t stream) {
    // fp32: a group is the 64 windows (one per transform slot) of one
    // workgroup pass; each workgroup transforms the filter once and walks
    // many groups, 2 workgroups per CU (the occupancy, with its span
    // prefetch).  2^26 values, 9 taps: 232 us, against 294 us for runs of 4
    // groups.
    // half2: 256-point windows on MFMA (conv1d_valid_mfma_kernel), 16 windows
    // per workgroup tile, a device grid of 4 workgroups per CU.
    if (precision != 0) {
        const long long valid = 257 - ntaps;
        const long long windows = (len - ntaps + 1 + valid - 1) / valid;
        const long long groups = (windows + 15) / 16 * batch;
        const Grid g = make_grid(groups, 4, num_cus);
        conv1d_valid_mfma_kernel<256><<<g.blocks, 256, 0, stream>>>(
            static_cast<const __half2*>(x), taps, static_cast<__half2*>(y), len, ntaps, batch,
            g.tiles_per_block);
        return hipGetLastError();
    }
    const long long valid = 65 - ntaps;
    const long long windows = (len - ntaps + 1 + valid - 1) / valid;
    const long long groups = (windows + 63) / 64 * batch;
    const Grid g = make_grid(groups, 2, num_cus);
    conv1d_valid_kernel<float2><<<g.blocks, 256, 0, stream>>>(
        static_cast<const float2*>(x), taps, static_cast<float2*>(y), len, ntaps, batch, tw,
        g.tiles_per_block);
    return hipGetLastError();
}

hipError_t launch_conv2d64(int precision, const void* x, const void* h, void* y, int batch,
                           const float2* tw, int num_cus, hipStream_t stream) {
    // One image per tile; a device grid at the kernel's occupancy walks the
    // images grid-stride, and each workgroup transforms the filter once.
    // fp32: the VALU kernel, 4 workgroups per CU.  fp16: the MFMA kernel
    // (conv2d64_mfma_kernel), kConv2dMfmaPerCu per CU.
    if (precision == 0) {
        const Grid g = make_grid(batch, 4, num_cus);
        conv2d64_kernel<float2><<<g.blocks, 256, 0, stream>>>(
            static_cast<const float2*>(x), static_cast<const float2*>(h), static_cast<float2*>(y),
            batch, tw, g.tiles_per_block);
    } else {
        constexpr int kConv2dMfmaPerCu = 3;
        const Grid g = make_grid(batch, kConv2dMfmaPerCu, num_cus);
        conv2d64_mfma_kernel<kConv2dMfmaPerCu><<<g.blocks, 256, 0, stream>>>(
            static_cast<const __half2*>(x), static_cast<const __half2*>(h),
            static_cast<__half2*>(y), batch, tw, g.tiles_per_block);
    }
    return hipGetLastError();
}
#endif

#if THFF_N == 128
hipError_t launch_conv2d128(int precision, const void* x, const void* h, void* y, int batch,
                            const float2* tw, int num_cus, hipStream_t stream) {
    // One image per workgroup: fp32 on VALU (conv2d128_lanes_kernel: 1024
    // lanes, a 129 KiB exchange buffer), fp16 on MFMA (conv2d128_mfma_kernel:
    // 512 lanes, 146 KiB of LDS); one workgroup per CU either way, so a device
    // grid of one per CU walks the images grid-stride.
    const Grid g = make_grid(batch, 1, num_cus);
    if (precision == 0)
        conv2d128_lanes_kernel<><<<g.blocks, 1024, 0, stream>>>(
            static_cast<const float2*>(x), static_cast<const float2*>(h), static_cast<float2*>(y),
            batch, tw);
    else
        conv2d128_mfma_kernel<1><<<g.blocks, 512, 0, stream>>>(
            static_cast<const __half2*>(x), static_cast<const __half2*>(h),
            static_cast<__half2*>(y), batch, tw, g.tiles_per_block);
    return hipGetLastError();
}
#endif

#if THFF_N == 1024
hipError_t launch_conv2d_cols(int precision, bool conv, const void* in, void* out,
                              const float2* H, int cols, long long images, float scale,
                              const float2* tw, int num_cus, hipStream_t stream) {
    if (cols != 1024) return hipErrorInvalidValue;  // the kernels are built for 1024 columns
    // kCols columns per unit (one wave per column for fp32, two per wave for
    // half); workgroups walk the units grid-stride, and the grid is a multiple
    // of the image's column blocks, so every workgroup keeps one column block
    // (and its H columns).  The unit's rows move as 16-byte pieces, 64 bytes
    // of each row (fp32: 8 columns; half: 16), through one 512-lane workgroup
    // per CU.  Measured on MI355X, 32 images of 1024 x 1024 end to end: fp32
    // 8 columns with the next block prefetched 359 us (16 columns, two per
    // wave, no prefetch: 358 us, 124 bytes of spill); half 16 columns 253 us
    // against 277 us with 8 columns (32-byte pieces: a wave's loads then touch
    // twice the rows); one column per wave on MFMA with 16-byte pieces (4
    // columns per 256-lane workgroup) 545 us.  A pass over fewer units than
    // two per CU (one or a few images, and the filter's column pass of every
    // call) runs 4-column units instead, 256-lane workgroups of one column
    // per wave, so that more CUs share the columns: one image end to end
    // (filter spectrum included) fp16 43.5 against 60.8 us, fp32 48.6 against
    // 52.4 us (2-column fp32 units: 57.5 us); 32 images fp16 248.5 against
    // 253.1 us (the filter's pass).
    auto launch = [&](auto cols_tag, const void* src, void* dst) {
        constexpr int kCols = decltype(cols_tag)::value;
        constexpr int kPerCu = kColsWavesPerEU<kCols> * 4 / (kColsLanes<kCols> / 64);
        const long long blocks_per_image = cols / kCols;
        const long long units = blocks_per_image * images;
        long long grid = static_cast<long long>(kPerCu) * (num_cus > 0 ? num_cus : 256);
        if (grid >= blocks_per_image) grid -= grid % blocks_per_image;
        const dim3 blocks(static_cast<unsigned>(units < grid ? units : grid));
        const dim3 lanes(kColsLanes<kCols>);
        if (precision == 0) {
            if (conv)
                conv2d_cols_kernel<float2, float2, 1024, 1024, true, kCols><<<blocks, lanes, 0, stream>>>(
                    static_cast<const float2*>(src), static_cast<float2*>(dst), H, units, scale, tw);
            else
                conv2d_cols_kernel<float2, float2, 1024, 1024, false, kCols><<<blocks, lanes, 0, stream>>>(
                    static_cast<const float2*>(src), static_cast<float2*>(dst), H, units, scale, tw);
        } else {
            if (conv)
                conv2d_cols_kernel<__half2, __half2, 1024, 1024, true, kCols><<<blocks, lanes, 0, stream>>>(
                    static_cast<const __half2*>(src), static_cast<__half2*>(dst), H, units, scale, tw);
            else
                conv2d_cols_kernel<__half2, float2, 1024, 1024, false, kCols><<<blocks, lanes, 0, stream>>>(
                    static_cast<const __half2*>(src), static_cast<float2*>(dst), H, units, scale, tw);
        }
    };
    const long long wide = precision == 0 ? 8 : 16;
    const long long cus = num_cus > 0 ? num_cus : 256;
    if (images * (cols / wide) < 2LL * cus) {
        launch(std::integral_constant<int, 4>{}, in, out);
    } else if (precision != 0 && conv) {
        // half2 with the product: 16 columns per unit on MFMA, one 512-lane
        // workgroup per CU (conv2d_cols_mfma_kernel): 32 images end to end
        // 214.8 against 249.7 us with the VALU pass below.
        const long long units = images * (cols / 16);
        long long grid = cus;
        if (grid >= cols / 16) grid -= grid % (cols / 16);
        conv2d_cols_mfma_kernel<><<<static_cast<unsigned>(units < grid ? units : grid), 512, 0, stream>>>(
            static_cast<const __half2*>(in), static_cast<__half2*>(out), H, units, tw);
    } else if (precision == 0)
        launch(std::integral_constant<int, 8>{}, in, out);
    else
        launch(std::integral_constant<int, 16>{}, in, out);
    return hipGetLastError();
}
#endif

template hipError_t launch_c2c<THFF_N>(int, bool, bool, const void*, void*, int, const float2*,
                                       int, hipStream_t);
template hipError_t launch_conv1d<THFF_N>(int, bool, const void*, const void*, void*, int,
                                          const float2*, int, hipStream_t);
template hipError_t launch_conv1d_real_filter<THFF_N>(const float*, float2*, int, float,
                                                      const float2*, hipStream_t);
template hipError_t launch_conv1d_real<THFF_N>(int, const void*, const float2*, void*, int, int,
                                               const float2*, int, hipStream_t);

}  // namespace thff
