// fft_conv_mfma.hpp -- fused half2 convolutions with the radix-16 stages on
// MFMA (v_mfma_f32_16x16x32_f16), for N = 256*C, C in {1, 2, 4}.
//
// The forward transform (fft_mfma.hpp: stage 1 from LDS, twiddles, DFT_C,
// LDS transpose, stage 2) leaves lane (n, q) of block b = (f, m) holding
// Z_f[n + 16 m + 16C (q + 4 r)], r = 0..3.  Read as inputs of the inverse,
// those are sequence t = 16 m + n (lane n, block m: where the inverse's
// stage 1 wants it) at inputs j = q + 4 r: the inverse's stage 1 consumes the
// product straight from registers with column-permuted operands
// (dft16_operands<..., true>), so the spectra never leave registers.
//
// Every transform here runs forward: the inverse of a product P is computed
// as conj(DFT(conj(P))), with the conjugation folded into the f16 packing on
// the way into the inverse's stage 1 and on the way out.  So one set of
// operands and twiddles serves all three transforms, and the W_16C^(n m)
// twiddle before the last DFT16 is folded into that stage's operands
// (Stage3Folded, fft_mfma.hpp).
#pragma once

#include "fft_conv.hpp"
#include "fft_mfma.hpp"

namespace thff {

// Two dwords of half values -> one: {s1.lo, s0.lo} (kHalvesLow) or {s1.hi,
// s0.hi} (kHalvesHigh), one v_perm_b32 (selector bytes 0-3 pick bytes of s1,
// 4-7 bytes of s0) instead of a mask, a shift and an or.
inline constexpr unsigned kHalvesLow = 0x05040100u, kHalvesHigh = 0x07060302u;
__device__ __forceinline__ unsigned halves(unsigned s0, unsigned s1, unsigned sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

// Two rows of halves (8 per 16-byte word) <-> 8 half2 (row 0 = real part).
__device__ __forceinline__ void interleave_rows(u32x4 r0, u32x4 r1, u32x4& lo, u32x4& hi) {
    const unsigned a[4] = {r0.x, r0.y, r0.z, r0.w}, b[4] = {r1.x, r1.y, r1.z, r1.w};
    unsigned z[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        z[2 * i] = halves(b[i], a[i], kHalvesLow);
        z[2 * i + 1] = halves(b[i], a[i], kHalvesHigh);
    }
    lo = u32x4{z[0], z[1], z[2], z[3]};
    hi = u32x4{z[4], z[5], z[6], z[7]};
}
__device__ __forceinline__ void split_rows(u32x4 lo, u32x4 hi, u32x4& r0, u32x4& r1) {
    const unsigned z[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    unsigned a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = halves(z[2 * i + 1], z[2 * i], kHalvesLow);
        b[i] = halves(z[2 * i + 1], z[2 * i], kHalvesHigh);
    }
    r0 = u32x4{a[0], a[1], a[2], a[3]};
    r1 = u32x4{b[0], b[1], b[2], b[3]};
}

// Real-input fused convolution (conv1d_real_kernel's contract, fp16 storage)
// on MFMA: complex transform tau = p * D + d carries rows (2p, d) and
// (2p + 1, d) as real and imaginary parts; a wave owns kFPW = 4/C transforms
// (1024 complex values) for C <= 4 and one of 2048 for C = 8, a tile is 4
// waves.  Lane l moves 8 values of both rows per 16-byte step: values
// e = 8 l + 512 i (i < kSteps) of the wave.  For C <= 4 the spectra of a
// wave's transforms are kept in fp32 registers across tiles (reloaded when
// the channels change), which holds C = 1 (four transforms per wave, each
// with its own channel) to 2 waves per SIMD and the others to 3.  At C = 8
// the transform's 32 values per lane leave no registers for them: the
// product reads the channel's spectrum (fp32, L2-resident) per tile.
template <int C>
inline constexpr int kConvMfmaMinWavesPerEU = C == 1 || C == 8 ? 2 : 3;
// At C = 8 (N = 2048) the DFT8 between the two DFT16 stages of the complex
// fp16 convolution runs on the matrix cores (mfma8_steps2to6_dft8mfma)
// instead of in-lane: 81.5-82.8 against 84.3-86.8 us for 16384 x 2048
// per-signal filters, 59.5-60.9 against 62.1-64.3 us with a shared filter,
// rel L2 against fp64 6.55e-4 against 5.71e-4 (one more f16 rounding,
// MI355X).  The real convolution at N = 2048 keeps the in-lane DFT8: on the
// matrix cores it measured 68.5-69.6 against 67.6-69.1 us, with more error.
inline constexpr bool kConv1dDft8OnMfma = true;

// kBufferIO addressing of conv1d_real_mfma_kernel.  A wave's transforms tau0
// ... tau0 + kFPW - 1 (pairs p, channels d, consecutive in tau) read and
// write rows (2p, d) and (2p + 1, d); one resource per wave and tile starts
// at row 0 of tau0 and runs to the end of the [batch][channels][N] array.
// Rows are laid out in increasing (p, d) order, so every row of those
// transforms lies at or after that start, and a row that does not exist --
// row 1 of the last pair of an odd batch, or any row of a transform past the
// last -- lies past the end of the array, where the range check reads zeros
// and drops stores.  Byte offsets from the start stay below
// (2 channels + 2 kFPW) N * 2, which kBufferIO requires to fit in 31 bits.
__host__ __device__ __forceinline__ long long real_row(long long p, int d, int r, int channels,
                                                       int n) {
    return ((2 * p + r) * static_cast<long long>(channels) + d) * n;
}
struct RealWaveSpan {
    long long start;  // element offset of row 0 of the wave's first transform
    int bytes;        // from there to the end of the array (0 when past it)
    __host__ __device__ static RealWaveSpan at(ChannelPos first, int channels, int batch, int n) {
        const long long start = real_row(first.p, first.d, 0, channels, n);
        const long long total = static_cast<long long>(batch) * channels * n;
        const long long left = total > start ? total - start : 0;
        const long long cap = 0x7ffffff0LL / 2;
        return {start, static_cast<int>(2 * (left < cap ? left : cap))};
    }
};
template <int C>
inline constexpr int kRealWaveTransforms = 4 / C > 1 ? 4 / C : 1;
template <int C>
__host__ __device__ __forceinline__ bool real_buffer_fits(int channels) {
    return (2LL * channels + 2 * kRealWaveTransforms<C>) * (256LL * C) * 2 < 0x7ffffff0LL;
}

template <int C, bool kBufferIO = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kConvMfmaMinWavesPerEU<C>))) void
conv1d_real_mfma_kernel(const __half* __restrict__ x, const float2* __restrict__ spectrum,
                        __half* __restrict__ y, int batch, int channels,
                        const float2* __restrict__ tw, int tiles_per_block) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    constexpr int kB = P::kBlocks;
    constexpr int kSteps = P::kWaveVals / 512;  // 16-byte steps of 8 values per lane
    constexpr bool kKeepSpectra = C <= 4;
    __shared__ unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    __shared__ u32x4 a3[P::kA3];
    const int tid = threadIdx.x;
    // uniform over the wave: a scalar, so the per-wave resources stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;

    f16x8 a[2], a_regs[2];
    mfma_setup<C, true>(a, w1, a3, nullptr, tw);  // forward operands and twiddles
    dft16_operands<true, true>(a_regs, lane);
    const Stage3Folded s3{a, a3, lane};

    const long long pairs = (static_cast<long long>(batch) + 1) / 2;
    const long long transforms = pairs * channels;
    const long long ntiles = (transforms + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
    int spec_d = -1;  // chan[0] of the spectra spec holds
    cpx spec[kKeepSpectra ? kB : 1][4];
    // Pair and channel of the wave's first transform, advanced per tile.
    const ChannelWalk walk(step * P::kFPB, channels);
    ChannelPos pos = walk.at(tile * P::kFPB + wave * P::kFPW);

    // At N = 2048 (one transform per wave) a wave's issue priority falls as
    // its workgroup gets ahead of the others: 70 against 72-73 us at 2^26
    // samples; neutral at N <= 1024.
    long long left = (tile_end - tile + step - 1) / step;
    const ProgressPriority priority(left);
    for (; tile < tile_end; tile += step, --left) {
        if constexpr (C == 8) priority.set(left);
        // Rows of this wave's transforms, as element offsets (-1: none).
        long long base0[kSteps], base1[kSteps];
        int chan[P::kFPW];
#pragma unroll
        for (int i = 0; i < kSteps; ++i) {
            const int e = 8 * lane + 512 * i;
            const long long tau = tile * P::kFPB + wave * P::kFPW + e / N;
            long long p;
            int d;
            walk.locate(pos, e / N, p, d);
            const int k = e % N;
            base0[i] = tau < transforms ? (2 * p * channels + d) * N + k : -1;
            base1[i] = tau < transforms && 2 * p + 1 < batch ? ((2 * p + 1) * channels + d) * N + k
                                                             : -1;
        }
        // (past the last transform too: a channel is always a valid spectrum row)
#pragma unroll
        for (int f = 0; f < P::kFPW; ++f) {
            long long p;
            walk.locate(pos, f, p, chan[f]);
        }
        // kBufferIO: byte offsets of both rows from the wave's resource start,
        // whether the rows exist or not (see RealWaveSpan).
        [[maybe_unused]] int off0[kSteps], off1[kSteps];
        [[maybe_unused]] RealWaveSpan span;
        if constexpr (kBufferIO) {
            span = RealWaveSpan::at(pos, channels, batch, N);
#pragma unroll
            for (int i = 0; i < kSteps; ++i) {
                const int e = 8 * lane + 512 * i;
                long long p;
                int d;
                walk.locate(pos, e / N, p, d);
                off0[i] = static_cast<int>(2 * (real_row(p, d, 0, channels, N) + e % N - span.start));
                off1[i] = static_cast<int>(2 * (real_row(p, d, 1, channels, N) + e % N - span.start));
            }
        }
        pos = walk.advance(pos);
        u32x4 r0[kSteps], r1[kSteps];
        if constexpr (kBufferIO) {
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<__half*>(x + span.start), 0, span.bytes, 0x00020000);
#pragma unroll
            for (int i = 0; i < kSteps; ++i) {
                r0[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off0[i], 0, 2);
                r1[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off1[i], 0, 2);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kSteps; ++i) {
                r0[i] = base0[i] >= 0 ? ld_nt(reinterpret_cast<const u32x4*>(x + base0[i])) : u32x4{};
                r1[i] = base1[i] >= 0 ? ld_nt(reinterpret_cast<const u32x4*>(x + base1[i])) : u32x4{};
            }
        }
        wave_lds_sync();  // the previous tile's output reads are done
#pragma unroll
        for (int i = 0; i < kSteps; ++i) {
            const int e = 8 * lane + 512 * i;
            u32x4 lo, hi;
            interleave_rows(r0[i], r1[i], lo, hi);
            *reinterpret_cast<u32x4*>(region + P::in_pad(e)) = lo;
            *reinterpret_cast<u32x4*>(region + P::in_pad(e + 4)) = hi;
        }
        wave_lds_sync();

        cpx v[kB][4];
        mfma_stage1_lds<C>(region, a, lane, v);
        mfma_steps2to6<C, true>(region, w1, s3, lane, v);
        // ---- product: block (f, m), lane (n, q): bin k = n + 16 m + 16C (q + 4 r) ----
        // The spectra of the wave's transforms stay in registers while their
        // channels do not change: they are chan[0] + f mod D, so chan[0]
        // decides, and on a grid-stride walk whose stride in transforms is a
        // multiple of D it never changes.
        if constexpr (kKeepSpectra) {
            if (chan[0] != spec_d) {
#pragma unroll
                for (int b = 0; b < kB; ++b) {
                    const float2* hs = spectrum + static_cast<long long>(chan[b / C]) * N + n +
                                       16 * (b % C) + P::kM * q;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float2 hk = hs[P::kM * 4 * r];
                        spec[b][r] = cpx{hk.x, hk.y};
                    }
                }
                spec_d = chan[0];
            }
#pragma unroll
            for (int b = 0; b < kB; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[b][r] = cmul(v[b][r], spec[b][r]);
        } else {
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const float2* hs = spectrum + static_cast<long long>(chan[b / C]) * N + n +
                                   16 * (b % C) + P::kM * q;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float2 hk = hs[P::kM * 4 * r];
                    v[b][r] = cmul(v[b][r], cpx{hk.x, hk.y});
                }
            }
        }
        // ---- inverse = conj(DFT(conj(product))), stage 1 straight from the registers ----
        mfma_stage1_regs<C, true>(a_regs, v);
        mfma_steps2to6<C, true>(region, w1, s3, lane, v);
        // ---- real part -> row 2p, imaginary part -> row 2p + 1 (conjugated back) ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < kB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::out_pad((b / C) * N + n + 16 * (b % C) + P::kM * (q + 4 * r))] =
                    pack_half2({v[b][r].re, -v[b][r].im});
        wave_lds_sync();
        [[maybe_unused]] __amdgpu_buffer_rsrc_t ys;
        if constexpr (kBufferIO)
            ys = __builtin_amdgcn_make_buffer_rsrc(y + span.start, 0, span.bytes, 0x00020000);
#pragma unroll
        for (int i = 0; i < kSteps; ++i) {
            const int e = 8 * lane + 512 * i;
            const u32x4 lo = *reinterpret_cast<const u32x4*>(region + P::out_pad(e));
            const u32x4 hi = *reinterpret_cast<const u32x4*>(region + P::out_pad(e + 4));
            u32x4 o0, o1;
            split_rows(lo, hi, o0, o1);
            if constexpr (kBufferIO) {
                __builtin_amdgcn_raw_buffer_store_b128(o0, ys, off0[i], 0, 2);
                __builtin_amdgcn_raw_buffer_store_b128(o1, ys, off1[i], 0, 2);
            } else {
                if (base0[i] >= 0) st_nt(reinterpret_cast<u32x4*>(y + base0[i]), o0);
                if (base1[i] >= 0) st_nt(reinterpret_cast<u32x4*>(y + base1[i]), o1);
            }
        }
    }
}

}  // namespace thff

namespace thff {

// Complex fused convolution (conv1d_kernel's contract, half2 storage) on
// MFMA: y[b] = IFFT(FFT(x[b]) * FFT(h[b or 0])) / N.  A wave owns kFPW
// transforms (1024 values for C <= 4, one transform of 2048 for C = 8); the
// filter spectrum is kept packed as half2 between the transforms.
template <int C>
inline constexpr int kConv1dMfmaMinWavesPerEU = C <= 4 ? 3 : 2;

template <int C, bool kPerSignal>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kConv1dMfmaMinWavesPerEU<C>))) void
conv1d_mfma_kernel(const __half2* __restrict__ x, const __half2* __restrict__ h,
                   __half2* __restrict__ y, int batch, const float2* __restrict__ tw,
                   int tiles_per_block) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    constexpr int kB = P::kBlocks;
    constexpr int kRaw = P::kVals / 4;  // 16-byte loads per lane
    __shared__ unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    __shared__ u32x4 a3[P::kA3];
    const int tid = threadIdx.x;
    // The wave index is uniform over the wave: read into a scalar, so that
    // the per-wave buffer resources below stay in scalar registers.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;

    f16x8 a[2], a_regs[2];
    mfma_setup<C, true>(a, w1, a3, nullptr, tw);
    // The inverse's stage-1 operands carry the 1/N of the convolution: a
    // power of two, exact in f16 for every coefficient here (|c| >= 0.38).
    dft16_operands<true, true>(a_regs, lane);
#pragma unroll
    for (int h = 0; h < 2; ++h) a_regs[h] *= static_cast<_Float16>(1.0f / N);
    const Stage3Folded s3{a, a3, lane};
    // Steps 2-6 of a transform; at C = 8 the DFT8 runs on the matrix cores.
    [[maybe_unused]] const f16x4 a8 = dft8_mfma_operand(lane);
    auto steps = [&](cpx (&v)[kB][4]) {
        if constexpr (C == 8 && kConv1dDft8OnMfma)
            mfma8_steps2to6_dft8mfma(
                region, [&](int c, int r) { return w1[(c * 4 + r) * 64 + lane]; }, s3, a8, lane, v);
        else
            mfma_steps2to6<C, true>(region, w1, s3, lane, v);
    };

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);

    // Valid values (0..kWaveVals) of this wave's transforms in tile tl.
    auto valid = [&](long long tl) {
        const long long v = (static_cast<long long>(batch) - tl * P::kFPB - wave * P::kFPW) * N;
        return v <= 0 ? 0 : (v >= P::kWaveVals ? P::kWaveVals : static_cast<int>(v));
    };
    // This wave's kWaveVals values of `src` (nv of them valid), 16-byte loads
    // through a buffer resource of the nv valid values: pieces past them read
    // zeros by the hardware's range check, so every load is issued with no
    // branch and the compiler waits for exactly the pieces it uses (with a
    // guard per piece it waited for every outstanding access, the previous
    // tile's stores included).  nv = 0 issues loads that touch no memory.
    auto load = [&](const __half2* src, int nv, u32x4 (&raw)[kRaw]) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<__half2*>(src), 0, 4 * nv, 0x00020000);
#pragma unroll
        for (int i = 0; i < kRaw; ++i) raw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * lane, 1024 * i, 2);
    };
    // Stage loaded values in the wave's region; transform what is staged.
    auto stage = [&](const u32x4 (&raw)[kRaw]) {
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < kRaw; ++i)
            *reinterpret_cast<u32x4*>(region + P::in_pad(4 * lane) + P::kInStep * i) = raw[i];
        wave_lds_sync();
    };
    auto forward = [&](cpx (&v)[kB][4]) {
        mfma_stage1_lds<C>(region, a, lane, v);
        steps(v);
    };

    unsigned hp[kB][4];  // FFT(h), packed half2
    auto keep = [&](const cpx (&v)[kB][4]) {
#pragma unroll
        for (int b = 0; b < kB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) hp[b][r] = pack_half2(v[b][r]);
    };
    if constexpr (!kPerSignal) {
        // Every transform of the wave is the shared filter: stage it kFPW times.
        cpx v[kB][4];
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < kRaw; ++i) {
            const int e = 4 * lane + 256 * i;
            *reinterpret_cast<u32x4*>(region + P::in_pad(e)) =
                ld_nt(reinterpret_cast<const u32x4*>(h + e % N));
        }
        wave_lds_sync();
        mfma_stage1_lds<C>(region, a, lane, v);
        steps(v);
        keep(v);
    }

    auto offset = [&](long long tl) { return (tl * P::kFPB + wave * P::kFPW) * N; };
    // Per-signal filters at C <= 4: the loads run a transform ahead of their
    // use, in registers that are free at that point -- the signal's while the
    // filter is transformed (its packed spectrum is not live yet), the next
    // tile's filter while the inverse runs (the spectrum is dead after the
    // product).  1-4% faster at N = 256...1024.  At C = 8 (256 VGPRs) only
    // the signal's loads move ahead of the filter's transform (90-91 against
    // 92-94 us for 16384 x 2048, same 8-byte spill); loading the next filter
    // during the inverse as well spills 44 bytes per lane (97 us).
    constexpr bool kPipelined = kPerSignal && C <= 4;
    // A shared filter at C <= 4: the next tile's signal loads are issued as
    // soon as the current one is staged (its registers are free then); 1-3%
    // faster at 2^25 values (at C = 8 the registers are not there).
    constexpr bool kPrefetchShared = !kPerSignal && C <= 4;
    u32x4 rh[kRaw];
    if constexpr (kPipelined) load(h + offset(tile), tile < tile_end ? valid(tile) : 0, rh);
    u32x4 rn[kRaw];
    if constexpr (kPrefetchShared) load(x + offset(tile), tile < tile_end ? valid(tile) : 0, rn);
    // At N = 2048 a wave's issue priority falls as its workgroup gets ahead
    // (ProgressPriority): 63.5 against 66-67 us (shared filter) and 91.0
    // against 91.7-92.0 us (per-signal) at 2^25 values; neutral at N <= 1024.
    // The next tile's level is set after the stores: set at the top of the
    // loop body, it cost the per-signal kernel 8 more bytes of register spill.
    long long left = (tile_end - tile + step - 1) / step;
    const ProgressPriority priority(left);
    if constexpr (C == 8) priority.set(left);
    for (; tile < tile_end; tile += step) {
        const int nv = valid(tile);
        const long long off = offset(tile);
        cpx v[kB][4];
        {
            u32x4 rx[kRaw];
            if constexpr (kPipelined) {
                stage(rh);
                load(x + off, nv, rx);
                forward(v);
                keep(v);
            } else if constexpr (kPerSignal) {
                load(h + off, nv, rh);
                load(x + off, nv, rx);
                stage(rh);
                forward(v);
                keep(v);
            } else if constexpr (kPrefetchShared) {
                stage(rn);
                load(x + offset(tile + step), tile + step < tile_end ? valid(tile + step) : 0, rn);
                forward(v);
            } else {
                load(x + off, nv, rx);
            }
            if constexpr (!kPrefetchShared) {
                stage(rx);
                forward(v);
            }
        }
#pragma unroll
        for (int b = 0; b < kB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float2 hk = __half22float2(__builtin_bit_cast(__half2, hp[b][r]));
                v[b][r] = cmul(v[b][r], cpx{hk.x, hk.y});
            }
        if constexpr (kPipelined)
            load(h + offset(tile + step), tile + step < tile_end ? valid(tile + step) : 0, rh);
        // ---- inverse = conj(DFT(conj(product))) / N, stage 1 from the registers ----
        mfma_stage1_regs<C, true>(a_regs, v);
        steps(v);
        // ---- store: block (f, m), lane (n, q) holds y_f[n + 16 m + 16C (q + 4 r)] ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < kB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::out_pad((b / C) * N + n + 16 * (b % C) + P::kM * (q + 4 * r))] =
                    pack_half2({v[b][r].re, -v[b][r].im});
        wave_lds_sync();
        // The staging addresses as one base and constant steps: computed per
        // piece, they kept enough registers live to spill one (8 bytes per
        // lane, reloaded among the stores at N = 2048).
        // Stores through a resource of the nv valid values (pieces past them
        // are dropped by the range check), with no branch.
        const __amdgpu_buffer_rsrc_t ys =
            __builtin_amdgcn_make_buffer_rsrc(y + off, 0, 4 * nv, 0x00020000);
        const unsigned* const obase = region + P::out_pad(4 * lane);
#pragma unroll
        for (int i = 0; i < kRaw; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(
                *reinterpret_cast<const u32x4*>(obase + P::kOutStep * i), ys, 16 * lane, 1024 * i, 2);
        if constexpr (C == 8) priority.set(--left);
    }
}

}  // namespace thff

namespace thff {

// Real-input fused convolution at N = 4096 (the reference's default length)
// on the three-stage MFMA transform of c2c_mfma4096_kernel, one complex
// transform (two real rows) per workgroup tile.
//   forward: stage 1 over j for t = 64 w + 4 n + b (inputs straight from the
//            two rows: 4 consecutive values of each, interleaved into half2),
//            exchange, stage 2, transpose, stage 3 -> lane (n, q) of block b
//            holds Z[k1 + 16 k2 + 256 k3], k1 = 4 w + b, k2 = n, k3 = q + 4 r;
//   product with the channel's spectrum, conjugated;
//   inverse: as conj(DFT(conj(Z H))), the same forward stages: stage 1
//            straight from those registers (sequence t' = k1 + 16 k2
//            = 4 w + b + 16 n, inputs k3 = q + 4 r: interleaved operands),
//            exchange with t0' = 4 w + b, t1' = n, stage 2, transpose,
//            stage 3 -> conj(y[k1' + 16 k2' + 256 k3']), then staged output
//            (conjugated back) split into the two rows.
// The exchange layout is xaddr4096 (fft_mfma.hpp).  The stage-1 -> 2 twiddle
// W^(t k1) is not multiplied in: with t = t0 + 16 t1 it is W_256^(t1 k1)
// W_4096^(t0 k1); the exchange gives each stage-2 block one k1 (its inputs
// t1, its sequences t0), so the first factor is folded into that block's
// operand columns (dft16_operand_twiddled) and the second into the stage-2 ->
// 3 twiddle.  Against the fp32 multiply after stage 1 (and the inverse's own
// operands, and the interleave by shifts and masks instead of v_perm_b32):
// 62.0-64.6 against 73.9-76.5 us for 2^26 samples, per-tile VALU 499 -> 360
// instructions, rel L2 against fp64 5.99e-4 against 6.14e-4 (MI355X).
// Every HBM access is 16 bytes: lanes n and n + 1 (n even) need the same 8
// consecutive values of both rows (4 each), so the even lane loads row 0's 8,
// the odd lane row 1's, and they swap the halves the other needs (a DPP lane
// swap); the stores pair up the same way.  The next tile's pieces are loaded
// before the current tile is transformed.  Against 8-byte accesses without
// the prefetch: 76.6-76.8 against 78.0 us for 2^26 samples (MI355X).  The
// swaps and selects cost most of what the 16-byte accesses and the prefetch
// gain: with the same bytes moved in 16-byte pieces by every lane (no swap,
// wrong results) the kernel took 69 us.

// The value of lane l ^ 1 (adjacent lanes swap; DPP quad_perm [1, 0, 3, 2]).
__device__ __forceinline__ unsigned swap_lane_pair(unsigned v) {
    return static_cast<unsigned>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, false));
}

// Buffer addressing of the tile's two rows for kBufferIO: one resource per
// tile starts at row (2p, d) and spans through row (2p + 1, d), channels * N
// values further, or covers row 0 alone when the batch is odd and row 1 does
// not exist.  Every lane then issues the same unconditional 16-byte access:
// even lanes at their row-0 offset, odd lanes at channels * N values further,
// and the hardware's range check returns zeros for (and drops the stores of)
// the missing row.  Byte offsets are 32-bit: the form is used while
// (channels + 1) * N * 2 bytes fit in 31 bits.
struct RealRowPair {
    long long row0;  // element offset of row (2p, d)
    int bytes;       // resource size: both rows, or row 0 alone
    __host__ __device__ static RealRowPair at(long long p, int d, int channels, int batch,
                                              int n) {
        const long long row0 = (2 * p * channels + d) * static_cast<long long>(n);
        const int values = 2 * p + 1 < batch ? (channels + 1) * n : n;
        return {row0, 2 * values};
    }
};
// Byte offset, from row 0, of load piece e (values 64 w + 4 (n & ~1) + 1024 q
// + 256 e .. + 7 of row 0 for an even lane, of row 1 for an odd one).
__host__ __device__ __forceinline__ int real4096_load_offset(int channels, int wave, int n, int q,
                                                             int e) {
    const int row = (n & 1) ? channels * 4096 : 0;
    return 2 * (row + 64 * wave + 4 * (n & ~1) + 1024 * q + 256 * e);
}
// Byte offset, from row 0, of store piece i of lane tid (values k .. k + 7 of
// row 0 for an even lane, k - 4 .. k + 3 of row 1 for an odd one, k = 4 tid +
// 1024 i).
__host__ __device__ __forceinline__ int real4096_store_offset(int channels, int tid, int i) {
    const int k = 4 * tid + 1024 * i;
    return 2 * ((tid & 1) ? channels * 4096 + k - 4 : k);
}
// The largest channel count kBufferIO takes at N = 4096.
inline constexpr int kReal4096BufferMaxChannels = (0x7fffffff / (2 * 4096)) - 1;

template <int N, bool kBufferIO = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
conv1d_real_mfma4096_kernel(const __half* __restrict__ x, const float2* __restrict__ spectrum,
                            __half* __restrict__ y, int batch, int channels,
                            const float2* __restrict__ tw, int tiles_per_block) {
    using P = Mfma4096;
    static_assert(N == P::N, "the three-stage transform is N = 4096");
    __shared__ __align__(16) unsigned xbuf[P::kExchange];
    __shared__ __align__(16) unsigned obuf[P::kOut];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* const region = xbuf + 4 * P::kMatrix * wave;

    // Both directions run the forward transform: the inverse is
    // conj(DFT(conj(P))), its input conjugated at the product and its output
    // at the store.  Operands: `a` plain (forward stage 1, stage 3),
    // `a_regs` column-permuted (the inverse's stage 1 from registers), and
    // per block b the stage-2 matrix of k1 = 4 w + b with the stage-1 -> 2
    // twiddle's factor W_256^(t1 k1) folded into its columns (the exchange
    // gives every block one k1: its 16 sequences are t0 = n, its inputs t1).
    // The rest of that twiddle, W_4096^(t0 k1), joins the stage-2 -> 3
    // twiddle W_256^(t0 k2): w2[b][r] = W^(n (k1 + 16 k2)), k2 = q + 4 r
    // (positive angles, conjugated at use).  No multiply remains between
    // stages 1 and 2; the folded factor is rounded into the f16 coefficient,
    // the size of the f16 rounding of the data at that stage.
    f16x8 a[2], a_regs[2], a2[4][2];
    dft16_operands<true>(a, lane);
    dft16_operands<true, true>(a_regs, lane);
    cpx w2[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int h = 0; h < 2; ++h) a2[b][h] = dft16_operand_twiddled<true>(lane, h, 4 * wave + b, 16, tw);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float2 g = tw[(n * (4 * wave + b + 16 * (q + 4 * r))) & (N - 1)];
            w2[b][r] = cpx{g.x, g.y};
        }
    }

    // tiles_per_block = 0: the grid is sized to the device and walks the
    // transforms grid-stride (tile_walk); otherwise contiguous runs.
    const long long transforms = (static_cast<long long>(batch) + 1) / 2 * channels;
    long long tile, tile_end, step;
    tile_walk(transforms, tiles_per_block, tile, tile_end, step);

    // Stage 2 (twiddle-folded operands), the wave-local transpose and stage 3.
    auto stages23 = [&](cpx (&v)[4][4]) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(
                region + P::kMatrix * b + 16 * n + 4 * ((q + (n >> 2)) & 3));
            u32x4 xv;  // t1 = 4 q + e sits at position (e + k1) & 3 = (e + b) & 3
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = raw[(e + b) & 3];
            dft16_block(a2[b], as_f16x8(xv), v[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[b][r] = cmulc(v[b][r], w2[b][r]);
        }
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[tpos(b, q + 4 * r, n)] =
                    pack_half2(v[b][r]);
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 xv = *reinterpret_cast<const u32x4*>(
                region + tchunk(b, n, q));
            dft16_block(a, as_f16x8(xv), v[b]);
        }
    };

    // The channel's spectrum stays in registers while the channel does not
    // change: on a grid-stride walk whose stride is a multiple of the channel
    // count every tile of a workgroup has the same channel.
    long long spec_d = -1;
    cpx spec[4][4];
    const ChannelWalk walk(step, channels);  // pair and channel of the tile, advanced per tile
    ChannelPos pos = walk.at(tile);
    const bool odd = (lane & 1) != 0;
    // Byte selectors of v_perm_b32 (halves): kLow {s1.lo, s0.lo}, kHigh
    // {s1.hi, s0.hi}, and the other order.  Per lane they put row 0's value
    // in the low half of each half2.
    constexpr unsigned kLow = kHalvesLow, kHigh = kHalvesHigh;
    constexpr unsigned kLowSwapped = 0x01000504u, kHighSwapped = 0x03020706u;
    const unsigned sel_lo = odd ? kLowSwapped : kLow, sel_hi = odd ? kHighSwapped : kHigh;
    // Output: a row's two values out of two half2 dwords: row 0 (kLow) or row 1 (kHigh).
    const unsigned sel_keep = odd ? kHigh : kLow, sel_send = odd ? kLow : kHigh;
    // Element offsets of a tile's two rows (row 1: -1 past an odd batch's end).
    auto rows = [&](ChannelPos ps, long long& r0, long long& r1) {
        r0 = (2 * ps.p * channels + ps.d) * N;
        r1 = 2 * ps.p + 1 < batch ? ((2 * ps.p + 1) * channels + ps.d) * N : -1;
    };
    // Values 64 w + 4 (n & ~1) + 1024 q + 256 e .. + 7 of row 0 (even lanes)
    // or row 1 (odd lanes).
    const int load_off = real4096_load_offset(channels, wave, n, q, 0);
    // kBufferIO: `live` false gives the resource no bytes, so the loads
    // return zeros without touching memory; every tile then issues the same
    // loads with no branch, and the compiler counts them exactly (it waits
    // for the prefetched pieces, not for the previous tile's stores).
    auto load = [&](ChannelPos ps, u32x4 (&raw)[4], bool live = true) {
        if constexpr (kBufferIO) {
            const RealRowPair rp = RealRowPair::at(ps.p, ps.d, channels, batch, N);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<__half*>(x + rp.row0), 0, live ? rp.bytes : 0, 0x00020000);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                raw[e] = __builtin_amdgcn_raw_buffer_load_b128(rs, load_off, 512 * e, 2);
        } else {
            long long r0, r1;
            rows(ps, r0, r1);
            const long long row = odd ? r1 : r0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = 64 * wave + 4 * (n & ~1) + 1024 * q + 256 * e;
                raw[e] = row >= 0 ? ld_nt(reinterpret_cast<const u32x4*>(x + row + k)) : u32x4{};
            }
        }
    };
    u32x4 next[4];
    if constexpr (kBufferIO) {
        if (tile >= tile_end) return;  // uniform over the workgroup
        load(pos, next);
        // Four stores to a resource of no bytes (dropped by the range check):
        // the loop is then entered, like every later pass, with the pieces
        // followed by four stores in flight, so the compiler's count at the
        // loop top waits for the pieces only, not for the last tile's stores.
        // (The size is written as a run-time value, batch >= 0 always, which
        // keeps the compiler from deleting stores it can prove are dropped.)
        const __amdgpu_buffer_rsrc_t none =
            __builtin_amdgcn_make_buffer_rsrc(y, 0, batch < 0 ? 16 : 0, 0x00020000);
        __builtin_amdgcn_sched_barrier(0);  // after the loads, as in the loop
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_amdgcn_raw_buffer_store_b128(u32x4{}, none, 16 * i, 0, 2);
    } else if (tile < tile_end)
        load(pos, next);
    for (; tile < tile_end; tile += step) {
        const long long p = pos.p, d = pos.d;
        long long row0, row1;
        rows(pos, row0, row1);
        [[maybe_unused]] __amdgpu_buffer_rsrc_t yrs;
        if constexpr (kBufferIO) {
            const RealRowPair rp = RealRowPair::at(pos.p, pos.d, channels, batch, N);
            yrs = __builtin_amdgcn_make_buffer_rsrc(y + rp.row0, 0, rp.bytes, 0x00020000);
        }
        pos = walk.advance(pos);
        // ---- stage-1 inputs: values 64 w + 4 n + 1024 q + 256 e .. + 3 of both rows ----
        u32x4 z[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u32x4 w = next[e];
            // even lane: keeps row 0's first half (u), gets row 1's (g);
            // odd: keeps row 1's second half, gets row 0's
            const unsigned u0 = odd ? w.z : w.x, u1 = odd ? w.w : w.y;
            const unsigned g0 = swap_lane_pair(odd ? w.x : w.z);
            const unsigned g1 = swap_lane_pair(odd ? w.y : w.w);
            z[e] = u32x4{halves(g0, u0, sel_lo), halves(g0, u0, sel_hi),
                         halves(g1, u1, sel_lo), halves(g1, u1, sel_hi)};
        }
        if constexpr (kBufferIO)
            load(pos, next, tile + step < tile_end);
        else if (tile + step < tile_end)
            load(pos, next);
        cpx v[4][4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            u32x4 xv;
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = z[e][b];
            dft16_block(a, as_f16x8(xv), v[b]);
        }
        __syncthreads();  // every wave is done with the previous tile's exchange buffer
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                xbuf[xaddr4096(q + 4 * r, 4 * (n & 3) + b, 4 * wave + (n >> 2))] = pack_half2(v[b][r]);
        __syncthreads();
        stages23(v);
        // ---- product: bin k = 4 w + b + 16 n + 256 (q + 4 r) ----
        if (d != spec_d) {  // uniform: a new channel's spectrum
            const float2* hs = spectrum + d * N + 4 * wave + 16 * n + 256 * q;
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float2 hk = hs[b + 1024 * r];
                    spec[b][r] = cpx{hk.x, -hk.y};  // conj(H)
                }
            // Wait here, on this rarely taken path: a wait after the branch
            // would have to count these loads as the latest ones and so
            // would also wait for the next tile's pieces on every tile.
            wait_vmem_all();
            spec_d = d;
        }
        // ---- inverse stage 1 from the registers: the forward DFT16 over k3
        // of conj(Z H) = conj(Z conj(G)), G = conj(H) held in spec, sequences
        // t' = 4 w + b + 16 n (written as two products each, which the
        // compiler fuses with the f16 rounding) ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            u32x4 xv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const cpx z = v[b][r], g = spec[b][r];
                xv[r] = pack_half2(cpx{z.re * g.re + z.im * g.im, z.re * g.im - z.im * g.re});
            }
            dft16_block(a_regs, as_f16x8(xv), v[b]);
        }
        __syncthreads();  // every wave's forward stage-3 reads are done
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                xbuf[xaddr4096(q + 4 * r, 4 * wave + b, n)] = pack_half2(v[b][r]);
        __syncthreads();
        stages23(v);
        // ---- output: conj of the forward result is y[k1 + 16 k2 + 256 k3],
        // k1 = 4 w + b, k2 = n, k3 = q + 4 r ----
#pragma unroll
        for (int r = 0; r < 4; ++r)
            reinterpret_cast<u32x4*>(obuf)[P::out_chunk(wave + 4 * n + 64 * (q + 4 * r))] =
                u32x4{pack_half2(cpx{v[0][r].re, -v[0][r].im}), pack_half2(cpx{v[1][r].re, -v[1][r].im}),
                      pack_half2(cpx{v[2][r].re, -v[2][r].im}), pack_half2(cpx{v[3][r].re, -v[3][r].im})};
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = 4 * tid + 1024 * i;
            const u32x4 z4 = reinterpret_cast<const u32x4*>(obuf)[P::out_chunk(tid + 256 * i)];
            // values k .. k + 3 of both rows; the even lane stores row 0's
            // k .. k + 7, the odd lane row 1's k - 4 .. k + 3: each keeps
            // its own row's four values and sends the other row's
            const u32x2 keep{halves(z4.y, z4.x, sel_keep),
                             halves(z4.w, z4.z, sel_keep)};
            const unsigned g0 = swap_lane_pair(halves(z4.y, z4.x, sel_send));
            const unsigned g1 = swap_lane_pair(halves(z4.w, z4.z, sel_send));
            if constexpr (kBufferIO) {
                const u32x4 w4 = odd ? u32x4{g0, g1, keep.x, keep.y} : u32x4{keep.x, keep.y, g0, g1};
                __builtin_amdgcn_raw_buffer_store_b128(w4, yrs, real4096_store_offset(channels, tid, i),
                                                       0, 2);
            } else {
                if (!odd)
                    st_nt(reinterpret_cast<u32x4*>(y + row0 + k), u32x4{keep.x, keep.y, g0, g1});
                else if (row1 >= 0)
                    st_nt(reinterpret_cast<u32x4*>(y + row1 + k - 4), u32x4{g0, g1, keep.x, keep.y});
            }
        }
    }
}

}  // namespace thff

namespace thff {

// Complex fused convolution at N = 4096 on the three-stage MFMA transform
// (conv1d_kernel's contract, half2 storage): per tile (one signal) the
// filter's forward transform (per-signal filters; a shared filter is
// transformed once per workgroup), the signal's, the product with the
// filter spectrum kept packed as half2 (1/N folded in) and the inverse from
// registers, as in conv1d_real_mfma4096_kernel.  Grid: sized to the device
// (a few workgroups per CU), walking the signals grid-stride (tile_walk).
// The stage-1 -> 2 twiddle is folded into the stage-2 operands and the
// stage-2 -> 3 twiddle, and the inverse runs the forward stages on the
// conjugated product, as there: 89.5-91.2 against 95.5-97.0 us (per-signal
// filters), 58.2-60.3 against 64.1-66.4 us (shared filter), 2^25 values.
// Per-signal filters: held to 168 VGPRs (3 workgroups per CU) at the cost of a
// 24-byte spill: 89.5-91.2 us against 92.8-93.8 us at 2 per CU (170 VGPRs, no
// spill; MI355X).  A shared filter keeps its spectrum live across the loop: 2
// per CU, and the next signal's loads are issued before the current one's
// transform (64 us against 73 us before the fold; for per-signal filters the
// extra registers spill and it measured slower, 102 against 97 us).
template <bool kPerSignal>
inline constexpr int kConv4096MinWavesPerEU = kPerSignal ? 3 : 2;

template <int N, bool kPerSignal>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kConv4096MinWavesPerEU<kPerSignal>))) void
conv1d_mfma4096_kernel(const __half2* __restrict__ x, const __half2* __restrict__ h,
                       __half2* __restrict__ y, int batch, const float2* __restrict__ tw) {
    using P = Mfma4096;
    static_assert(N == P::N, "the three-stage transform is N = 4096");
    __shared__ __align__(16) unsigned xbuf[P::kExchange];
    __shared__ __align__(16) unsigned obuf[P::kOut];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* const region = xbuf + 4 * P::kMatrix * wave;
    constexpr float kScale = 1.0f / N;

    // As in conv1d_real_mfma4096_kernel: both directions run the forward
    // transform (the inverse as conj(DFT(conj(P)))), with the stage-1 -> 2
    // twiddle folded into the per-block stage-2 operands a2 and the
    // stage-2 -> 3 twiddles w2[b][r] = W^(n (k1 + 16 k2)).
    f16x8 a[2], a_regs[2], a2[4][2];
    dft16_operands<true>(a, lane);
    dft16_operands<true, true>(a_regs, lane);
    cpx w2[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) a2[b][hh] = dft16_operand_twiddled<true>(lane, hh, 4 * wave + b, 16, tw);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float2 g = tw[(n * (4 * wave + b + 16 * (q + 4 * r))) & (N - 1)];
            w2[b][r] = cpx{g.x, g.y};
        }
    }

    auto stages23 = [&](cpx (&v)[4][4]) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(
                region + P::kMatrix * b + 16 * n + 4 * ((q + (n >> 2)) & 3));
            u32x4 xv;
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = raw[(e + b) & 3];
            dft16_block(a2[b], as_f16x8(xv), v[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[b][r] = cmulc(v[b][r], w2[b][r]);
        }
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[tpos(b, q + 4 * r, n)] =
                    pack_half2(v[b][r]);
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 xv = *reinterpret_cast<const u32x4*>(
                region + tchunk(b, n, q));
            dft16_block(a, as_f16x8(xv), v[b]);
        }
    };
    // Stage-1 inputs of the 4096 values at src: x[64 w + 4 n + b + 256 j],
    // j = 4 q + e, in z[e][b].
    auto load = [&](const __half2* src, u32x4 (&z)[4]) {
        const __half2* s = src + 64 * wave + 4 * n + 1024 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e) z[e] = ld_nt(reinterpret_cast<const u32x4*>(s + 256 * e));
    };
    // Forward transform of loaded inputs (callers: every wave done with xbuf
    // before, as the first barrier inside requires).
    auto forward = [&](const u32x4 (&z)[4], cpx (&v)[4][4]) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            u32x4 xv;
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = z[e][b];
            dft16_block(a, as_f16x8(xv), v[b]);
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                xbuf[xaddr4096(q + 4 * r, 4 * (n & 3) + b, 4 * wave + (n >> 2))] = pack_half2(v[b][r]);
        __syncthreads();
        stages23(v);
    };

    // conj(FFT(h)) / N at bins 4 w + b + 16 n + 256 (q + 4 r), packed half2
    unsigned hp[4][4];
    auto keep = [&](const cpx (&v)[4][4]) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) hp[b][r] = pack_half2({v[b][r].re * kScale, -v[b][r].im * kScale});
    };
    long long tile, tile_end, step;
    tile_walk(batch, 0, tile, tile_end, step);
    if (tile >= tile_end) return;  // uniform over the workgroup
    u32x4 zx[4];  // shared filter: the next signal's inputs
    if constexpr (!kPerSignal) {
        cpx v[4][4];
        u32x4 zh[4];
        load(h, zh);
        forward(zh, v);
        keep(v);
        load(x + tile * N, zx);
    }
    // A wave's issue priority falls as its workgroup gets ahead of the others
    // (ProgressPriority): 95 against 99-101 us (per-signal) and 65 against
    // 67-69 us (shared filter) at 2^25 values.
    long long left = (tile_end - tile + step - 1) / step;
    const ProgressPriority priority(left);
    for (; tile < tile_end; tile += step, --left) {
        priority.set(left);
        cpx v[4][4];
        if constexpr (kPerSignal) {
            u32x4 z[4];
            load(h + tile * N, z);
            forward(z, v);
            keep(v);
            load(x + tile * N, z);
            forward(z, v);
        } else {
            u32x4 z[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) z[i] = zx[i];
            if (tile + step < tile_end) load(x + (tile + step) * N, zx);
            forward(z, v);
        }
        // ---- inverse: the forward DFT16 over k3 of conj(Z H) = conj(Z
        // conj(G)), G = conj(H) held in hp, from the registers; exchange,
        // stages 2-3; the output conjugated at the staging ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            u32x4 xv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float2 g = __half22float2(__builtin_bit_cast(__half2, hp[b][r]));
                const cpx z = v[b][r];
                xv[r] = pack_half2(cpx{z.re * g.x + z.im * g.y, z.re * g.y - z.im * g.x});
            }
            dft16_block(a_regs, as_f16x8(xv), v[b]);
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                xbuf[xaddr4096(q + 4 * r, 4 * wave + b, n)] = pack_half2(v[b][r]);
        __syncthreads();
        stages23(v);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            reinterpret_cast<u32x4*>(obuf)[P::out_chunk(wave + 4 * n + 64 * (q + 4 * r))] =
                u32x4{pack_half2(cpx{v[0][r].re, -v[0][r].im}), pack_half2(cpx{v[1][r].re, -v[1][r].im}),
                      pack_half2(cpx{v[2][r].re, -v[2][r].im}), pack_half2(cpx{v[3][r].re, -v[3][r].im})};
        __syncthreads();
        __half2* dst = y + tile * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            st_nt(reinterpret_cast<u32x4*>(dst + 4 * tid + 1024 * i),
                  reinterpret_cast<const u32x4*>(obuf)[P::out_chunk(tid + 256 * i)]);
        }
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// Tiled valid correlation for half2 on MFMA with 256-point windows (the
// contract of conv1d_valid_kernel, fft_conv.hpp; the reference's
// conv1d_direct_fft_kernel, sample/conv1d/main.cu:38-128, slides 64-point
// windows):
//   y[b][i] = sum_{k < F} x[b][i + k] * f[k],   i < L - F + 1,  1 <= F <= 64.
// Window w of a signal is x[w V .. w V + 255] with V = 257 - F (193..256
// valid outputs): its circular convolution with g[m] = f[(256 - m) mod 256]
// equals y[w V + j] for j < V, which never wrap.  Against 64-point windows
// this re-reads (F - 1)/256 of the input instead of (F - 1)/64 and moves
// 4 windows per wave instead of 16, on the two-stage MFMA transform of
// N = 256 (fft_mfma.hpp, C = 1: a wave owns 4 transforms, one per window).
// Per wave and group of 4 windows: stage the span x[w0 V .. w0 V + 3 V + 255]
// in the wave's LDS region (16-byte loads when the signal starts on a
// 16-byte boundary; zeros past its end), the forward transform straight
// from the span (window b starts at b V), the product with G = FFT(g) / 256,
// the inverse as conj(DFT(conj(P))) from registers, then the V valid outputs
// of each window compacted into the region and stored as one run of 4 V
// values (16-byte stores when the output signal starts on a 16-byte
// boundary; w0 V is a multiple of 4 values).
// Set-up per workgroup, no table but the kernel's own: W_256 twiddles
// (sincospi, fp32) in LDS, G in fp32 by direct evaluation over the F taps
// (one bin per lane), the step-2 twiddles and the DFT16 operands.  Nothing
// crosses waves after the set-up.
// ---------------------------------------------------------------------------
template <int N = 256>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void
conv1d_valid_mfma_kernel(const __half2* __restrict__ x, const float2* __restrict__ taps,
                         __half2* __restrict__ y, long long len, int ntaps, int batch,
                         int groups_per_block) {
    static_assert(N == 256, "256-point windows (the two-stage MFMA transform, C = 1)");
    using P = MfmaPlan<1>;
    constexpr int kWindows = P::kBlocks;         // 4 windows per wave
    constexpr int kGroup = 4 * kWindows;         // windows per workgroup tile
    static_assert(P::kRegion >= 1024 + 16 * 16, "span of 3 V + 256 <= 1024 values, padded");
    __shared__ __align__(16) unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    __shared__ float2 tw256[N];
    __shared__ cpx spectrum[N];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* const region = lds + wave * P::kRegion;
    const int V = 257 - ntaps;

    {
        float s, c;
        sincospif(static_cast<float>(tid) / 128.0f, &s, &c);  // (cos, sin)(2 pi tid / 256)
        tw256[tid] = make_float2(c, s);
    }
    __syncthreads();
    {
        // G[k] = (1/256) sum_{k' < F} f[k'] e^(+2 pi i k' k / 256): the forward
        // transform of g, one bin per lane.
        const int k = tid;
        cpx acc{0.f, 0.f};
        for (int kk = 0; kk < ntaps; ++kk) {
            const float2 f = taps[kk];
            const float2 w = tw256[(kk * k) & (N - 1)];
            acc = cadd(acc, cmul(cpx{f.x, f.y}, cpx{w.x, w.y}));
        }
        spectrum[k] = {acc.re * (1.0f / N), acc.im * (1.0f / N)};
        // step-2 twiddles W_256^(n k1), k1 = q + 4 r (C = 1), forward
        const int l = tid & 63, r = tid >> 6;
        const float2 w = tw256[((l & 15) * ((l >> 4) + 4 * r)) & (N - 1)];
        w1[tid] = cpx{w.x, -w.y};
    }
    f16x8 a[2], a_regs[2];
    dft16_operands<true>(a, lane);
    dft16_operands<true, true>(a_regs, lane);
    const Stage3Plain<false> s3{a, nullptr};
    __syncthreads();
    // The lane's bins n + 16 (q + 4 r) of G, the same for its 4 windows.
    cpx gk[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) gk[r] = spectrum[n + 16 * (q + 4 * r)];

    const long long out_len = len - ntaps + 1;
    const long long windows = (out_len + V - 1) / V;  // per signal
    const long long groups_per_signal = (windows + kGroup - 1) / kGroup;
    const long long groups = groups_per_signal * batch;
    const bool x16 = (reinterpret_cast<unsigned long long>(x) & 15) == 0;
    const bool y16 = (reinterpret_cast<unsigned long long>(y) & 15) == 0;
    const int need = 3 * V + N;  // values of the span the wave's windows read
    // (The division below stays per group: stepping the quotient as the fp32
    // kernel does spilled 36 bytes here at 128 VGPRs and measured 5% slower.)

    long long g, g_end, step;
    tile_walk(groups, groups_per_block, g, g_end, step);
    for (; g < g_end; g += step) {
        const long long b = g / groups_per_signal;
        const long long w0 = (g - b * groups_per_signal) * kGroup + wave * kWindows;
        const long long span0 = w0 * V;  // a multiple of 4 values
        if (span0 >= out_len) continue;  // none of the wave's windows has an output
        const long long avail_l = len - span0 < need ? len - span0 : need;
        const int avail = static_cast<int>(avail_l);
        const __half2* src = x + b * len + span0;
        const bool in_vec = x16 && (b * len) % 4 == 0;
        const bool out_vec = y16 && (b * out_len) % 4 == 0;

        wave_lds_sync();  // the previous group's reads of the region are done
        if (in_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = 4 * lane + 256 * i;
                u32x4 v{};
                if (e + 4 <= avail) {
                    v = ld_nt(reinterpret_cast<const u32x4*>(src + e));
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (e + c < avail) v[c] = *reinterpret_cast<const unsigned*>(src + e + c);
                }
                *reinterpret_cast<u32x4*>(region + P::in_pad(e)) = v;
            }
        } else {
#pragma unroll 4
            for (int i = 0; i < 16; ++i) {
                const int e = lane + 64 * i;
                region[P::in_pad(e)] = e < avail ? *reinterpret_cast<const unsigned*>(src + e) : 0u;
            }
        }
        wave_lds_sync();
        // ---- forward: window bb's stage-1 inputs x[bb V + n + 16 j] ----
        cpx v[kWindows][4];
#pragma unroll
        for (int bb = 0; bb < kWindows; ++bb) {
            const int base = bb * V + n;
            u32x4 xv;
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = region[P::in_pad(base + 16 * (4 * q + e))];
            dft16_block(a, as_f16x8(xv), v[bb]);
        }
        mfma_steps2to6<1, true>(region, w1, s3, lane, v);
        // ---- product with G, inverse = conj(DFT(conj(product))) from registers ----
#pragma unroll
        for (int bb = 0; bb < kWindows; ++bb)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[bb][r] = cmul(v[bb][r], gk[r]);
        mfma_stage1_regs<1, true>(a_regs, v);
        mfma_steps2to6<1, true>(region, w1, s3, lane, v);
        // ---- the V valid outputs of each window, compacted: window bb, lane (n, q)
        // holds positions n + 16 (q + 4 r) ----
        wave_lds_sync();
#pragma unroll
        for (int bb = 0; bb < kWindows; ++bb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int p = n + 16 * (q + 4 * r);
                if (p < V) region[bb * V + p] = pack_half2({v[bb][r].re, -v[bb][r].im});
            }
        wave_lds_sync();
        const long long left = out_len - span0;
        const int count = left < kWindows * V ? static_cast<int>(left) : kWindows * V;
        __half2* dst = y + b * out_len + span0;
        if (out_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = 4 * lane + 256 * i;
                if (e + 4 <= count) {
                    st_nt(reinterpret_cast<u32x4*>(dst + e), *reinterpret_cast<const u32x4*>(region + e));
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (e + c < count) *reinterpret_cast<unsigned*>(dst + e + c) = region[e + c];
                }
            }
        } else {
#pragma unroll 4
            for (int i = 0; i < 16; ++i) {
                const int e = lane + 64 * i;
                if (e < count) *reinterpret_cast<unsigned*>(dst + e) = region[e];
            }
        }
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// half2 2-D convolution of 64 x 64 images on MFMA (conv2d64_kernel's contract:
// y = IFFT2(FFT2(x) * FFT2(h)) / 4096, one shared filter), one image per
// workgroup tile.  Both 64-point transforms of the 2-D DFT split as 64 = 16 x 4:
// a DFT16 on v_mfma_f32_16x16x32_f16 over the stride-4 index, the twiddle
// W64^(j k), then an in-lane DFT4.  With lane (n, q) (lane = n + 16 q) of wave w:
//   F1 columns: wave w owns the 16 columns c = 16 w + n; block b = r0 holds the
//      DFT16 inputs r1 = 4 q + e (row r = r0 + 4 r1) from the staged image; the
//      grouped operands (dft16_operands_grouped) leave kr1 = 4 q + t in t, so
//      after W64^(r0 kr1) and the DFT4 over r0 the lane holds
//      Xc[kr = 4 q + t + 16 kr0][c], four consecutive rows per kr0.
//   exchange (LDS, column-major, 16-byte writes) to rows: wave w owns the rows
//      kr = 16 w + n; block c0 holds inputs c1 = 4 q + e (c = c0 + 4 c1).
//   F2 rows: DFT16 (grouped outputs kc1 = 4 q + t), W64^(c0 kc1), DFT4 over c0
//      -> spectrum X[kr = 16 w + n][kc = 4 q + t + 16 kc0], the filter's alike.
// The inverse is conj(DFT2(conj(P))), rows first, straight from the spectrum:
// kc = kc1 + 16 kc0 gives the DFT4 over kc0 in-lane first, W64^(kc1 k1), then
// the DFT16 over kc1 (whose lane group q already holds kc1 = 4 q + t) -> column
// c = k1 + 16 q + 4 r; an exchange (row-major, 16-byte writes) back to columns
// with rows kr = 4 q + e + 16 n2 per lane: DFT4 over n2, W64^((4 q + e) k1),
// DFT16 over n1 = 4 q + e (plain q + 4 r outputs) -> row k1 + 4 q + 16 r, staged
// for 16-byte stores.  Every twiddle multiplies a DFT16's outputs (F1, F2) or
// inputs (the inverse) in block j = 1..3, so it is folded into that block's
// DFT16 operands: output k, input i of the complex coefficient matrix become
// W64^(k (j + 4 i)) (outputs twiddled) or W64^(i (4 k + j)) (inputs
// twiddled), rounded to f16 like the data at that stage.  Block 0 uses the
// plain operands; the 18 other operand sets (3 forms x 3 blocks x 2 halves)
// are built once per workgroup into an LDS table.  f16 data enters each DFT16,
// fp32 elsewhere; the filter spectrum (x 1/4096) stays in fp32 registers.  Two
// LDS buffers alternate, so an image takes four workgroup barriers.
// Bank-conflict-free layouts (dword units):
//   input staging  (r, c) at r 64 + c + 16 (r >> 4)
//   forward exchange (kr, c) at c 68 + (kr ^ 16 (c >> 4))
//   inverse exchange and output staging (r, c) at r 68 + c
// ---------------------------------------------------------------------------
namespace conv2dm {
constexpr int kStride = 68;
constexpr int kBuf = 64 * kStride;  // dwords per buffer (>= every layout's extent)
__device__ __forceinline__ int in_addr(int r, int c) { return r * 64 + c + 16 * (r >> 4); }
__device__ __forceinline__ int fx_addr(int kr, int c) {
    return c * kStride + (kr ^ (16 * (c >> 4)));
}
__device__ __forceinline__ int rm_addr(int r, int c) { return r * kStride + c; }

// DFT4 over the block index of v[b][t] for every t (in-lane), forward.
__device__ __forceinline__ void dft4_blocks(cpx (&v)[4][4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        cpx u[4] = {v[0][t], v[1][t], v[2][t], v[3][t]};
        Dft<4, true>::run(u);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k][t] = u[k];
    }
}

// Operand table: form f (0: outputs twiddled, grouped outputs -- F1, F2;
// 1: inputs twiddled, grouped outputs -- inverse rows; 2: inputs twiddled,
// q + 4 r outputs -- inverse columns), block j = 1..3, half h, lane.
constexpr int kForms = 3;
constexpr int kOps = kForms * 3 * 2 * 64;  // u32x4 entries (18 KB)
__device__ __forceinline__ int op_index(int form, int j, int h, int lane) {
    return ((form * 3 + (j - 1)) * 2 + h) * 64 + lane;
}

// Entry e of the table, from the positive-angle table of length 64 (forward
// sign: the conjugate).  Row m of half h is output k (grouped: 4 (m/4) + 2 h +
// (m%4)/2; q + 4 r order: m/4 + 4 (2 h + (m%4)/2)), part (m%4)%2; column kk is
// input i = kk/2, part kk%2.
__device__ __forceinline__ u32x4 op_entry(int e, const float2* __restrict__ tw64) {
    const int lane = e & 63, h = (e >> 6) & 1, j = (e >> 7) % 3 + 1, form = (e >> 7) / 3;
    const int m = lane & 15, kq = lane >> 4;
    const int gq = m >> 2, i2 = m & 3, o = i2 & 1;
    const int k = form == 2 ? gq + 4 * (2 * h + (i2 >> 1)) : 4 * gq + 2 * h + (i2 >> 1);
    f16x8 r;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        const int kk = 8 * kq + x;
        const int in = kk >> 1, p = kk & 1;
        const int idx = form == 0 ? k * (j + 4 * in) : in * (4 * k + j);
        const float2 w = tw64[idx & 63];
        const float c = w.x, sn = -w.y;
        // out.re = c*in.re - s*in.im ; out.im = s*in.re + c*in.im
        const float v = o == 0 ? (p == 0 ? c : -sn) : (p == 0 ? sn : c);
        r[x] = static_cast<_Float16>(v);
    }
    return __builtin_bit_cast(u32x4, r);
}

// Operands of block b of a stage of form `form`: the plain ones for b = 0.
__device__ __forceinline__ void stage_ops(const u32x4* ops, const f16x8 (&plain)[2], int form,
                                          int b, int lane, f16x8 (&op)[2]) {
    if (b == 0) {
        op[0] = plain[0];
        op[1] = plain[1];
    } else {
        op[0] = __builtin_bit_cast(f16x8, ops[op_index(form, b, 0, lane)]);
        op[1] = __builtin_bit_cast(f16x8, ops[op_index(form, b, 1, lane)]);
    }
}

// The 2-D forward transform of the image staged in `in` (in_addr layout)
// through the exchange buffer `fx` -> spectrum v[kc0][t] of row 16 w + n,
// column 4 q + t + 16 kc0.  `fx` is written without a barrier before: its
// previous readers must have passed one.  Ends after the F2 reads (fx busy).
__device__ __forceinline__ void forward(const unsigned* in, unsigned* fx, const f16x8 (&ag)[2],
                                        const u32x4* ops, int wave, int lane, cpx (&v)[4][4]) {
    const int n = lane & 15, q = lane >> 4;
    // F1: columns 16 w + n, block r0, inputs r1 = 4 q + e; W64^(r0 kr1) folded
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        u32x4 xv;
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = in[in_addr(b + 16 * q + 4 * e, 16 * wave + n)];
        f16x8 op[2];
        stage_ops(ops, ag, 0, b, lane, op);
        dft16_block(op, as_f16x8(xv), v[b]);
    }
    dft4_blocks(v);  // v[kr0][t]: row 4 q + t + 16 kr0
#pragma unroll
    for (int k = 0; k < 4; ++k)
        *reinterpret_cast<u32x4*>(fx + fx_addr(4 * q + 16 * k, 16 * wave + n)) =
            u32x4{pack_half2(v[k][0]), pack_half2(v[k][1]), pack_half2(v[k][2]),
                  pack_half2(v[k][3])};
    __syncthreads();
    // F2: rows 16 w + n, block c0, inputs c1 = 4 q + e; W64^(c0 kc1) folded
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        u32x4 xv;
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = fx[fx_addr(16 * wave + n, b + 16 * q + 4 * e)];
        f16x8 op[2];
        stage_ops(ops, ag, 0, b, lane, op);
        dft16_block(op, as_f16x8(xv), v[b]);
    }
    dft4_blocks(v);  // v[kc0][t]: column 4 q + t + 16 kc0
}

}  // namespace conv2dm

template <int kPerCu = 3>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kPerCu))) void
conv2d64_mfma_kernel(const __half2* __restrict__ x, const __half2* __restrict__ h,
                     __half2* __restrict__ y, int batch, const float2* __restrict__ tw64,
                     int tiles_per_block) {
    using namespace conv2dm;
    __shared__ __align__(16) unsigned buf[2][kBuf];
    __shared__ u32x4 ops[kOps];
    unsigned* const A = buf[0];
    unsigned* const B = buf[1];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;

    f16x8 ag[2], as[2];
    dft16_operands_grouped<true>(ag, lane);
    dft16_operands<true>(as, lane);
    for (int e = tid; e < kOps; e += 256) ops[e] = op_entry(e, tw64);  // read after a barrier below

    long long img, img_end, step;
    tile_walk(batch, tiles_per_block, img, img_end, step);
    if (img >= img_end) return;  // uniform over the workgroup

    // An image's 16-byte pieces 4 tid + 1024 i, loaded and written to A.
    auto load = [&](const __half2* src, u32x4 (&raw)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            raw[i] = ld_nt(reinterpret_cast<const u32x4*>(src + 4 * tid + 1024 * i));
    };
    auto stage = [&](const u32x4 (&raw)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = 4 * tid + 1024 * i;
            *reinterpret_cast<u32x4*>(A + in_addr(f >> 6, f & 63)) = raw[i];
        }
    };

    // The filter's spectrum / 4096, in the spectrum layout.
    cpx hs[4][4];
    u32x4 next[4];  // the next image's pieces, loaded while the current one is transformed
    load(h, next);
    stage(next);
    load(x + img * 4096, next);
    __syncthreads();
    forward(A, B, ag, ops, wave, lane, hs);
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) hs[k][t] = {hs[k][t].re * (1.0f / 4096), hs[k][t].im * (1.0f / 4096)};

    long long left = (img_end - img + step - 1) / step;  // tiles still to do, this one included
    const ProgressPriority priority(left);
    for (; img < img_end; img += step, --left) {
        priority.set(left);
        // A's previous readers (the filter's F1, or the last image's inverse
        // exchange reads) passed a barrier since; B's (F2 reads) pass the one
        // after this staging.
        stage(next);
        if (img + step < img_end) load(x + (img + step) * 4096, next);
        __syncthreads();
        cpx v[4][4];
        forward(A, B, ag, ops, wave, lane, v);
        // ---- product, then the inverse as conj(DFT2(conj(P))), rows first ----
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const cpx p = cmul(v[k][t], hs[k][t]);
                v[k][t] = {p.re, -p.im};
            }
        dft4_blocks(v);  // over kc0 -> k1
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            u32x4 xv;
#pragma unroll
            for (int t = 0; t < 4; ++t) xv[t] = pack_half2(v[k][t]);  // inputs kc1 = 4 q + t
            f16x8 op[2];
            stage_ops(ops, ag, 1, k, lane, op);  // W64^(kc1 k1) folded
            dft16_block(op, as_f16x8(xv), v[k]);  // v[k1][r]: column k1 + 16 q + 4 r
        }
        // exchange to columns (A: every wave's F1 reads passed the barrier in forward)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<u32x4*>(A + rm_addr(16 * wave + n, 16 * q + 4 * r)) =
                u32x4{pack_half2(v[0][r]), pack_half2(v[1][r]), pack_half2(v[2][r]),
                      pack_half2(v[3][r])};
        __syncthreads();
        // columns 16 w + n: rows n1 + 16 n2, n1 = 4 q + e
#pragma unroll
        for (int n2 = 0; n2 < 4; ++n2)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[n2][e] = unpack_half2(A[rm_addr(4 * q + e + 16 * n2, 16 * wave + n)]);
        dft4_blocks(v);  // over n2 -> k1
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            u32x4 xv;
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = pack_half2(v[k][e]);  // inputs n1 = 4 q + e
            f16x8 op[2];
            stage_ops(ops, as, 2, k, lane, op);  // W64^(n1 k1) folded
            dft16_block(op, as_f16x8(xv), v[k]);  // v[k1][r]: row k1 + 4 q + 16 r
        }
        // output staging in B (every wave's F2 reads passed the last barrier),
        // conjugated back
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                B[rm_addr(k + 4 * q + 16 * r, 16 * wave + n)] = pack_half2({v[k][r].re, -v[k][r].im});
        __syncthreads();
        __half2* dst = y + img * 4096;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = 4 * tid + 1024 * i;
            st_nt(reinterpret_cast<u32x4*>(dst + f),
                  *reinterpret_cast<const u32x4*>(B + rm_addr(f >> 6, f & 63)));
        }
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// half2 2-D convolution of 128 x 128 images on MFMA (the contract of
// conv2d128_lanes_kernel: y = IFFT2(FFT2(x) * FFT2(h)) / 16384, one shared filter;
// the reference's 128-tile sketch is sample/conv2d/thunder_tile128.cu:64-237),
// one image per workgroup tile of 512 lanes (8 waves).  Both 128-point
// transforms split as 128 = 16 x 8: a DFT16 on v_mfma_f32_16x16x32_f16 over
// the stride-8 index with the twiddle W128^(j k) folded into block j's
// operands, then an in-lane DFT8 over the block index.  Lane (n, q) (lane =
// n + 16 q) of wave w:
//   F1 columns: wave w owns the columns c = 16 w + n; block b = r0 holds the
//      inputs r1 = 4 q + e (row r = r0 + 8 r1) of the staged image; grouped
//      outputs kr1 = 4 q + t, so after the DFT8 over r0 the lane holds
//      Xc[kr = 4 q + t + 16 kr0][c]: four consecutive rows per kr0, written
//      to the exchange buffer as one 16-byte chunk.
//   F2 rows: wave w owns the rows kr = 16 w + n; block c0 holds the inputs
//      c1 = 4 q + e (c = c0 + 8 c1) -> spectrum S[16 w + n][4 q + t + 16 kc0].
// The product with the filter spectrum (built by the same steps once per
// workgroup, x 1/16384, fp32 registers) is lane-local.  The inverse is
// conj(DFT2(conj(P))): conj(P) is written back in the image's layout (each
// lane's four consecutive columns of its row as one 16-byte chunk) and the
// same F1 / F2 run on it; conj of their result is staged the same way and
// stored in 16-byte pieces.  Two LDS buffers swap roles per image (staging /
// product / output in one, the exchange in the other): five workgroup
// barriers per image.  2 x 66 KiB of buffers and the 14 KiB operand table
// allow one workgroup per CU (2 waves per SIMD); the next image's pieces are
// loaded while the current one is transformed.
// Layouts (dwords = half2 values), conflict-free for every access in a bank
// model checked on the CPU (16-byte accesses 16 lanes per cycle over 64
// banks, dword reads 32 lanes per cycle over 32):
//   image / product / output (r, c) at r 132 + c + 16 (r >> 5)
//   exchange (kr, c) at c 132 + (kr ^ 16 ((c >> 5) & 1))
// ---------------------------------------------------------------------------
namespace conv2dm128 {
constexpr int kStride = 132;
constexpr int kBuf = 128 * kStride + 48;  // dwords per buffer
__device__ __forceinline__ int rm_addr(int r, int c) { return r * kStride + c + 16 * (r >> 5); }
__device__ __forceinline__ int cm_addr(int c, int kr) {
    return c * kStride + (kr ^ (16 * ((c >> 5) & 1)));
}

// Operand table of the twiddled blocks j = 1..7, half h, lane (grouped
// outputs k; output k, input i of block j is W128^(k (j + 8 i)), forward).
constexpr int kOps = 7 * 2 * 64;  // u32x4 entries (14 KB)
__device__ __forceinline__ int op_index(int j, int h, int lane) { return ((j - 1) * 2 + h) * 64 + lane; }

// Entry e of the table, from the positive-angle table of length 128 (the
// forward sign is its conjugate).  Row m of half h is output k = 4 (m / 4) +
// 2 h + (m % 4) / 2, part (m % 4) % 2; column kk is input kk / 2, part kk % 2.
__device__ __forceinline__ u32x4 op_entry(int e, const float2* __restrict__ tw128) {
    const int lane = e & 63, h = (e >> 6) & 1, j = (e >> 7) + 1;
    const int m = lane & 15, kq = lane >> 4;
    const int o = m & 1;
    const int k = 4 * (m >> 2) + 2 * h + ((m & 3) >> 1);
    f16x8 r;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        const int kk = 8 * kq + x;
        const int in = kk >> 1, p = kk & 1;
        const float2 w = tw128[(k * (j + 8 * in)) & 127];
        const float c = w.x, sn = -w.y;
        // out.re = c*in.re - s*in.im ; out.im = s*in.re + c*in.im
        const float v = o == 0 ? (p == 0 ? c : -sn) : (p == 0 ? sn : c);
        r[x] = static_cast<_Float16>(v);
    }
    return __builtin_bit_cast(u32x4, r);
}

// DFT8 over the block index of v[b][t] for every t (in-lane), forward.
__device__ __forceinline__ void dft8_blocks(cpx (&v)[8][4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        cpx u[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) u[b] = v[b][t];
        Dft<8, true>::run(u);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k][t] = u[k];
    }
}

// One 128-point stage over the 16 sequences of the lane's column n: block b
// reads its inputs 4 q + e through addr(b, e).
template <class Addr>
__device__ __forceinline__ void stage128(const unsigned* src, Addr addr, const f16x8 (&ag)[2],
                                         const u32x4* ops, int lane, cpx (&v)[8][4]) {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        u32x4 xv;
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = src[addr(b, e)];
        f16x8 op[2];
        if (b == 0) {
            op[0] = ag[0];
            op[1] = ag[1];
        } else {
            op[0] = __builtin_bit_cast(f16x8, ops[op_index(b, 0, lane)]);
            op[1] = __builtin_bit_cast(f16x8, ops[op_index(b, 1, lane)]);
        }
        dft16_block(op, as_f16x8(xv), v[b]);
    }
    dft8_blocks(v);
}

// The 2-D forward transform of the values staged in `in` (rm_addr layout)
// through the exchange buffer `fx` -> v[kc0][t] = S[16 w + n][4 q + t + 16 kc0].
// `fx` is written with no barrier before: its previous readers must have
// passed one.  Ends after the F2 reads (fx still being read by other waves).
__device__ __forceinline__ void forward(const unsigned* in, unsigned* fx, const f16x8 (&ag)[2],
                                        const u32x4* ops, int wave, int lane, cpx (&v)[8][4]) {
    const int n = lane & 15, q = lane >> 4;
    const int c = 16 * wave + n;
    stage128(in, [&](int b, int e) { return rm_addr(b + 32 * q + 8 * e, c); }, ag, ops, lane, v);
#pragma unroll
    for (int k = 0; k < 8; ++k)
        *reinterpret_cast<u32x4*>(fx + cm_addr(c, 4 * q + 16 * k)) =
            u32x4{pack_half2(v[k][0]), pack_half2(v[k][1]), pack_half2(v[k][2]), pack_half2(v[k][3])};
    __syncthreads();
    stage128(fx, [&](int b, int e) { return cm_addr(b + 32 * q + 8 * e, c); }, ag, ops, lane, v);
}

// conj(v) of the lane's row 16 w + n into `buf` (rm_addr layout): columns
// 4 q + t + 16 k, one 16-byte chunk per k.
__device__ __forceinline__ void put_rows_conj(unsigned* buf, const cpx (&v)[8][4], int wave,
                                              int lane) {
    const int n = lane & 15, q = lane >> 4;
#pragma unroll
    for (int k = 0; k < 8; ++k)
        *reinterpret_cast<u32x4*>(buf + rm_addr(16 * wave + n, 4 * q + 16 * k)) =
            u32x4{pack_half2({v[k][0].re, -v[k][0].im}), pack_half2({v[k][1].re, -v[k][1].im}),
                  pack_half2({v[k][2].re, -v[k][2].im}), pack_half2({v[k][3].re, -v[k][3].im})};
}
}  // namespace conv2dm128

template <int kPerCu = 1>  // workgroups per CU (the LDS allows one)
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2 * kPerCu))) void
conv2d128_mfma_kernel(const __half2* __restrict__ x, const __half2* __restrict__ h,
                      __half2* __restrict__ y, int batch, const float2* __restrict__ tw128,
                      int tiles_per_block) {
    using namespace conv2dm128;
    constexpr int kImg = 128 * 128;
    __shared__ __align__(16) unsigned buf[2][kBuf];
    __shared__ u32x4 ops[kOps];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;

    f16x8 ag[2];
    dft16_operands_grouped<true>(ag, lane);
    for (int e = tid; e < kOps; e += 512) ops[e] = op_entry(e, tw128);  // read after a barrier below

    long long img, img_end, step;
    tile_walk(batch, tiles_per_block, img, img_end, step);
    if (img >= img_end) return;  // uniform over the workgroup

    // An image's 16-byte pieces 4 tid + 2048 i (rows (4 tid + 2048 i) / 128).
    auto load = [&](const __half2* src, u32x4 (&raw)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            raw[i] = ld_nt(reinterpret_cast<const u32x4*>(src + 4 * tid + 2048 * i));
    };
    auto stage = [&](unsigned* dst, const u32x4 (&raw)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = 4 * tid + 2048 * i;
            *reinterpret_cast<u32x4*>(dst + rm_addr(f >> 7, f & 127)) = raw[i];
        }
    };

    // The filter's spectrum / 16384 in the spectrum layout (buf[0] staging,
    // buf[1] exchange; the first image then stages into buf[0], whose last
    // readers passed the barrier inside forward).
    cpx hs[8][4];
    u32x4 next[8];
    load(h, next);
    stage(buf[0], next);
    load(x + img * kImg, next);
    __syncthreads();
    forward(buf[0], buf[1], ag, ops, wave, lane, hs);
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t)
            hs[k][t] = {hs[k][t].re * (1.0f / kImg), hs[k][t].im * (1.0f / kImg)};

    int s = 0;  // this image's staging buffer; the other is its exchange buffer
    for (; img < img_end; img += step, s ^= 1) {
        unsigned* const X = buf[s];
        unsigned* const Y = buf[s ^ 1];
        // X's last readers (the previous image's F1) passed a barrier since;
        // Y's (its stores) pass the one after this staging.
        stage(X, next);
        if (img + step < img_end) load(x + (img + step) * kImg, next);
        __syncthreads();
        cpx v[8][4];
        forward(X, Y, ag, ops, wave, lane, v);
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[k][t] = cmul(v[k][t], hs[k][t]);
        put_rows_conj(X, v, wave, lane);  // X's readers (F1) passed forward's barrier
        __syncthreads();
        forward(X, Y, ag, ops, wave, lane, v);  // Y's readers (F2) passed the last barrier
        put_rows_conj(X, v, wave, lane);
        __syncthreads();
        __half2* dst = y + img * kImg;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = 4 * tid + 2048 * i;
            st_nt(reinterpret_cast<u32x4*>(dst + f),
                  *reinterpret_cast<const u32x4*>(X + rm_addr(f >> 7, f & 127)));
        }
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// The fused column pass of the 1024 x 1024 half2 convolution on MFMA: for
// each of a unit's 16 adjacent columns, IFFT_col(FFT_col(y) * H) with the
// two-stage N = 1024 transform of c2c_mfma_kernel (conv2d_cols_kernel's
// contract with conv = true; H is the fp32 filter spectrum, 1/2^20 folded
// in, read once per workgroup).  One 512-lane workgroup per CU, 8 waves of
// two columns each:
//   load:  the unit's 1024 rows as 64-byte row pieces (16 rows per wave
//          instruction; lane l of half h takes piece 2h + ((l & 31) >> 4) of
//          row 16 (8 i + w) + (l & 15));
//   stage: each piece's four half2 go to the four columns' slots at the
//          transform's input positions (MfmaPlan<4>::in_pad).  Slots are
//          kSlot = 1284 dwords apart (4 mod 32): the pieces 2h and 2h + 1 of
//          16 consecutive rows that one half-wave writes fall on 32 banks;
//   per column: stage 1 from the slot, steps 2-6 (their wave-local
//          transposes in a 256-byte-aligned window of the slot), the product
//          with H's column (fp32 registers, the forward's output layout),
//          the inverse as conj(DFT(conj(P))) from the registers, and the
//          result into the slot at the output positions (out_pad);
//   store: the four columns of each row piece back together, 16 bytes.
// The workgroups walk the units grid-stride with the grid a multiple of the
// image's 64 column blocks, so each keeps one block (and its H columns) for
// every image; blocks that share a 128-byte line are renamed onto one XCD
// as in conv2d_cols_kernel.  The next unit's pieces are loaded while the
// current unit is transformed (250 VGPRs, 96.5 KB of LDS).  Measured on
// MI355X, 32 images end to end: 214.8 us against 249.7 us with the VALU
// column pass; without the prefetch 224.6 us; 16 waves of one column each
// (4 per SIMD, 128 VGPRs, no room for the prefetch) 224.4 us.  The f16
// roundings of the two transforms take the convolution's rel L2 against the
// fp64 direct convolution from 5.3e-4 to 7.0e-4.
// ---------------------------------------------------------------------------
namespace conv2dcolsm {
inline constexpr int kCols = 16;
inline constexpr int kRows = 1024;
inline constexpr int kImgCols = 1024;
inline constexpr int kSlot = 1284;
static_assert(MfmaPlan<4>::kRegion <= kSlot, "a slot holds the transform's staging region");
static_assert(1024 + 60 <= kSlot, "a slot holds a 256-byte-aligned transpose window");
}  // namespace conv2dcolsm

template <int kUnused = 0>  // a template: the header is compiled into several objects
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void
conv2d_cols_mfma_kernel(const __half2* in, __half2* out, const float2* __restrict__ H,
                        long long units, const float2* __restrict__ tw) {
    using namespace conv2dcolsm;
    using P = MfmaPlan<4>;
    constexpr int kWaves = 8;
    constexpr int kLanes = 64 * kWaves;
    constexpr int kSteps = kRows * (kCols / 4) / kLanes;  // 16-byte pieces per lane
    constexpr int kRowStep = 16 * kWaves;                 // rows between a lane's pieces
    constexpr int kCPW = kCols / kWaves;                  // columns per wave
    __shared__ __align__(256) unsigned blk[kCols * kSlot];
    __shared__ cpx w1[P::kTw1];
    __shared__ u32x4 a3[P::kA3];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;

    f16x8 a[2], a_regs[2];
    mfma_setup<4, true, kLanes>(a, w1, a3, nullptr, tw);
    dft16_operands<true, true>(a_regs, lane);
    const Stage3Folded s3{a, a3, lane};

    // This lane's row pieces: piece p of rows row0 + kRowStep i.
    const int p = 2 * (lane >> 5) + ((lane & 31) >> 4);
    const int row0 = 16 * wave + (lane & 15);

    constexpr long long blocks_per_image = kImgCols / kCols;
    constexpr int kShare = 2;  // 64-byte pieces: two column blocks per 128-byte line
    constexpr int kGroup = 8 * kShare;
    static_assert(blocks_per_image % kGroup == 0, "column blocks per image: whole groups");
    auto where = [&](long long u0, long long& base, int& c0) {
        const int i = static_cast<int>(u0 % kGroup);
        const long long u = u0 - i + kShare * (i % 8) + i / 8;
        const long long img = u / blocks_per_image;
        c0 = static_cast<int>(u - img * blocks_per_image) * kCols;
        base = img * kRows * static_cast<long long>(kImgCols) + c0;
    };
    long long u = blockIdx.x;
    if (u >= units) return;  // uniform over the workgroup

    int h_c0 = -1;
    cpx hs[kCPW][4][4];  // H of the wave's columns, bin n + 16 m + 64 (q + 4 r)
    auto load = [&](long long b, u32x4 (&raw)[kSteps]) {
#pragma unroll
        for (int i = 0; i < kSteps; ++i)
            raw[i] = ld_nt(reinterpret_cast<const u32x4*>(
                in + b + static_cast<long long>(row0 + kRowStep * i) * kImgCols + 4 * p));
    };
    long long base;
    int c0;
    where(u, base, c0);
    u32x4 raw[kSteps];
    load(base, raw);  // the next unit's pieces are loaded during the current unit
    {
        // kSteps stores to a resource of no bytes (dropped by the range
        // check): the loop is then entered, like every later pass, with the
        // pieces followed by kSteps stores in flight, so the compiler's count
        // at the staging waits for the pieces only, not for the previous
        // unit's stores.  (The size is a run-time value, units >= 0 always,
        // so the stores are not deleted.)
        const __amdgpu_buffer_rsrc_t none =
            __builtin_amdgcn_make_buffer_rsrc(out, 0, units < 0 ? 16 : 0, 0x00020000);
        __builtin_amdgcn_sched_barrier(0);  // after the loads, as in the loop
#pragma unroll
        for (int i = 0; i < kSteps; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{}, none, 16 * i, 0, 2);
    }
    for (; u < units; u += gridDim.x) {
        if (c0 != h_c0) {  // uniform: this workgroup's column block changed
#pragma unroll
            for (int cv = 0; cv < kCPW; ++cv)
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int k = n + 16 * m + 64 * (q + 4 * r);
                        const float2 hk = H[static_cast<long long>(k) * kImgCols + c0 + wave + kWaves * cv];
                        hs[cv][m][r] = cpx{hk.x, hk.y};
                    }
            wait_vmem_all();  // here, on this rarely taken path (not after the branch)
            h_c0 = c0;
        }
        __syncthreads();  // the previous unit's store reads of the slots are done
#pragma unroll
        for (int i = 0; i < kSteps; ++i) {
            const int pos = P::in_pad(row0 + kRowStep * i);
            const unsigned w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) blk[(4 * p + c) * kSlot + pos] = w[c];
        }
        const long long cur = base;
        if (u + gridDim.x < units) {
            where(u + gridDim.x, base, c0);
            load(base, raw);
        }
        __syncthreads();
#pragma unroll
        for (int cv = 0; cv < kCPW; ++cv) {
            const int col = wave + kWaves * cv;
            unsigned* const slot = blk + col * kSlot;
            // the transposes' window: the slot's first 256-byte boundary
            unsigned* const win = slot + ((64 - (col * kSlot) % 64) % 64);
            cpx v[4][4];
            mfma_stage1_lds<4>(slot, a, lane, v);
            mfma_steps2to6<4, true>(win, w1, s3, lane, v);
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[m][r] = cmul(v[m][r], hs[cv][m][r]);
            mfma_stage1_regs<4, true>(a_regs, v);
            mfma_steps2to6<4, true>(win, w1, s3, lane, v);
            wave_lds_sync();
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    slot[P::out_pad(n + 16 * m + 64 * (q + 4 * r))] =
                        pack_half2({v[m][r].re, -v[m][r].im});
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kSteps; ++i) {
            const int pos = P::out_pad(row0 + kRowStep * i);
            u32x4 w;
#pragma unroll
            for (int c = 0; c < 4; ++c) w[c] = blk[(4 * p + c) * kSlot + pos];
            st_nt(reinterpret_cast<u32x4*>(out + cur + static_cast<long long>(row0 + kRowStep * i) * kImgCols +
                                           4 * p),
                  w);
        }
    }
}

}  // namespace thff
