// fft_mfma.hpp -- half2 batched C2C FFT with the radix-16 stages on MFMA.
//
// Same contract as c2c_kernel (fft_c2c.hpp) for __half2 storage: natural-order
// signals of N complex values at in[b*N] / out[b*N], unnormalized, partial last
// tile masked.  The reference runs its FP16 path on tensor cores with FP16
// accumulation (include/thunderfft/detail/kernel/unit_kernel_fp16.cuh:123-134);
// here the 16-point DFTs run as v_mfma_f32_16x16x32_f16 with FP32
// accumulation, everything between them in FP32.
//
// One DFT16 over 16 sequences is D(32 x 16) = F(32 x 32) * X(32 x 16) in real
// form: column n of X holds one sequence's 16 complex inputs as 32 reals
// (re, im interleaved -- exactly the __half2 storage order), row 2k+o of F
// gives real (o=0) or imaginary (o=1) part of output k.  F is split into two
// 16-row halves (two MFMAs), and each half into F_hi + F_lo (both f16, F_lo =
// f16(F - F_hi)) so the coefficients are exact to ~2^-22; the data operand
// is f16 as stored (stage 1) or rounded once to f16 (stage 2).
//
// MFMA operand layouts on gfx950 (v_mfma_f32_16x16x32_f16, checked on the
// device): A[m][k] in lane m + 16*(k/8), element k%8; B[k][n] in lane
// n + 16*(k/8), element k%8; D[m][n] in lane n + 16*(m/4), element m%4.
// With the data as B, lane l = n + 16*q holds inputs 4q..4q+3 of sequence n
// and receives outputs 4q+i..; the rows of F are permuted so that lane group
// q receives outputs k = q + 4r, r = 0..3 (r = 2*half + i/2, o = i%2).
//
// N = 1024 = 16 x 64, one wave per transform (x[t + 64 j], t < 64, j < 16):
//   1. DFT16 over j for the 64 sequences t = 16c + n (c = column block 0..3)
//      -> y[c][r] = Y_t[k1], k1 = q + 4r                      (16 MFMAs)
//   2. y *= W_1024^(t*k1)                                     (per-lane constants)
//   3. DFT4 over c (in-lane)  -> z[m][r], m < 4                (VALU)
//   4. z *= W_64^(n*m)                                        (per-lane constants)
//   5. LDS transpose (f16, swizzled, conflict-free) so that lane
//      l' = k1 + 16 q' holds inputs n = 4q'..4q'+3 of sequence (k1, m) in
//      column block m
//   6. DFT16 over n -> X[k1 + 16 m + 64 (q' + 4 r')]            (16 MFMAs)
// Global I/O goes through LDS so that every access is a 16-byte
// non-temporal load or store.
#pragma once

#include "fft_core.hpp"

namespace thff {

using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// A-operand registers of the DFT16 matrix for this lane: [half][hi/lo].
// Row m of half h is output k = m/4 + 4*(2h + (m%4)/2), part (m%4)%2;
// column k' is input j = k'/2, part k'%2.
template <bool FWD>
__device__ __forceinline__ void dft16_operands(f16x8 (&a)[2][2], int lane) {
    const int m = lane & 15, q = lane >> 4;
    const int gq = m >> 2, i = m & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = gq + 4 * (2 * h + (i >> 1));
        const int o = i & 1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int kk = 8 * q + e;
            const int j = kk >> 1, p = kk & 1;
            const int ang = (j * k) & 15;
            const float c = kCos16[ang];
            const float s = FWD ? -kSin16[ang] : kSin16[ang];
            // out.re = c*in.re - s*in.im ; out.im = s*in.re + c*in.im
            const float v = o == 0 ? (p == 0 ? c : -s) : (p == 0 ? s : c);
            const _Float16 hi = static_cast<_Float16>(v);
            a[h][0][e] = hi;
            a[h][1][e] = static_cast<_Float16>(v - static_cast<float>(hi));
        }
    }
}

// Outputs r = 0..3 (k = q + 4r) of one 16-sequence DFT16 block, as complex f32.
__device__ __forceinline__ void dft16_block(const f16x8 (&a)[2][2], f16x8 b, cpx* y) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        d = mfma16x16x32(a[h][0], b, d);
        d = mfma16x16x32(a[h][1], b, d);
        y[2 * h] = {d[0], d[1]};
        y[2 * h + 1] = {d[2], d[3]};
    }
}

__device__ __forceinline__ unsigned pack_half2(cpx v) {
    return __builtin_bit_cast(unsigned, __floats2half2_rn(v.re, v.im));
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 w) { return __builtin_bit_cast(f16x8, w); }

struct MfmaPlan1024 {
    static constexpr int N = 1024;
    static constexpr int kFPB = 4;          // transforms per tile (one per wave)
    static constexpr int kTile = 4096;      // complex values per tile
    static constexpr int kRegion = 1280;    // LDS dwords per wave
    static constexpr int kTw1 = 16 * 64;    // step-2 twiddles, [c][r][lane]
};

// Padded LDS positions (in half2 units) of the staging layouts.
__device__ __forceinline__ int in_pad(int k) { return k + 4 * (k >> 6); }
__device__ __forceinline__ int out_pad(int k) { return k + 16 * (k >> 6); }

template <bool FWD, bool kPrefetch>
__global__ __launch_bounds__(256) void c2c_mfma1024_kernel(const __half2* __restrict__ in,
                                                           __half2* __restrict__ out, int batch,
                                                           const float2* __restrict__ tw,
                                                           int tiles_per_block) {
    using P = MfmaPlan1024;
    __shared__ unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;

    f16x8 a[2][2];
    dft16_operands<FWD>(a, lane);
    // Step-2 twiddles W_1024^(t*k1), t = 16c + n, k1 = q + 4r, shared by the
    // four waves through LDS (wave c fills column block c), and step-4
    // twiddles W_64^(n*m) = W_1024^(16 n m); all from the positive-angle table.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float2 x = tw[((16 * wave + n) * (q + 4 * r)) & 1023];
        w1[(wave * 4 + r) * 64 + lane] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
    }
    cpx w2[3];
#pragma unroll
    for (int m = 1; m < 4; ++m) {
        const float2 x = tw[(16 * n * m) & 1023];
        w2[m - 1] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
    }
    __syncthreads();

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile = static_cast<long long>(blockIdx.x) * tiles_per_block;
    const long long tile_end = tile + tiles_per_block < ntiles ? tile + tiles_per_block : ntiles;
    if (tile >= tile_end) return;  // uniform over the workgroup

    // Each wave owns transform tile*4 + wave; it is valid or not as a whole.
    auto load = [&](u32x4 (&r)[4], long long tl) {
        const bool valid = tl * P::kFPB + wave < batch;
        const __half2* src = in + (tl * P::kFPB + wave) * P::N;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r[i] = valid ? ld_nt(reinterpret_cast<const u32x4*>(src + 4 * lane + 256 * i)) : u32x4{};
    };

    u32x4 next[4];
    if constexpr (kPrefetch) load(next, tile);
    for (; tile < tile_end; ++tile) {
        u32x4 cur[4];
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = next[i];
            if (tile + 1 < tile_end) load(next, tile + 1);
        } else {
            load(cur, tile);
        }

        // ---- stage the transform in LDS (natural order, 4 dwords pad per 64) ----
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4*>(region + in_pad(4 * lane + 256 * i)) = cur[i];
        wave_lds_sync();

        // ---- step 1: DFT16 over j of x[t + 64 j], t = 16c + n ----
        cpx y[4][4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            u32x4 b;
#pragma unroll
            for (int e = 0; e < 4; ++e) b[e] = region[in_pad(16 * c + n + 64 * (4 * q + e))];
            dft16_block(a, as_f16x8(b), y[c]);
        }
        // ---- steps 2-4: twiddle, DFT4 over c, twiddle ----
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cpx v[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = cmul(y[c][r], w1[(c * 4 + r) * 64 + lane]);
            Dft<4, FWD>::run(v);
            y[0][r] = v[0];
#pragma unroll
            for (int m = 1; m < 4; ++m) y[m][r] = cmul(v[m], w2[m - 1]);
        }
        // ---- step 5: transpose to (column block m, column k1, rows n) ----
        // Row R = 16 m + k1 holds the 16 inputs n of sequence (k1, m); its
        // 4-value chunks are rotated by k1/4 so reads and writes are
        // bank-conflict free.
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int k1 = q + 4 * r;
                region[(16 * m + k1) * 16 + 4 * (((n >> 2) + r) & 3) + (n & 3)] = pack_half2(y[m][r]);
            }
        wave_lds_sync();
        // ---- step 6: DFT16 over n ----
        cpx z[4][4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const u32x4 b = *reinterpret_cast<const u32x4*>(
                region + (16 * m + n) * 16 + 4 * ((q + (n >> 2)) & 3));
            dft16_block(a, as_f16x8(b), z[m]);
        }
        // ---- store: lane (n = k1, q) holds X[k1 + 16 m + 64 (q + 4 r)] ----
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[out_pad(n + 16 * m + 64 * (q + 4 * r))] = pack_half2(z[m][r]);
        wave_lds_sync();
        if (tile * P::kFPB + wave < batch) {
            __half2* dst = out + (tile * P::kFPB + wave) * P::N;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st_nt(reinterpret_cast<u32x4*>(dst + 4 * lane + 256 * i),
                      *reinterpret_cast<const u32x4*>(region + out_pad(4 * lane + 256 * i)));
        }
    }
}

}  // namespace thff
