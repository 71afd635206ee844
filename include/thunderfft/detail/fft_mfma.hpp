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
// 16-row halves (two MFMAs).  Its coefficients are rounded to f16 (relative
// error <= 2^-12, the same size as the f16 rounding of the data between the
// stages); the data operand is f16 as stored (stage 1) or rounded once to f16
// (stage 2).  Measured at N = 1024 on MI355X: relative L2 3.2e-4 against the
// fp32 kernel, against 2.9e-4 when each coefficient also carries an f16
// correction term (twice the MFMAs, 2-6% slower end to end).
//
// MFMA operand layouts on gfx950 (v_mfma_f32_16x16x32_f16, checked on the
// device): A[m][k] in lane m + 16*(k/8), element k%8; B[k][n] in lane
// n + 16*(k/8), element k%8; D[m][n] in lane n + 16*(m/4), element m%4.
// With the data as B, lane l = n + 16*q holds inputs 4q..4q+3 of sequence n
// and receives outputs 4q+i..; the rows of F are permuted so that lane group
// q receives outputs k = q + 4r, r = 0..3 (r = 2*half + i/2, o = i%2).
//
// The kernel below handles N = 256*C = 16 x (C x 16) for C in {1, 2, 4, 8};
// for N = 1024 (C = 4) = 16 x 64, one wave per transform (x[t + 64 j], t < 64, j < 16):
//   1. DFT16 over j for the 64 sequences t = 16c + n (c = column block 0..3)
//      -> y[c][r] = Y_t[k1], k1 = q + 4r                      (8 MFMAs)
//   2. y *= W_1024^(t*k1)                                     (per-lane constants)
//   3. DFT4 over c (in-lane)  -> z[m][r], m < 4                (VALU)
//   4. z *= W_64^(n*m)                                        (per-lane constants)
//   5. LDS transpose (f16, swizzled, conflict-free) so that lane
//      l' = k1 + 16 q' holds inputs n = 4q'..4q'+3 of sequence (k1, m) in
//      column block m
//   6. DFT16 over n -> X[k1 + 16 m + 64 (q' + 4 r')]            (8 MFMAs)
// Global I/O goes through LDS so that every access is a 16-byte
// non-temporal load or store.
#pragma once

#include "fft_core.hpp"
#include "fft_tile.hpp"

namespace thff {

using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// A-operand registers of the DFT16 matrix for this lane: [half].
// Row m of half h is output k = m/4 + 4*(2h + (m%4)/2), part (m%4)%2;
// column k' is input j = k'/2, part k'%2.
// With kInterleaved, lane group q of the data operand holds inputs
// j = q + 4 e (e = 0..3) instead of 4 q + e: the columns are permuted to match,
// so a transform can consume another transform's output registers (whose
// lane group q holds outputs q + 4 r) without moving them.
template <bool FWD, bool kInterleaved = false>
__device__ __forceinline__ void dft16_operands(f16x8 (&a)[2], int lane) {
    const int m = lane & 15, q = lane >> 4;
    const int gq = m >> 2, i = m & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = gq + 4 * (2 * h + (i >> 1));
        const int o = i & 1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int kk = 8 * q + e;
            const int j = kInterleaved ? (kk >> 3) + 4 * ((kk >> 1) & 3) : kk >> 1;
            const int p = kk & 1;
            const int ang = (j * k) & 15;
            const float c = kCos16[ang];
            const float s = FWD ? -kSin16[ang] : kSin16[ang];
            // out.re = c*in.re - s*in.im ; out.im = s*in.re + c*in.im
            const float v = o == 0 ? (p == 0 ? c : -s) : (p == 0 ? s : c);
            a[h][e] = static_cast<_Float16>(v);
        }
    }
}

// The DFT16 operands of dft16_operands<FWD> (plain input order) with the
// rows permuted so that lane group q receives outputs k = 4q + r, r = 0..3
// (four consecutive outputs) instead of q + 4r: row m of half h is output
// k = 4 (m / 4) + 2 h + (m % 4) / 2, part (m % 4) % 2.  dft16_block then
// leaves output 4q + r in y[r].
template <bool FWD>
__device__ __forceinline__ void dft16_operands_grouped(f16x8 (&a)[2], int lane) {
    const int m = lane & 15, q = lane >> 4;
    const int gq = m >> 2, i = m & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = 4 * gq + 2 * h + (i >> 1);
        const int o = i & 1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int kk = 8 * q + e;
            const int j = kk >> 1, p = kk & 1;
            const int ang = (j * k) & 15;
            const float c = kCos16[ang];
            const float s = FWD ? -kSin16[ang] : kSin16[ang];
            const float v = o == 0 ? (p == 0 ? c : -s) : (p == 0 ? s : c);
            a[h][e] = static_cast<_Float16>(v);
        }
    }
}

// Outputs r = 0..3 (k = q + 4r) of one 16-sequence DFT16 block, as complex f32.
__device__ __forceinline__ void dft16_block(const f16x8 (&a)[2], f16x8 b, cpx* y) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const f32x4 d = mfma16x16x32(a[h], b, f32x4{0.f, 0.f, 0.f, 0.f});
        y[2 * h] = {d[0], d[1]};
        y[2 * h + 1] = {d[2], d[3]};
    }
}

__device__ __forceinline__ unsigned pack_half2(cpx v) {
    return __builtin_bit_cast(unsigned, __floats2half2_rn(v.re, v.im));
}

__device__ __forceinline__ cpx unpack_half2(unsigned w) {
    const float2 f = __half22float2(__builtin_bit_cast(__half2, w));
    return {f.x, f.y};
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 w) { return __builtin_bit_cast(f16x8, w); }

// Wave-local transpose between two DFT16 stages (dwords = half2 values):
// element i of sequence s of block b sits in 16-byte chunk 16 (i >> 2) +
// (s ^ 2 (i >> 2)) of the block's 64, at slot i & 3.  The reader lane (n, q)
// takes chunk q of sequence n (its inputs 4 q ... 4 q + 3): the 16 lanes of
// one q read the 16 chunks of one 256-byte row in XOR-permuted order, which
// measured conflict-free on MI355X (chunks 4 apart, as a row-per-sequence
// layout puts them, measured 2-way).  The writer lane (n, q) puts element n
// of sequence q + 4 r: over each 32-lane half the dword banks differ.
__device__ __forceinline__ int tpos(int b, int s, int i) {
    const int g = i >> 2;
    return 256 * b + 4 * ((s & 12) ^ (4 * (g >> 1))) + (64 * g + 4 * ((s & 3) ^ (2 * (g & 1))) + (i & 3));
}
__device__ __forceinline__ int tchunk(int b, int s, int g) {
    return 256 * b + 4 * (16 * g + (s ^ (2 * g)));
}

// Plan of the MFMA kernel for N = 256*C = 16 x (C x 16), C in {1, 2, 4, 8}.
template <int C>
struct MfmaPlan {
    static_assert(C == 1 || C == 2 || C == 4 || C == 8, "MFMA plan: C in {1, 2, 4, 8}");
    static constexpr int N = 256 * C;              // transform length
    static constexpr int kM = 16 * C;              // stride of the first DFT16's inputs (N/16)
    static constexpr int kBlocks = C < 4 ? 4 : C;  // 16-sequence MFMA blocks per wave
    static constexpr int kFPW = kBlocks / C;       // transforms per wave
    static constexpr int kVals = 4 * kBlocks;      // complex values per lane
    static constexpr int kWaveVals = 64 * kVals;   // values per wave (1024 or 2048)
    static constexpr int kFPB = 4 * kFPW;          // transforms per tile (4 waves)
    // LDS staging layouts (half2 units).  Input: pad kInPad after every
    // kInPeriod values, so the stride-16C first-stage reads of the 64 lanes
    // (n + 64C*q) hit 64 different banks.  Output: pad 16 after every C rows
    // of 16 (C >= 2), so the final writes (n + 16C*q) do too.
    static constexpr int kInPeriod = C <= 4 ? 64 : 128;
    static constexpr int kInPad = C <= 4 ? 16 / C : 4;
    static constexpr int kOutPeriod = 16 * C;
    static constexpr int kOutPad = C == 1 ? 0 : 16;
    static constexpr int kInSize = kWaveVals + kInPad * (kWaveVals / kInPeriod);
    static constexpr int kOutSize = kWaveVals + kOutPad * (kWaveVals / kOutPeriod);
    static constexpr int kRegion = kInSize > kOutSize ? kInSize : kOutSize;  // dwords per wave
    static constexpr int kTw1 = C * 4 * 64;        // first twiddles, [c][r][lane]
    static constexpr int kA3 = (C > 1 ? C - 1 : 1) * 2 * 64;  // folded stage-3 operands (u32x4)
    __device__ static __forceinline__ int in_pad(int k) { return k + kInPad * (k / kInPeriod); }
    // Padded offsets of the 16-byte staging pieces e = 4 l + 256 i of lane l:
    // both pad periods divide 256, so piece i sits a constant step past piece 0.
    static constexpr int kInStep = 256 + kInPad * (256 / kInPeriod);
    static constexpr int kOutStep = 256 + kOutPad * (256 / kOutPeriod);
    static_assert(256 % kInPeriod == 0 && 256 % kOutPeriod == 0, "constant staging steps");
    __device__ static __forceinline__ int out_pad(int k) {
        return k + kOutPad * (k / kOutPeriod);
    }
};

// Half h of this lane's DFT16 A operand built from the positive-angle table
// tw of length N = 256 C, with input (column) j of the matrix scaled by
// W_16C^(j m): entry (k, j) is W_16^(j k) W_16C^(j m) = W_N^(16 j (k C + m)).
// m = 0 gives the plain DFT16 matrix (the table's values at multiples of N/16
// are the correctly rounded cos/sin, as the constants of dft16_operands).
// Row and column order as dft16_operands<FWD, false>.
template <bool FWD>
__device__ __forceinline__ f16x8 dft16_operand_twiddled(int lane, int h, int m, int C,
                                                        const float2* __restrict__ tw) {
    const int N = 256 * C;
    const int mr = lane & 15, q = lane >> 4;
    const int k = (mr >> 2) + 4 * (2 * h + ((mr & 3) >> 1));
    const int o = mr & 1;
    f16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int kk = 8 * q + e;
        const int j = kk >> 1, p = kk & 1;
        const float2 w = tw[(16 * j * (k * C + m)) & (N - 1)];
        const float c = w.x, sn = FWD ? -w.y : w.y;
        // out.re = c*in.re - s*in.im ; out.im = s*in.re + c*in.im
        const float v = o == 0 ? (p == 0 ? c : -sn) : (p == 0 ? sn : c);
        r[e] = static_cast<_Float16>(v);
    }
    return r;
}

// Where steps 5-6 take the DFT16 operands of block column m (the DFT16 over n
// of the sequences (k1, m)) and how the twiddle W_16C^(n m) between the
// DFT_C and that DFT16 is applied.
//
// Stage3Folded: the twiddle is folded into the operands.  Column n of block
// column m's matrix is scaled by W_16C^(n m) (dft16_operand_twiddled), so no
// multiply remains between the DFT_C and the transpose; m = 0 uses the plain
// operands `a`, m >= 1 read theirs from the workgroup's LDS table
// a3[m - 1][half][lane] (mfma_setup).  The factor is rounded into the f16
// coefficient, the size of the f16 rounding of the data at that stage.
struct Stage3Folded {
    static constexpr bool kTwiddle = false;
    const f16x8* a;   // a[2]: plain operands
    const u32x4* a3;  // [(m - 1) * 2 + half] * 64 + lane
    int lane;
    __device__ __forceinline__ cpx twiddle(int, cpx v) const { return v; }
    __device__ __forceinline__ void operands(int m, f16x8 (&op)[2]) const {
        if (m == 0) {
            op[0] = a[0];
            op[1] = a[1];
        } else {
            op[0] = __builtin_bit_cast(f16x8, a3[((m - 1) * 2) * 64 + lane]);
            op[1] = __builtin_bit_cast(f16x8, a3[((m - 1) * 2 + 1) * 64 + lane]);
        }
    }
};

// Stage3Plain: plain operands for every block column and the fp32 twiddles
// w2[m - 1] = W_16C^(n m) in registers (conjugated at use with kConj), for
// callers without the workgroup set-up (the device-side API).
template <bool kConj>
struct Stage3Plain {
    static constexpr bool kTwiddle = true;
    const f16x8* a;
    const cpx* w2;
    __device__ __forceinline__ cpx twiddle(int m, cpx v) const {
        return kConj ? cmulc(v, w2[m - 1]) : cmul(v, w2[m - 1]);
    }
    __device__ __forceinline__ void operands(int, f16x8 (&op)[2]) const {
        op[0] = a[0];
        op[1] = a[1];
    }
};

// Workgroup set-up of the MFMA kernels for direction FWD, from the
// positive-angle table: this lane's plain DFT16 operands, the step-2 twiddles
// W_N^(t*k1) (t = 16c + n, k1 = q + 4r) shared through LDS as
// w1 = [c][r][lane], and for the stage before the last DFT16 either the
// folded operands a3 (Stage3Folded; a3 non-null) or this lane's twiddles
// w2[m - 1] = W_16C^(n m) (Stage3Plain; w2 non-null).  Collective over the
// kThreads-lane workgroup (ends with a barrier).
template <int C, bool FWD, int kThreads = 256>
__device__ __forceinline__ void mfma_setup(f16x8 (&a)[2], cpx* w1, u32x4* a3, cpx* w2,
                                           const float2* __restrict__ tw) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15;
    dft16_operands<FWD>(a, lane);
    for (int e = tid; e < P::kTw1; e += kThreads) {
        const int l = e & 63, r = (e >> 6) & 3, c = e >> 8;
        const float2 x = tw[((16 * c + (l & 15)) * ((l >> 4) + 4 * r)) & (N - 1)];
        w1[e] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
    }
    if constexpr (C > 1) {
        if (a3) {
            for (int e = tid; e < (C - 1) * 2 * 64; e += kThreads) {
                const int l = e & 63, h = (e >> 6) & 1, m = 1 + (e >> 7);
                a3[e] = __builtin_bit_cast(u32x4, dft16_operand_twiddled<FWD>(l, h, m, C, tw));
            }
        }
        if (w2) {
#pragma unroll
            for (int m = 1; m < C; ++m) {
                const float2 x = tw[(16 * n * m) & (N - 1)];
                w2[m - 1] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
            }
        }
    }
    __syncthreads();
}

// Step 1 from LDS: the kFPW transforms a wave has staged in `region` (natural
// order at MfmaPlan<C>::in_pad positions); block b = (f, c) gets the DFT16
// over j of x_f[16 c + n + 16C j] -> y[b][r] = Y[k1 = q + 4 r].
template <int C>
__device__ __forceinline__ void mfma_stage1_lds(const unsigned* region, const f16x8 (&a)[2],
                                                int lane, cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
    using P = MfmaPlan<C>;
    const int n = lane & 15, q = lane >> 4;
#pragma unroll
    for (int b = 0; b < P::kBlocks; ++b) {
        const int base = (b / C) * P::N + 16 * (b % C) + n;
        u32x4 x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = region[P::in_pad(base + P::kM * (4 * q + e))];
        dft16_block(a, as_f16x8(x), y[b]);
    }
}

// Step 1 from registers: y[b][r] holds z_f[16 c + n + 16C (q + 4 r)] (the
// layout a forward transform leaves), `a` built with kInterleaved.  With
// kConj the inputs are conjugated on the way in (folded into the f16 pack).
template <int C, bool kConj = false>
__device__ __forceinline__ void mfma_stage1_regs(const f16x8 (&a)[2],
                                                 cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
#pragma unroll
    for (int b = 0; b < MfmaPlan<C>::kBlocks; ++b) {
        u32x4 x;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            x[r] = pack_half2(kConj ? cpx{y[b][r].re, -y[b][r].im} : y[b][r]);
        dft16_block(a, as_f16x8(x), y[b]);
    }
}

// Steps 2-6 on the stage-1 outputs: twiddle, DFT_C over c, twiddle (S3),
// LDS transpose through `region` (overwritten), DFT16 over n with S3's
// operands.  The step-2 twiddles hold the direction TW_FWD; a transform of
// the other direction uses their conjugates.  On return lane (n = k1, q)
// holds, for block b = (f, m), y[b][r] = X_f[k1 + 16 m + 16C (q + 4 r)].
// `w1(c, r)` returns this lane's step-2 twiddle of block column c, output r.
template <int C, bool FWD, bool TW_FWD = FWD, class W1, class S3>
__device__ __forceinline__ void mfma_steps2to6_w(unsigned* region, W1 w1, const S3& s3, int lane,
                                                 cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
    using P = MfmaPlan<C>;
    constexpr int kB = P::kBlocks;
    constexpr bool kConj = FWD != TW_FWD;
    const int n = lane & 15, q = lane >> 4;
    // ---- steps 2-4: twiddle, DFT_C over c, twiddle ----
#pragma unroll
    for (int f = 0; f < P::kFPW; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cpx v[C];
#pragma unroll
            for (int c = 0; c < C; ++c) {
                const cpx w = w1(c, r);
                v[c] = kConj ? cmulc(y[f * C + c][r], w) : cmul(y[f * C + c][r], w);
            }
            Dft<C, FWD>::run(v);
            y[f * C][r] = v[0];
#pragma unroll
            for (int m = 1; m < C; ++m) y[f * C + m][r] = S3::kTwiddle ? s3.twiddle(m, v[m]) : v[m];
        }
    // ---- step 5: transpose: sequence (k1, m) of block b = (f, m) gets its
    // 16 inputs n (tpos: conflict-free writes and 16-byte reads) ----
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k1 = q + 4 * r;
            region[tpos(b, k1, n)] = pack_half2(y[b][r]);
        }
    wave_lds_sync();
    // ---- step 6: DFT16 over n ----
#pragma unroll
    for (int b = 0; b < kB; ++b) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(
            region + tchunk(b, n, q));
        f16x8 op[2];
        s3.operands(b % C, op);
        dft16_block(op, as_f16x8(x), y[b]);
    }
}

// Steps 2-6 with the step-2 twiddles in the workgroup's LDS table w1 = [c][r][lane].
template <int C, bool FWD, bool TW_FWD = FWD, class S3>
__device__ __forceinline__ void mfma_steps2to6(unsigned* region, const cpx* w1, const S3& s3,
                                               int lane, cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
    mfma_steps2to6_w<C, FWD, TW_FWD>(
        region, [&](int c, int r) { return w1[(c * 4 + r) * 64 + lane]; }, s3, lane, y);
}

// ---------------------------------------------------------------------------
// Steps 2-6 of the N = 2048 plan (C = 8, one transform per wave) with the
// DFT8 over c on the matrix cores instead of in-lane VALU butterflies.
//   2. y[c][r] *= w1(c, r), rounded to half2 (the multiply fused with the
//      rounding);
//   3. for each r, a 4 x 4 transpose of 8-byte chunks across the wave's four
//      16-lane rows (two v_permlane32_swap and two v_permlane16_swap per
//      dword): lane (n, q) then holds, for each j, inputs c = 2q, 2q + 1 of
//      the sequence (n, k1 = j + 4 r) -- the B operand of
//      v_mfma_f32_16x16x16_f16, whose 16 columns are the 16 n of one k1 and
//      whose A operand is the DFT8 matrix (dft8_mfma_operand); lane (n, q)
//      receives outputs m = 2q, 2q + 1 of its column;
//   4. (W_128^(n m) folded into S3's operands: S3 must be Stage3Folded);
//   5. the transpose of mfma_steps2to6 (tpos), with block m at 256 m +
//      4 floor((m + 2) / 4) (mfma8_block_base): the blocks do not overlap and
//      the two 16-lane rows of a half-wave, which write blocks 2q + i, are 4
//      dwords apart mod 8, so their dword writes fall on different banks;
//   6. DFT16 over n, as mfma_steps2to6.
// Forward direction only (the convolutions run their inverse as
// conj(DFT(conj(x)))).  The data is rounded to f16 once more than with the
// in-lane DFT8 (before the DFT8 instead of after it).
using f16x4 = _Float16 __attribute__((ext_vector_type(4)));

// Forward DFT8 A operand of v_mfma_f32_16x16x16_f16 for this lane: lane
// (i, q) holds A[i][4 q + e]; row i = 2 m + o is output m, part o; column
// 2 c + p is input c, part p.
__device__ __forceinline__ f16x4 dft8_mfma_operand(int lane) {
    const int i = lane & 15, q = lane >> 4;
    const int m = i >> 1, o = i & 1;
    f16x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int c = 2 * q + (e >> 1), p = e & 1;
        const int ang = (2 * m * c) & 15;  // W_8^(m c) = W_16^(2 m c)
        const float cs = kCos16[ang], sn = -kSin16[ang];
        r[e] = static_cast<_Float16>(o == 0 ? (p == 0 ? cs : -sn) : (p == 0 ? sn : cs));
    }
    return r;
}

// Offset of block b in the C = 8 step-5 layout, added to tpos / tchunk
// (0, 0, 4, 4, 4, 4, 8, 8 dwords; the region holds 2048 + 8).
__device__ __forceinline__ int mfma8_block_base(int b) { return 4 * ((b + 2) >> 2); }

template <class W1, class S3>
__device__ __forceinline__ void mfma8_steps2to6_dft8mfma(unsigned* region, W1 w1, const S3& s3,
                                                         f16x4 a8, int lane, cpx (&y)[8][4]) {
    static_assert(!S3::kTwiddle, "step 4 must be folded into the stage-3 operands");
    static_assert(MfmaPlan<8>::kRegion >= 2048 + 8, "region holds the shifted blocks");
    const int n = lane & 15, q = lane >> 4;
    f32x4 d[4][4];  // [r][j]: outputs m = 2q, 2q + 1 of the sequence (n, k1 = j + 4 r)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        unsigned pk[8];  // input c of the lane's sequence k1 = q + 4 r, half2
#pragma unroll
        for (int c = 0; c < 8; ++c) pk[c] = pack_half2(cmul(y[c][r], w1(c, r)));
        unsigned t[4][2];  // t[j][h]: dword h of the chunk for instance k1 = j + 4 r
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // chunk j (inputs 2j, 2j + 1) of row q goes to row j
            const auto s02 = __builtin_amdgcn_permlane32_swap(pk[h], pk[4 + h], false, false);
            const auto s13 = __builtin_amdgcn_permlane32_swap(pk[2 + h], pk[6 + h], false, false);
            const auto t01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
            const auto t23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
            t[0][h] = t01[0];
            t[1][h] = t01[1];
            t[2][h] = t23[0];
            t[3][h] = t23[1];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            d[r][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                a8, __builtin_bit_cast(f16x4, u32x2{t[j][0], t[j][1]}), f32x4{0.f, 0.f, 0.f, 0.f},
                0, 0, 0);
    }
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int m = 2 * q + i;
                region[mfma8_block_base(m) + tpos(m, j + 4 * r, n)] =
                    pack_half2(cpx{d[r][j][2 * i], d[r][j][2 * i + 1]});
            }
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(region + mfma8_block_base(b) + tchunk(b, n, q));
        f16x8 op[2];
        s3.operands(b, op);
        dft16_block(op, as_f16x8(x), y[b]);
    }
}

// Steps 1-6 for the kFPW transforms a wave has staged in `region`, with the
// workgroup set-up of mfma_setup and the stage-3 form S3.
template <int C, bool FWD, class S3>
__device__ __forceinline__ void mfma_fft_staged(unsigned* region, const f16x8 (&a)[2],
                                                const cpx* w1, const S3& s3, int lane,
                                                cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
    mfma_stage1_lds<C>(region, a, lane, y);
    mfma_steps2to6<C, FWD>(region, w1, s3, lane, y);
}

// The DFT16 operands of dft16_operands with the entries computed by cis_rev
// instead of read from the constant table (no memory access; the f16
// rounding of each entry dominates the transcendental's error).
template <bool FWD, bool kInterleaved = false>
__device__ __forceinline__ void dft16_operands_arith(f16x8 (&a)[2], int lane) {
    const int m = lane & 15, q = lane >> 4;
    const int gq = m >> 2, i = m & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = gq + 4 * (2 * h + (i >> 1));
        const int o = i & 1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int kk = 8 * q + e;
            const int j = kInterleaved ? (kk >> 3) + 4 * ((kk >> 1) & 3) : kk >> 1;
            const int p = kk & 1;
            const cpx cs = cis_rev(j * k, 16);
            const float c = cs.re, s = FWD ? -cs.im : cs.im;
            const float v = o == 0 ? (p == 0 ? c : -s) : (p == 0 ? s : c);
            a[h][e] = static_cast<_Float16>(v);
        }
    }
}

// Per-lane coefficients of one direction of the two-stage MFMA transform
// held in registers (mfma_fft_regs): the stage-1 operands for inputs in the
// transform's own output layout (a_in, column-permuted), the plain operands,
// the step-2 twiddles W_N^(t k1) (t = 16c + n, k1 = q + 4r) and the step-4
// twiddles W_16C^(n m), conjugated for the forward direction.  load() reads
// the twiddles from the ThunderFFTInitialize table; build() computes
// everything with cis_rev (the device API's precomputed fp16 coefficients).
template <int C>
struct MfmaCoeffs {
    static constexpr int N = 256 * C;
    f16x8 a_in[2], a[2];
    cpx w1[C * 4];
    cpx w2[C > 1 ? C - 1 : 1];
    // Uniform views for the device API's packed form: operand register i
    // (a_in, then a) and twiddle i (w1, then the w2 in use).
    static constexpr int kTwiddles = 4 * C + C - 1;
    __device__ __forceinline__ f16x8& op(int i) { return i < 2 ? a_in[i] : a[i - 2]; }
    __device__ __forceinline__ cpx& twiddle(int i) { return i < 4 * C ? w1[i] : w2[i - 4 * C]; }

    template <bool FWD, class Tw>
    __device__ __forceinline__ void fill(int lane, Tw tw_at) {
        const int n = lane & 15, q = lane >> 4;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const cpx x = tw_at((16 * c + n) * (q + 4 * r));
                w1[c * 4 + r] = FWD ? cpx{x.re, -x.im} : x;
            }
#pragma unroll
        for (int m = 1; m < C; ++m) {
            const cpx x = tw_at(16 * n * m);
            w2[m - 1] = FWD ? cpx{x.re, -x.im} : x;
        }
    }
    template <bool FWD>
    __device__ __forceinline__ void load(const float2* __restrict__ tw, int lane) {
        dft16_operands<FWD, true>(a_in, lane);
        dft16_operands<FWD>(a, lane);
        fill<FWD>(lane, [&](int k) {
            const float2 x = tw[k & (N - 1)];
            return cpx{x.x, x.y};
        });
    }
    template <bool FWD>
    __device__ __forceinline__ void build(int lane) {
        dft16_operands_arith<FWD, true>(a_in, lane);
        dft16_operands_arith<FWD>(a, lane);
        fill<FWD>(lane, [](int k) { return cis_rev(k, N); });
    }
};

// One MFMA transform of the kFPW transforms a wave holds in registers, for
// callers without the workgroup set-up (the device-side API): y[b][r] holds
// z_f[16 c + n + 16C (q + 4 r)] for block b = (f, c) on entry (the layout the
// transform leaves, so forward and inverse chain), and
// X_f[k1 + 16 m + 16C (q + 4 r)] for block b = (f, m), k1 = n, on return.
// `k` holds this direction's coefficients; `region` is the wave's LDS
// scratch (16 * kBlocks * 16 dwords), written after a wave-level sync.
template <int C, bool FWD>
__device__ __forceinline__ void mfma_fft_regs(unsigned* region, const MfmaCoeffs<C>& k, int lane,
                                              cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
    mfma_stage1_regs<C>(k.a_in, y);
    mfma_steps2to6_w<C, FWD>(
        region, [&](int c, int r) { return k.w1[c * 4 + r]; }, Stage3Plain<false>{k.a, k.w2}, lane,
        y);
}

// As above, the coefficients read from the positive-angle table `tw` of
// length N for this call.
template <int C, bool FWD>
__device__ __forceinline__ void mfma_fft_regs(unsigned* region, const float2* __restrict__ tw,
                                              int lane, cpx (&y)[MfmaPlan<C>::kBlocks][4]) {
    MfmaCoeffs<C> k;
    k.template load<FWD>(tw, lane);
    mfma_fft_regs<C, FWD>(region, k, lane, y);
}

// Batched C2C of half2 signals of N = 256*C on MFMA (C = 4 is N = 1024 as
// described at the top of this file; in general N = 16 x (C x 16)):
//   1. DFT16 over j of x[t + 16C j] for the 16C sequences t = 16c + n
//   2. twiddle W_N^(t*k1), k1 = q + 4r   3. DFT_C over c (in-lane)
//   4. twiddle W_16C^(n*m)               5. LDS transpose
//   6. DFT16 over n -> X[k1 + 16 m + 16C (q' + 4 r')]
// A wave owns 4/C transforms (C <= 4, 16 values per lane) or one (C = 8,
// 32 values per lane); a workgroup of 4 waves walks tiles of 4 waves' worth.
// C <= 4 is held to <= 128 VGPRs (4 waves per SIMD) without spilling.
template <int C>
inline constexpr int kMfmaMinWavesPerEU = C <= 4 ? 4 : 1;

template <int C, bool FWD, bool kPrefetch>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kMfmaMinWavesPerEU<C>))) void
c2c_mfma_kernel(const __half2* __restrict__ in,
                                                       __half2* __restrict__ out, int batch,
                                                       const float2* __restrict__ tw,
                                                       int tiles_per_block) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    constexpr int kB = P::kBlocks;
    constexpr int kRaw = P::kVals / 4;  // 16-byte loads per lane
    __shared__ unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;

    // The twiddle before the last DFT16 stays an fp32 multiply here: folding
    // it into LDS-held operands (as the convolutions do) measured slower for
    // the transform alone (compute pass 29.8 vs 27.8 us at N = 1024).
    f16x8 a[2];
    cpx w2[C > 1 ? C - 1 : 1];
    mfma_setup<C, FWD>(a, w1, nullptr, w2, tw);
    const Stage3Plain<false> s3{a, w2};

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
    if (tile >= tile_end) return;  // uniform over the workgroup

    // Valid values (0..kWaveVals) of this wave's kFPW transforms in tile tl.
    auto valid = [&](long long tl) {
        const long long v = (static_cast<long long>(batch) - tl * P::kFPB - wave * P::kFPW) * N;
        return v <= 0 ? 0 : (v >= P::kWaveVals ? P::kWaveVals : static_cast<int>(v));
    };
    auto load = [&](u32x4 (&r)[kRaw], long long tl) {
        const int nv = valid(tl);
        const __half2* src = in + (tl * P::kFPB + wave * P::kFPW) * N;
#pragma unroll
        for (int i = 0; i < kRaw; ++i) {
            const int e = 4 * lane + 256 * i;
            r[i] = e < nv ? ld_nt(reinterpret_cast<const u32x4*>(src + e)) : u32x4{};
        }
    };

    u32x4 next[kRaw];
    if constexpr (kPrefetch) load(next, tile);
    for (; tile < tile_end; tile += step) {
        u32x4 cur[kRaw];
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < kRaw; ++i) cur[i] = next[i];
            if (tile + step < tile_end) load(next, tile + step);
        } else {
            load(cur, tile);
        }

        // ---- stage the wave's transforms in LDS (natural order, padded) ----
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < kRaw; ++i)
            *reinterpret_cast<u32x4*>(region + P::in_pad(4 * lane + 256 * i)) = cur[i];
        wave_lds_sync();

        cpx y[kB][4];
        mfma_fft_staged<C, FWD>(region, a, w1, s3, lane, y);
        // ---- store: lane (n = k1, q), block (f, m) holds X_f[k1 + 16 m + 16C (q + 4 r)] ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < kB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::out_pad((b / C) * N + n + 16 * (b % C) + P::kM * (q + 4 * r))] =
                    pack_half2(y[b][r]);
        wave_lds_sync();
        const int nv = valid(tile);
        __half2* dst = out + (tile * P::kFPB + wave * P::kFPW) * N;
#pragma unroll
        for (int i = 0; i < kRaw; ++i) {
            const int e = 4 * lane + 256 * i;
            if (e < nv)
                st_nt(reinterpret_cast<u32x4*>(dst + e),
                      *reinterpret_cast<const u32x4*>(region + P::out_pad(e)));
        }
    }
}

}  // namespace thff

namespace thff {

// One-shot form of c2c_mfma_kernel: every wave moves one tile of kFPW
// transforms and exits, as a streaming copy does (the dispatcher then keeps
// the CUs evenly fed), with no LDS table and no workgroup barrier: the
// lane's DFT16 operands come from the constant table and its 16 + (C - 1)
// twiddles are computed with the hardware sine and cosine (cis_rev, accurate
// to far below the f16 rounding the data takes), so nothing but the data
// touches memory.  The wave's loads are issued before the coefficients are
// computed.  Grid: one 256-lane workgroup per four tiles.
template <int C, bool FWD, int kWaves = 4>
__global__ __launch_bounds__(64 * kWaves) void c2c_mfma_wave_kernel(const __half2* __restrict__ in,
                                                                    __half2* __restrict__ out,
                                                                    int batch) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    constexpr int kB = P::kBlocks;
    constexpr int kRaw = P::kVals / 4;
    __shared__ unsigned lds[kWaves * P::kRegion];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;
    const long long first = (static_cast<long long>(blockIdx.x) * kWaves + wave) * P::kFPW;  // transform
    const long long v = (static_cast<long long>(batch) - first) * N;
    const int nv = v <= 0 ? 0 : (v >= P::kWaveVals ? P::kWaveVals : static_cast<int>(v));
    if (nv == 0) return;  // uniform over the wave; no workgroup barrier follows
    const __half2* src = in + first * N;
    u32x4 cur[kRaw];
#pragma unroll
    for (int i = 0; i < kRaw; ++i) {
        const int e = 4 * lane + 256 * i;
        cur[i] = e < nv ? ld_nt(reinterpret_cast<const u32x4*>(src + e)) : u32x4{};
    }
    f16x8 a[2];
    dft16_operands<FWD>(a, lane);
    cpx w1[C * 4], w2[C > 1 ? C - 1 : 1];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const cpx x = cis_rev((16 * c + n) * (q + 4 * r), N);
            w1[c * 4 + r] = FWD ? cpx{x.re, -x.im} : x;
        }
#pragma unroll
    for (int m = 1; m < C; ++m) {
        const cpx x = cis_rev(16 * n * m, N);
        w2[m - 1] = FWD ? cpx{x.re, -x.im} : x;
    }
#pragma unroll
    for (int i = 0; i < kRaw; ++i)
        *reinterpret_cast<u32x4*>(region + P::in_pad(4 * lane + 256 * i)) = cur[i];
    wave_lds_sync();
    cpx y[kB][4];
    mfma_stage1_lds<C>(region, a, lane, y);
    mfma_steps2to6_w<C, FWD>(region, [&](int c, int r) { return w1[c * 4 + r]; },
                             Stage3Plain<false>{a, w2}, lane, y);
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            region[P::out_pad((b / C) * N + n + 16 * (b % C) + P::kM * (q + 4 * r))] = pack_half2(y[b][r]);
    wave_lds_sync();
    __half2* dst = out + first * N;
#pragma unroll
    for (int i = 0; i < kRaw; ++i) {
        const int e = 4 * lane + 256 * i;
        if (e < nv)
            st_nt(reinterpret_cast<u32x4*>(dst + e), *reinterpret_cast<const u32x4*>(region + P::out_pad(e)));
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// half2 C2C of N = 4096 = 16 x 16 x 16 on MFMA, one transform per workgroup
// tile (4 waves, 16 values per lane).  With n = t0 + 16 t1 + 256 j and
// k = k1 + 16 k2 + 256 k3 (all digits < 16), t = t0 + 16 t1:
//   1. DFT16 over j of x[t + 256 j] -> Y1[t][k1].  Wave w, lane (n, q),
//      block b: t = 64 w + 4 n + b, so the lane's four blocks read four
//      consecutive values: each of its inputs j = 4 q + e is one 16-byte load
//      straight from HBM (no staging).  Outputs k1 = q + 4 r.
//   2. Y1 *= W_4096^(t k1); workgroup exchange through LDS so that wave w'
//      block b' holds, for k1 = 4 w' + b', the 16 sequences t0 = n (inputs t1)
//   3. DFT16 over t1 -> Y2[k1][t0][k2], k2 = q + 4 r
//   4. Y2 *= W_256^(t0 k2); wave-local transpose (as in mfma_fft_staged)
//   5. DFT16 over t0 -> X[k1 + 16 k2 + 256 k3], k2 = n, k3 = q + 4 r
// LDS layouts (dwords = half2 values):
//   exchange: matrix k1 at 272 k1; (t0, t1) at 16 t0 + 4 (((t1 >> 2) + (t0 >> 2)) & 3)
//             + ((t1 + k1) & 3).  Writers (fixed b, r) have t0 = 4 (n & 3) + b,
//             t1 = 4 w + (n >> 2), k1 = q + 4 r: banks 16 (b + q) + 4 ((w + n) & 3)
//             + (((n >> 2) + q) & 3) mod 64, all different.
//   output staging: in 16-byte chunks, out_chunk (conflict-free 16-byte writes and reads).
// Three workgroup barriers per tile.  The data is rounded to f16 before stages
// 2 and 3, as in the two-stage kernel.
// ---------------------------------------------------------------------------
struct Mfma4096 {
    static constexpr int N = 4096;
    static constexpr int kMatrix = 272;             // exchange matrix stride (dwords)
    static constexpr int kExchange = 16 * kMatrix;  // 4352
    static constexpr int kOut = 4096;               // output staging (dwords)
    // Output staging: value k sits in slot k & 3 of the 16-byte chunk
    // out_chunk(k >> 2), chunk K at position K ^ ((K >> 4) & 3).  Lane (n, q)
    // of wave w writes its four blocks' values 4 w + b + 16 n + 256 k3
    // (b = 0..3) as one chunk K = w + 4 n + 64 k3; over 16 lanes of one
    // q the positions mod 16 are (w + 4 (n & 3)) ^ (n >> 2), all different.
    // Lane t reads the chunks t + 256 i, 16 consecutive chunks (same K >> 4)
    // per 16 lanes, also all different: both sides are conflict-free
    // 16-byte accesses.
    __device__ static __forceinline__ int out_chunk(int K) { return K ^ ((K >> 4) & 3); }
};

// Exchange element (k1, t0, t1) sits at 272 k1 + 16 t0 + 4 (((t1 >> 2) +
// (t0 >> 2)) & 3) + ((t1 + k1) & 3); for the inverse's writers (fixed b, r)
// the banks are 16 (b + q) + 4 (((n >> 2) + w) & 3) + (((n & 3) + q) & 3)
// mod 64, all different, as for the forward ones.
__device__ __forceinline__ int xaddr4096(int k1, int t0, int t1) {
    return Mfma4096::kMatrix * k1 + 16 * t0 + 4 * (((t1 >> 2) + (t0 >> 2)) & 3) + ((t1 + k1) & 3);
}

// Per-lane coefficients of one direction of mfma4096_fft_regs: plain and
// column-permuted DFT16 operands, the stage-1 -> 2 twiddles
// W^((4 w + b + 16 n)(q + 4 r)) and the stage-2 -> 3 twiddles W^(16 n (q + 4 r)),
// conjugated for the forward direction (tid: the lane's index in the
// 256-lane block).  load() from the table, build() with cis_rev.
struct Mfma4096Coeffs {
    static constexpr int N = 4096;
    f16x8 a[2], a_in[2];
    cpx w1[4][4], w2[4];
    static constexpr int kTwiddles = 20;
    __device__ __forceinline__ f16x8& op(int i) { return i < 2 ? a[i] : a_in[i - 2]; }
    __device__ __forceinline__ cpx& twiddle(int i) { return i < 16 ? w1[i >> 2][i & 3] : w2[i - 16]; }

    template <bool FWD, class Tw>
    __device__ __forceinline__ void fill(int tid, Tw tw_at) {
        const int wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const cpx x = tw_at((4 * wave + b + 16 * n) * (q + 4 * r));
                w1[b][r] = FWD ? cpx{x.re, -x.im} : x;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const cpx x = tw_at(16 * n * (q + 4 * r));
            w2[r] = FWD ? cpx{x.re, -x.im} : x;
        }
    }
    template <bool FWD>
    __device__ __forceinline__ void load(const float2* __restrict__ tw, int tid) {
        dft16_operands<FWD>(a, tid & 63);
        dft16_operands<FWD, true>(a_in, tid & 63);
        fill<FWD>(tid, [&](int k) {
            const float2 x = tw[k & (N - 1)];
            return cpx{x.x, x.y};
        });
    }
    template <bool FWD>
    __device__ __forceinline__ void build(int tid) {
        dft16_operands_arith<FWD>(a, tid & 63);
        dft16_operands_arith<FWD, true>(a_in, tid & 63);
        fill<FWD>(tid, [](int k) { return cis_rev(k, N); });
    }
};

// One N = 4096 transform per workgroup from registers, either direction, for
// callers without the kernel's set-up (the device-side API).  Lane (n, q) of
// wave w holds, in v[b][r], element 4 w + b + 16 n + 256 (q + 4 r) on entry
// and on return (the layout the three stages leave, so transforms chain):
// stage 1 over k3 = q + 4 r for the sequences t' = 4 w + b + 16 n
// (column-permuted operands), W^(t' k1), the workgroup exchange with
// t0 = 4 w + b, t1 = n, stage 2, W_256^(t0 k2), the wave-local transpose
// and stage 3.  xbuf: Mfma4096::kExchange dwords of LDS; two workgroup
// barriers, the first before xbuf is written.  `k` holds this direction's
// coefficients.
template <bool FWD>
__device__ __forceinline__ void mfma4096_fft_regs(unsigned* xbuf, const Mfma4096Coeffs& k, int tid,
                                                  cpx (&v)[4][4]) {
    using P = Mfma4096;
    const int wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
    unsigned* const region = xbuf + 4 * P::kMatrix * wave;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        u32x4 xv;
#pragma unroll
        for (int r = 0; r < 4; ++r) xv[r] = pack_half2(v[b][r]);
        dft16_block(k.a_in, as_f16x8(xv), v[b]);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[b][r] = cmul(v[b][r], k.w1[b][r]);
    }
    __syncthreads();  // every wave is done with xbuf
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) xbuf[xaddr4096(q + 4 * r, 4 * wave + b, n)] = pack_half2(v[b][r]);
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(
            region + P::kMatrix * b + 16 * n + 4 * ((q + (n >> 2)) & 3));
        u32x4 xv;  // t1 = 4 q + e sits at position (e + k1) & 3 = (e + b) & 3
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = raw[(e + b) & 3];
        dft16_block(k.a, as_f16x8(xv), v[b]);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[b][r] = cmul(v[b][r], k.w2[r]);
    }
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            region[tpos(b, q + 4 * r, n)] = pack_half2(v[b][r]);
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(
            region + tchunk(b, n, q));
        dft16_block(k.a, as_f16x8(xv), v[b]);
    }
}

// As above, the coefficients read from the positive-angle table `tw` of
// length 4096 for this call.
template <bool FWD>
__device__ __forceinline__ void mfma4096_fft_regs(unsigned* xbuf, const float2* __restrict__ tw,
                                                  int tid, cpx (&v)[4][4]) {
    Mfma4096Coeffs k;
    k.template load<FWD>(tw, tid);
    mfma4096_fft_regs<FWD>(xbuf, k, tid, v);
}

template <bool FWD, bool kPrefetch>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void c2c_mfma4096_kernel(
    const __half2* __restrict__ in, __half2* __restrict__ out, int batch,
    const float2* __restrict__ tw, int tiles_per_block) {
    using P = Mfma4096;
    constexpr int N = P::N;
    __shared__ __align__(16) unsigned xbuf[P::kExchange];
    __shared__ __align__(16) unsigned obuf[P::kOut];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* const region = xbuf + 4 * P::kMatrix * wave;  // matrices k1 = 4 wave ... + 3

    f16x8 a[2];
    dft16_operands<FWD>(a, lane);
    // Twiddles: W_4096^(t k1), t = 64 wave + 4 n + b, k1 = q + 4 r; W_4096^(16 n k2), k2 = q + 4 r.
    cpx w1[4][4], w2[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float2 x = tw[((64 * wave + 4 * n + b) * (q + 4 * r)) & (N - 1)];
            w1[b][r] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float2 x = tw[(16 * n * (q + 4 * r)) & (N - 1)];
        w2[r] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
    }

    // tiles_per_block = 0: the grid is sized to the device and walks the batch
    // grid-stride (tile_walk); otherwise contiguous runs of that many.
    long long tile, tile_end, step;
    tile_walk(batch, tiles_per_block, tile, tile_end, step);
    if (tile >= tile_end) return;  // uniform over the workgroup

    // Input j = 4 q + e of the lane's blocks b = 0..3: x[64 wave + 4 n + b + 256 j].
    auto load = [&](u32x4 (&r)[4], long long tl) {
        const __half2* src = in + tl * N + 64 * wave + 4 * n + 1024 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = ld_nt(reinterpret_cast<const u32x4*>(src + 256 * e));
    };

    u32x4 next[4];
    if constexpr (kPrefetch) load(next, tile);
    for (; tile < tile_end; tile += step) {
        u32x4 cur[4];
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = next[i];
            if (tile + step < tile_end) load(next, tile + step);
        } else {
            load(cur, tile);
        }

        // ---- stage 1: DFT16 over j, then W_4096^(t k1) ----
        cpx y[4][4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            u32x4 x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = cur[e][b];
            dft16_block(a, as_f16x8(x), y[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) y[b][r] = cmul(y[b][r], w1[b][r]);
        }
        __syncthreads();  // every wave is done with the previous tile's exchange buffer
        // ---- exchange: k1 = q + 4 r, t0 = 4 (n & 3) + b, t1 = 4 wave + (n >> 2) ----
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                xbuf[P::kMatrix * (q + 4 * r) + 16 * (4 * (n & 3) + b) +
                     4 * ((wave + (n & 3)) & 3) + (((n >> 2) + q) & 3)] = pack_half2(y[b][r]);
        __syncthreads();
        // ---- stage 2: block b holds k1 = 4 wave + b; lane (t0 = n, chunk q of t1) ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(
                region + P::kMatrix * b + 16 * n + 4 * ((q + (n >> 2)) & 3));
            u32x4 x;  // t1 = 4 q + e sits at position (e + k1) & 3 = (e + b) & 3
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = raw[(e + b) & 3];
            dft16_block(a, as_f16x8(x), y[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) y[b][r] = cmul(y[b][r], w2[r]);
        }
        // ---- wave-local transpose: sequence (b, k2) gets its 16 t0 (tpos) ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int k2 = q + 4 * r;
                region[tpos(b, k2, n)] = pack_half2(y[b][r]);
            }
        wave_lds_sync();
        // ---- stage 3: DFT16 over t0 -> X[k1 + 16 k2 + 256 k3], k2 = n, k3 = q + 4 r ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 x = *reinterpret_cast<const u32x4*>(
                region + tchunk(b, n, q));
            dft16_block(a, as_f16x8(x), y[b]);
        }
        __half2* dst = out + tile * N;
        {
            // obuf's previous reads ended before this tile's first barrier.  (Writing
            // the lane's 4 consecutive outputs straight to HBM instead leaves each
            // 64-byte segment to four waves and measured 4x slower.)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                reinterpret_cast<u32x4*>(obuf)[P::out_chunk(wave + 4 * n + 64 * (q + 4 * r))] =
                    u32x4{pack_half2(y[0][r]), pack_half2(y[1][r]), pack_half2(y[2][r]),
                          pack_half2(y[3][r])};
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st_nt(reinterpret_cast<u32x4*>(dst + 4 * tid + 1024 * i),
                      reinterpret_cast<const u32x4*>(obuf)[P::out_chunk(tid + 256 * i)]);
        }
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// half2 C2C of N = 2048 = 8 x 256 on MFMA, two transforms per workgroup tile
// (4 waves, 16 values per lane).  With n = t + 256 j (j < 8), t = t0 + 16 t1
// and k = k1 + 8 k' (k1 < 8), k' = k2 + 16 k3:
//   1. DFT8 over j of x[t + 256 j] -> Y1[t][k1], two 8-point DFTs per MFMA
//      column (block-diagonal operands, dft8_pair_operands): wave w, lane
//      (n, q), block b carries transform f = w / 2, sequence
//      t = 128 (w & 1) + 64 (q / 2) + 4 n + b, inputs j = 4 (q & 1) + e -- one
//      16-byte load per e straight from HBM, as in the N = 4096 kernel -- and
//      receives outputs k1 = 2 q + i of its column's two sequences
//      (y[2 H + i]: sequence t + 64 H of the column, t with q / 2 = 0).
//   2. Y1 *= W_2048^(t k1); workgroup exchange into the N = 4096 kernel's
//      stage-2 layout: matrix 8 f + k1 (wave 2 f + k1 / 4, block k1 % 4) holds
//      the 256-point sequence over t of (f, k1).
//   3-5. That kernel's stages 2 and 3 as a DFT256 over t = t0 + 16 t1: DFT16
//      over t1, W_256^(t0 k2), wave-local transpose, DFT16 over t0 -> lane
//      (n, q), block b of wave w: X_f[k1 + 8 k2 + 128 k3], k1 = 4 (w & 1) + b,
//      k2 = n, k3 = q + 4 r; staged out in 16-byte chunks (out_chunk).
// The exchange matrices sit 264 dwords apart, which keeps stage 1's writers
// (matrices 2 q apart within an instruction) conflict-free; the readers are
// the N = 4096 kernel's.
struct Mfma2048 {
    static constexpr int N = 2048;
    static constexpr int kMatrix = 264;
    static constexpr int kExchange = 16 * kMatrix;
    static constexpr int kOut = 4096;  // two transforms
    __device__ static __forceinline__ int xaddr(int m, int t0, int t1) {
        return kMatrix * m + 16 * t0 + 4 * (((t1 >> 2) + (t0 >> 2)) & 3) + ((t1 + m) & 3);
    }
};

// A-operand registers of two 8-point DFTs per column (block-diagonal real
// 32 x 32 matrix): half H produces sequence H's outputs k1 = m / 2 (row m,
// part m % 2) from inputs K = 16 H ... 16 H + 15 (input j = (K % 16) / 2,
// part K % 2); entries of the other sequence's inputs are zero.  With
// kPermuted the columns follow the device API's N = 2048 fragment order
// instead: lane group kq of the data operand holds sequence kq % 2's inputs
// j = 2 c + kq / 2 in its complex slots c = 0..3.  kArith computes the
// entries with cis_rev instead of reading the constant table.
template <bool FWD, bool kPermuted = false, bool kArith = false>
__device__ __forceinline__ void dft8_pair_operands(f16x8 (&a)[2], int lane) {
    const int m = lane & 15, kq = lane >> 4;
    const int k1 = m >> 1, o = m & 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int slot = e >> 1, p = e & 1;
            const int seq = kPermuted ? (kq & 1) : kq >> 1;
            const int j = kPermuted ? 2 * slot + (kq >> 1) : 4 * (kq & 1) + slot;
            const int ang = (2 * j * k1) & 15;  // W_8^(j k1) = W_16^(2 j k1)
            float c, s;
            if constexpr (kArith) {
                const cpx cs = cis_rev(ang, 16);
                c = cs.re;
                s = FWD ? -cs.im : cs.im;
            } else {
                c = kCos16[ang];
                s = FWD ? -kSin16[ang] : kSin16[ang];
            }
            const float v = o == 0 ? (p == 0 ? c : -s) : (p == 0 ? s : c);
            a[h][e] = static_cast<_Float16>(seq == h ? v : 0.0f);
        }
    }
}

template <bool FWD, bool kPrefetch>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void c2c_mfma2048_kernel(
    const __half2* __restrict__ in, __half2* __restrict__ out, int batch,
    const float2* __restrict__ tw, int tiles_per_block) {
    using P = Mfma2048;
    constexpr int N = P::N;
    __shared__ __align__(16) unsigned xbuf[P::kExchange];
    __shared__ __align__(16) unsigned obuf[P::kOut];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    const int f = wave >> 1;  // this wave's transform within the tile (stage 1)
    unsigned* const region = xbuf + 4 * P::kMatrix * wave;

    f16x8 a8[2], a[2];
    dft8_pair_operands<FWD>(a8, lane);
    dft16_operands<FWD>(a, lane);
    // Twiddles: W_2048^(t k1), t = 128 (w & 1) + 64 H + 4 n + b, k1 = 2 q + i
    // (r = 2 H + i); W_256^(t0 k2) = W_2048^(8 n k2), k2 = q + 4 r.
    cpx w1[4][4], w2[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 128 * (wave & 1) + 64 * (r >> 1) + 4 * n + b, k1 = 2 * q + (r & 1);
            const float2 x = tw[(t * k1) & (N - 1)];
            w1[b][r] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float2 x = tw[(8 * n * (q + 4 * r)) & (N - 1)];
        w2[r] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
    }

    const long long ntiles = (static_cast<long long>(batch) + 1) / 2;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
    if (tile >= tile_end) return;  // uniform over the workgroup

    // Inputs j = 4 (q & 1) + e of the lane's blocks b = 0..3:
    // x_f[128 (w & 1) + 64 (q / 2) + 4 n + b + 256 j]; zero past the batch.
    auto load = [&](u32x4 (&r)[4], long long tl) {
        const bool ok = 2 * tl + f < batch;
        const __half2* src = in + (2 * tl + f) * N + 128 * (wave & 1) + 64 * (q >> 1) + 4 * n +
                             1024 * (q & 1);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            r[e] = ok ? ld_nt(reinterpret_cast<const u32x4*>(src + 256 * e)) : u32x4{};
    };

    u32x4 next[4];
    if constexpr (kPrefetch) load(next, tile);
    for (; tile < tile_end; tile += step) {
        u32x4 cur[4];
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = next[i];
            if (tile + step < tile_end) load(next, tile + step);
        } else {
            load(cur, tile);
        }

        // ---- stage 1: two DFT8s over j per column, then W_2048^(t k1) ----
        cpx y[4][4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            u32x4 x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = cur[e][b];
            dft16_block(a8, as_f16x8(x), y[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) y[b][r] = cmul(y[b][r], w1[b][r]);
        }
        __syncthreads();  // every wave is done with the previous tile's exchange buffer
        // ---- exchange: matrix 8 f + k1, t0 = t % 16, t1 = t / 16 ----
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                xbuf[P::xaddr(8 * f + 2 * q + (r & 1), 4 * (n & 3) + b,
                              8 * (wave & 1) + 4 * (r >> 1) + (n >> 2))] = pack_half2(y[b][r]);
        __syncthreads();
        // ---- stage 2: block b holds matrix 4 w + b; lane (t0 = n, chunk q of t1) ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(
                region + P::kMatrix * b + 16 * n + 4 * ((q + (n >> 2)) & 3));
            u32x4 x;  // t1 = 4 q + e sits at position (e + m) & 3 = (e + b) & 3
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = raw[(e + b) & 3];
            dft16_block(a, as_f16x8(x), y[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) y[b][r] = cmul(y[b][r], w2[r]);
        }
        // ---- wave-local transpose: sequence (b, k2) gets its 16 t0 (tpos) ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int k2 = q + 4 * r;
                region[tpos(b, k2, n)] = pack_half2(y[b][r]);
            }
        wave_lds_sync();
        // ---- stage 3: DFT16 over t0 -> X_f[k1 + 8 k2 + 128 k3], k2 = n, k3 = q + 4 r ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 x = *reinterpret_cast<const u32x4*>(
                region + tchunk(b, n, q));
            dft16_block(a, as_f16x8(x), y[b]);
        }
        // ---- output: chunk K = (f' 2048 + 4 (w & 1) + 8 n + 128 k3) / 4 of the
        // tile holds k1 = 4 (w & 1) + b, b = 0..3 (f' = w / 2) ----
#pragma unroll
        for (int r = 0; r < 4; ++r)
            reinterpret_cast<u32x4*>(obuf)[Mfma4096::out_chunk(512 * f + (wave & 1) + 2 * n +
                                                               32 * (q + 4 * r))] =
                u32x4{pack_half2(y[0][r]), pack_half2(y[1][r]), pack_half2(y[2][r]),
                      pack_half2(y[3][r])};
        __syncthreads();
        __half2* dst = out + 2 * tile * N;
        const bool second = 2 * tile + 1 < batch;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < 2 || second)
                st_nt(reinterpret_cast<u32x4*>(dst + 4 * tid + 1024 * i),
                      reinterpret_cast<const u32x4*>(obuf)[Mfma4096::out_chunk(tid + 256 * i)]);
    }
}

// Per-lane coefficients of one direction of mfma2048_fft_regs: the
// column-permuted DFT8-pair operands, the plain DFT16 operands, the stage-1
// -> 2 twiddles W_2048^(t k1) (t = 4 (w & 1) + b + 8 n + 128 (r / 2),
// k1 = 2 q + r % 2) and the stage-2 -> 3 twiddles W_2048^(8 n (q + 4 r)),
// conjugated for the forward direction (tid: the lane's index in the
// 256-lane block).  load() from the table, build() with cis_rev.
struct Mfma2048Coeffs {
    static constexpr int N = 2048;
    f16x8 a8[2], a[2];
    cpx w1[4][4], w2[4];
    static constexpr int kTwiddles = 20;
    __device__ __forceinline__ f16x8& op(int i) { return i < 2 ? a8[i] : a[i - 2]; }
    __device__ __forceinline__ cpx& twiddle(int i) { return i < 16 ? w1[i >> 2][i & 3] : w2[i - 16]; }

    template <bool FWD, class Tw>
    __device__ __forceinline__ void fill(int tid, Tw tw_at) {
        const int wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 4 * (wave & 1) + b + 8 * n + 128 * (r >> 1);
                const cpx x = tw_at(t * (2 * q + (r & 1)));
                w1[b][r] = FWD ? cpx{x.re, -x.im} : x;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const cpx x = tw_at(8 * n * (q + 4 * r));
            w2[r] = FWD ? cpx{x.re, -x.im} : x;
        }
    }
    template <bool FWD>
    __device__ __forceinline__ void load(const float2* __restrict__ tw, int tid) {
        dft8_pair_operands<FWD, true>(a8, tid & 63);
        dft16_operands<FWD>(a, tid & 63);
        fill<FWD>(tid, [&](int k) {
            const float2 x = tw[k & (N - 1)];
            return cpx{x.x, x.y};
        });
    }
    template <bool FWD>
    __device__ __forceinline__ void build(int tid) {
        dft8_pair_operands<FWD, true, true>(a8, tid & 63);
        dft16_operands_arith<FWD>(a, tid & 63);
        fill<FWD>(tid, [](int k) { return cis_rev(k, N); });
    }
};

// Two N = 2048 transforms per workgroup from registers, either direction,
// for callers without the kernel's set-up (the device-side API).  Lane
// (n, q) of wave w holds, in v[b][r], element 4 (w & 1) + b + 8 n +
// 128 (q + 4 r) of transform w / 2 on entry and on return (the layout
// c2c_mfma2048_kernel's three stages leave, so transforms chain).  In that
// order block b's column n carries the sequences t = 4 (w & 1) + b + 8 n +
// 128 H (H = q % 2) with inputs j = 2 r + q / 2, so stage 1 takes the
// column-permuted DFT8-pair operands and leaves outputs k1 = 2 q + r % 2 of
// sequence H = r / 2; W_2048^(t k1); the exchange into the kernel's stage-2
// layout (t0 = t % 16 = 4 (w & 1) + b + 8 (n & 1), t1 = t / 16 = n / 2 + 8 H;
// stride 264 keeps these writes conflict-free too); the kernel's stages 2
// and 3.  xbuf: Mfma2048::kExchange dwords of LDS; two workgroup barriers,
// the first before xbuf is written.  `k` holds this direction's coefficients.
template <bool FWD>
__device__ __forceinline__ void mfma2048_fft_regs(unsigned* xbuf, const Mfma2048Coeffs& k, int tid,
                                                  cpx (&v)[4][4]) {
    using P = Mfma2048;
    const int wave = tid >> 6, lane = tid & 63, n = lane & 15, q = lane >> 4;
    const int f = wave >> 1;
    unsigned* const region = xbuf + 4 * P::kMatrix * wave;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        u32x4 xv;
#pragma unroll
        for (int r = 0; r < 4; ++r) xv[r] = pack_half2(v[b][r]);
        dft16_block(k.a8, as_f16x8(xv), v[b]);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[b][r] = cmul(v[b][r], k.w1[b][r]);
    }
    __syncthreads();  // every wave is done with xbuf
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            xbuf[P::xaddr(8 * f + 2 * q + (r & 1), 4 * (wave & 1) + b + 8 * (n & 1),
                          (n >> 1) + 8 * (r >> 1))] = pack_half2(v[b][r]);
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(
            region + P::kMatrix * b + 16 * n + 4 * ((q + (n >> 2)) & 3));
        u32x4 xv;  // t1 = 4 q + e sits at position (e + m) & 3 = (e + b) & 3
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = raw[(e + b) & 3];
        dft16_block(k.a, as_f16x8(xv), v[b]);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[b][r] = cmul(v[b][r], k.w2[r]);
    }
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            region[tpos(b, q + 4 * r, n)] = pack_half2(v[b][r]);
    wave_lds_sync();
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(
            region + tchunk(b, n, q));
        dft16_block(k.a, as_f16x8(xv), v[b]);
    }
}

// As above, the coefficients read from the positive-angle table `tw` of
// length 2048 for this call.
template <bool FWD>
__device__ __forceinline__ void mfma2048_fft_regs(unsigned* xbuf, const float2* __restrict__ tw,
                                                  int tid, cpx (&v)[4][4]) {
    Mfma2048Coeffs k;
    k.template load<FWD>(tw, tid);
    mfma2048_fft_regs<FWD>(xbuf, k, tid, v);
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// half2 C2C of N = 128 = 16 x 8 on MFMA, eight transforms per wave (16 values
// per lane), a tile of four waves.  With n = t + 8 j (t < 8, j < 16) and
// k = k1 + 16 k2 (k2 < 8):
//   1. DFT16 over j of x_f[t + 8 j] from the wave's staged values: block b,
//      column n holds transform f = 2 b + n / 8 of the wave, sequence
//      t = n % 8 -> lane (n, q) receives k1 = q + 4 r;
//   2. Y1 *= W_128^(t k1);
//   3. wave-local transpose: block b, column k1 holds transforms 2 b and
//      2 b + 1 (lane groups q / 2), inputs t = 4 (q % 2) + e;
//   4. two DFT8s over t per column (dft8_pair_operands) -> lane (n, q),
//      block b: y[b][2 H + i] = X_f[n + 16 (2 q + i)], f = 2 b + H;
//   5. staged out in 16-byte pieces.
// LDS per wave: input staging padded k + 8 (k / 32) (the stride-8 stage-1
// reads of the 64 lanes hit 64 banks), the transpose with 16-byte chunks
// rotated by column / 4, output staging padded k + 16 (k / 64) (dword writes
// and 16-byte reads conflict-free).
struct Mfma128 {
    static constexpr int N = 128;
    static constexpr int kFPW = 8;          // transforms per wave
    static constexpr int kFPB = 4 * kFPW;   // per tile
    static constexpr int kWaveVals = kFPW * N;
    static constexpr int kRegion = 1272;    // in_pad(1023) + 1 dwords
    __device__ static __forceinline__ int in_pad(int k) { return k + 8 * (k >> 5); }
    __device__ static __forceinline__ int out_pad(int k) { return k + 16 * (k >> 6); }
    __device__ static __forceinline__ int taddr(int b, int col, int qq, int e) {
        return 256 * b + 16 * col + 4 * ((qq + (col >> 2)) & 3) + e;
    }
};

template <bool FWD, bool kPrefetch>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void c2c_mfma128_kernel(
    const __half2* __restrict__ in, __half2* __restrict__ out, int batch,
    const float2* __restrict__ tw, int tiles_per_block) {
    using P = Mfma128;
    constexpr int N = P::N;
    __shared__ __align__(16) unsigned lds[4 * P::kRegion];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* const region = lds + wave * P::kRegion;

    f16x8 a[2], a8[2];
    dft16_operands<FWD>(a, lane);
    dft8_pair_operands<FWD>(a8, lane);
    cpx w1[4];  // W_128^(t k1), t = n % 8, k1 = q + 4 r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float2 x = tw[((n & 7) * (q + 4 * r)) & (N - 1)];
        w1[r] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
    }

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
    if (tile >= tile_end) return;  // uniform over the workgroup

    // Valid values (0..kWaveVals) of this wave's transforms in tile tl.
    auto valid = [&](long long tl) {
        const long long v = (static_cast<long long>(batch) - tl * P::kFPB - wave * P::kFPW) * N;
        return v <= 0 ? 0 : (v >= P::kWaveVals ? P::kWaveVals : static_cast<int>(v));
    };
    auto load = [&](u32x4 (&r)[4], long long tl) {
        const int nv = valid(tl);
        const __half2* src = in + (tl * P::kFPB + wave * P::kFPW) * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + 256 * i;
            r[i] = e < nv ? ld_nt(reinterpret_cast<const u32x4*>(src + e)) : u32x4{};
        }
    };

    u32x4 next[4];
    if constexpr (kPrefetch) load(next, tile);
    for (; tile < tile_end; tile += step) {
        u32x4 cur[4];
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = next[i];
            if (tile + step < tile_end) load(next, tile + step);
        } else {
            load(cur, tile);
        }
        wave_lds_sync();  // the previous tile's output reads are done
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4*>(region + P::in_pad(4 * lane + 256 * i)) = cur[i];
        wave_lds_sync();

        // ---- stage 1: DFT16 over j, then W_128^(t k1) ----
        cpx y[4][4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int base = 128 * (2 * b + (n >> 3)) + (n & 7);
            u32x4 x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = region[P::in_pad(base + 8 * (4 * q + e))];
            dft16_block(a, as_f16x8(x), y[b]);
#pragma unroll
            for (int r = 0; r < 4; ++r) y[b][r] = cmul(y[b][r], w1[r]);
        }
        // ---- transpose: (f, t, k1) -> block f / 2, column k1, group 2 (f % 2) + t / 4 ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::taddr(b, q + 4 * r, 2 * (n >> 3) + ((n & 7) >> 2), n & 3)] =
                    pack_half2(y[b][r]);
        wave_lds_sync();
        // ---- stage 2: two DFT8s over t per column ----
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x4 x = *reinterpret_cast<const u32x4*>(region + P::taddr(b, n, q, 0));
            dft16_block(a8, as_f16x8(x), y[b]);
        }
        // ---- output staging: X_f[n + 16 (2 q + i)], f = 2 b + H ----
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::out_pad(128 * (2 * b + (r >> 1)) + n + 16 * (2 * q + (r & 1)))] =
                    pack_half2(y[b][r]);
        wave_lds_sync();
        const int nv = valid(tile);
        __half2* dst = out + (tile * P::kFPB + wave * P::kFPW) * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + 256 * i;
            if (e < nv)
                st_nt(reinterpret_cast<u32x4*>(dst + e),
                      *reinterpret_cast<const u32x4*>(region + P::out_pad(e)));
        }
    }
}

}  // namespace thff
