// bench_compute.hip -- in-register repeat kernels for the reference-style
// differential compute time (sample/bench/paper_fft.cu:131-148 and
// sample/bench/baseline/thunderfft_bench.h:7-57): each block loads its tile
// once, runs the transform `repeats` times on it and stores once, so
// (t(2R) - t(R)) / R is the time of one pass of the transform over the batch
// without global-memory traffic.  The repeated values are not meaningful
// (they grow without bound and may overflow) and are never checked, as in
// the reference.  Built into libthff_bench_compute.so for bench.py.
#include "thunderfft/detail/fft_c2c.hpp"
#include "thunderfft/detail/fft_mfma.hpp"
#include "thunderfft/thunderfft.h"

namespace thff {
namespace {

// fp32 arithmetic, VALU passes (the kernel the library runs for float).
template <class IO, int N>
__global__ __launch_bounds__(256) void repeat_valu(const IO* in, IO* out, int batch,
                                                   const float2* tw, int repeats) {
    using P = C2CPlan<N>;
    using T = TileIO<IO, N>;
    __shared__ cpx lds[P::kLdsSlots];
    const T io(lds, threadIdx.x);
    LaneTwiddles<N> w;
    w.load(io.t, tw);
    typename T::Raw r;
    io.load(r, in, blockIdx.x, batch);
    cpx v[16];
    io.stage(r, v);
#pragma unroll 1
    for (int i = 0; i < repeats; ++i) fft_registers<N, true>(v, io.slot, io.t, w);
    io.store(v, out, blockIdx.x, batch);
}

// half2 on MFMA (the kernel the library runs for half, N = 256*C): steps 1-6
// from the LDS staging, the result written back there in natural order.
template <int C>
__global__ __launch_bounds__(256) void repeat_mfma(const __half2* in, __half2* out, int batch,
                                                   const float2* tw, int repeats) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    constexpr int kRaw = P::kVals / 4;
    __shared__ unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;
    f16x8 a[2];
    cpx w2[C > 1 ? C - 1 : 1];
    mfma_setup<C, true>(a, w1, nullptr, w2, tw);
    const Stage3Plain<false> s3{a, w2};
    const long long first = static_cast<long long>(blockIdx.x) * P::kFPB + wave * P::kFPW;
    const bool valid = first + P::kFPW <= batch;
    const __half2* src = in + first * N;
#pragma unroll
    for (int i = 0; i < kRaw; ++i)
        *reinterpret_cast<u32x4*>(region + P::in_pad(4 * lane + 256 * i)) =
            valid ? ld_nt(reinterpret_cast<const u32x4*>(src + 4 * lane + 256 * i)) : u32x4{};
    cpx y[P::kBlocks][4];
#pragma unroll 1
    for (int i = 0; i < repeats; ++i) {
        wave_lds_sync();
        mfma_fft_staged<C, true>(region, a, w1, s3, lane, y);
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < P::kBlocks; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::in_pad((b / C) * N + n + 16 * (b % C) + P::kM * (q + 4 * r))] =
                    pack_half2(y[b][r]);
    }
    wave_lds_sync();
    if (valid) {
        __half2* dst = out + first * N;
#pragma unroll
        for (int i = 0; i < kRaw; ++i)
            st_nt(reinterpret_cast<u32x4*>(dst + 4 * lane + 256 * i),
                  *reinterpret_cast<const u32x4*>(region + P::in_pad(4 * lane + 256 * i)));
    }
}

// ---------------------------------------------------------------------------
// fp32 data with both DFT16 stages on the matrix cores, for the measurement
// of the float path on MFMA (CDNA4 has no xf32): the two-stage N = 1024
// transform of the fp16 kernel (fft_mfma.hpp: DFT16 over j, W_1024^(t k1),
// DFT4, W_64^(n m), transpose, DFT16 over n) with fp32 data, fp32 twiddles
// and one of two DFT16 engines:
//   kF32:    v_mfma_f32_16x16x4_f32, exact fp32 products; the 32 x 32 real
//            DFT matrix takes 8 K-steps x 2 halves = 16 MFMAs per 16 sequences.
//   kBf16x3: v_mfma_f32_16x16x32_bf16 on a split x = x_hi + x_lo, F = F_hi +
//            F_lo (bf16 parts, round to nearest even): F_hi x_hi + F_hi x_lo
//            + F_lo x_hi, 6 MFMAs per 16 sequences, products accurate to
//            about 2^-16 relative (the dropped F_lo x_lo and the residuals).
// The wave's transform is staged in LDS as fp32 (8 KiB + padding); the
// transpose goes through the same region in fp32 (rows of 36 floats).
enum class SplitMode { kF32, kBf16x3 };
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));

// Real DFT16 matrix entry of half h, lane-row m (output k = m/4 + 4(2h +
// (m%4)/2), part (m%4)%2), column col (input col/2, part col%2): the row
// order of dft16_operands.
__device__ __forceinline__ float dft16_real_entry(int h, int m, int col) {
    const int k = (m >> 2) + 4 * (2 * h + ((m & 3) >> 1));
    const int o = m & 1, j = col >> 1, p = col & 1;
    const int ang = (j * k) & 15;
    const float c = kCos16[ang], sn = -kSin16[ang];  // forward
    return o == 0 ? (p == 0 ? c : -sn) : (p == 0 ? sn : c);
}

struct SplitOperands {
    float f32[2][8];   // kF32: A of K-step s, half h: lane (m, kq) holds F[row(h, m)][4 s + kq]
    bf16x8 hi[2], lo[2];  // kBf16x3: lane (m, q) holds F[row(h, m)][8 q + e]
};

template <SplitMode M>
__device__ __forceinline__ void split_operands(SplitOperands& a, int lane) {
    const int m = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if constexpr (M == SplitMode::kF32) {
#pragma unroll
            for (int s8 = 0; s8 < 8; ++s8) a.f32[h][s8] = dft16_real_entry(h, m, 4 * s8 + kq);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = dft16_real_entry(h, m, 8 * kq + e);
                const __bf16 fh = static_cast<__bf16>(f);
                a.hi[h][e] = fh;
                a.lo[h][e] = static_cast<__bf16>(f - static_cast<float>(fh));
            }
        }
    }
}

// One DFT16 over 16 sequences: x holds this lane's B-operand reals (kF32:
// the 8 K-step values; kBf16x3: inputs 4q..4q+3 as 8 floats).
template <SplitMode M>
__device__ __forceinline__ void dft16_split(const SplitOperands& a, const float (&x)[8], cpx* y) {
    bf16x8 xh, xl;
    if constexpr (M == SplitMode::kBf16x3) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const __bf16 h = static_cast<__bf16>(x[e]);
            xh[e] = h;
            xl[e] = static_cast<__bf16>(x[e] - static_cast<float>(h));
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        if constexpr (M == SplitMode::kF32) {
#pragma unroll
            for (int s8 = 0; s8 < 8; ++s8)
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f32[h][s8], x[s8], d, 0, 0, 0);
        } else {
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi[h], xh, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi[h], xl, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo[h], xh, d, 0, 0, 0);
        }
        y[2 * h] = {d[0], d[1]};
        y[2 * h + 1] = {d[2], d[3]};
    }
}

// Natural-order fp32 staging of one N = 1024 transform: float offset of
// element e (component c), 16 float2 of padding per 64 elements, so the
// kF32 stage-1 reads of 64 lanes hit 64 banks.
__device__ __forceinline__ int split_stage_off(int e) { return 2 * (e + 16 * (e >> 6)); }
constexpr int kSplitStage = 2 * (1024 + 16 * 16);  // floats per wave
constexpr int kSplitRow = 36;                      // transpose row stride (floats)

template <SplitMode M>
__global__ __launch_bounds__(256) void repeat_mfma_split(const float2* in, float2* out, int batch,
                                                         const float2* tw, int repeats) {
    constexpr int N = 1024, C = 4;
    static_assert(64 * kSplitRow <= kSplitStage, "the transpose rows reuse the staging");
    __shared__ float lds[4 * kSplitStage];
    __shared__ cpx w1[C * 4 * 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    float* stage = lds + wave * kSplitStage;
    float* rows = stage;  // the transpose reuses the staging (48 KiB per workgroup)
    SplitOperands a;
    split_operands<M>(a, lane);
    for (int e = tid; e < C * 4 * 64; e += 256) {
        const int l = e & 63, r = (e >> 6) & 3, c = e >> 8;
        const float2 x = tw[((16 * c + (l & 15)) * ((l >> 4) + 4 * r)) & (N - 1)];
        w1[e] = cpx{x.x, -x.y};
    }
    cpx w2[C - 1];
#pragma unroll
    for (int m = 1; m < C; ++m) {
        const float2 x = tw[(16 * n * m) & (N - 1)];
        w2[m - 1] = cpx{x.x, -x.y};
    }
    __syncthreads();
    const long long first = static_cast<long long>(blockIdx.x) * 4 + wave;
    const bool valid = first < batch;
    const float2* src = in + first * N;
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
        const int e = lane + 64 * i;
        const float2 v = valid ? src[e] : make_float2(0.f, 0.f);
        stage[split_stage_off(e)] = v.x;
        stage[split_stage_off(e) + 1] = v.y;
    }
    cpx y[C][4];
#pragma unroll 1
    for (int it = 0; it < repeats; ++it) {
        wave_lds_sync();
        // stage 1: DFT16 over j of x[16 c + n + 64 j] -> Y[k1 = q + 4 r]
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float x[8];
            if constexpr (M == SplitMode::kF32) {
#pragma unroll
                for (int s8 = 0; s8 < 8; ++s8)
                    x[s8] = stage[split_stage_off(16 * c + n + 64 * (2 * s8 + (q >> 1))) + (q & 1)];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = split_stage_off(16 * c + n + 64 * (4 * q + e));
                    x[2 * e] = stage[o];
                    x[2 * e + 1] = stage[o + 1];
                }
            }
            dft16_split<M>(a, x, y[c]);
        }
        // twiddle W_1024^(t k1), DFT4 over c, twiddle W_64^(n m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cpx v[C];
#pragma unroll
            for (int c = 0; c < C; ++c) v[c] = cmul(y[c][r], w1[(c * 4 + r) * 64 + lane]);
            Dft<C, true>::run(v);
            y[0][r] = v[0];
#pragma unroll
            for (int m = 1; m < C; ++m) y[m][r] = cmul(v[m], w2[m - 1]);
        }
        // transpose: row 16 m + k1 holds the 16 inputs n of sequence (k1, m)
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < C; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * m + q + 4 * r;
                *reinterpret_cast<float2*>(rows + row * kSplitRow + 2 * n) =
                    make_float2(y[m][r].re, y[m][r].im);
            }
        wave_lds_sync();
        // stage 3: DFT16 over n -> X[k1 + 16 m + 64 (q + 4 r)], k1 = n
#pragma unroll
        for (int m = 0; m < C; ++m) {
            float x[8];
            const float* row = rows + (16 * m + n) * kSplitRow;
            if constexpr (M == SplitMode::kF32) {
#pragma unroll
                for (int s8 = 0; s8 < 8; ++s8) x[s8] = row[4 * s8 + q];
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = row[8 * q + e];
            }
            dft16_split<M>(a, x, y[m]);
        }
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < C; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int o = split_stage_off(n + 16 * m + 64 * (q + 4 * r));
                stage[o] = y[m][r].re;
                stage[o + 1] = y[m][r].im;
            }
    }
    wave_lds_sync();
    if (valid) {
        float2* dst = out + first * N;
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
            const int e = lane + 64 * i;
            dst[e] = make_float2(stage[split_stage_off(e)], stage[split_stage_off(e) + 1]);
        }
    }
}

}  // namespace
}  // namespace thff

// One launch of the repeat kernel for N = 1024 over `batch` transforms
// (a multiple of the tile size); precision 0 float (VALU), 1 half (MFMA),
// 2 float with both DFT16 stages on v_mfma_f32_16x16x4_f32, 3 float with
// them on the bf16x3 split (v_mfma_f32_16x16x32_bf16).  Modes 2 and 3 use
// the float twiddle table and run forward only.
// Returns 0, -22 (bad argument: no table for N = 1024, batch not a multiple)
// or -5 (launch error).  Asynchronous on `stream`.
extern "C" int thffx_compute_repeat(int precision, const void* x, void* y, int batch,
                                    int repeats, void* stream) {
    constexpr int N = 1024;
    const void* table = nullptr;
    int tn = 0;
    const int table_precision = precision >= 2 ? THFF_FLOAT : precision;
    if (thff_twiddle_info(table_precision, &table, &tn) != 0 || tn != N || !table) return -22;
    if (!x || !y || x == y || batch <= 0 || repeats < 0 || batch % 4) return -22;
    const auto* tw = static_cast<const float2*>(table);
    auto s = static_cast<hipStream_t>(stream);
    const unsigned grid = batch / 4;
    if (precision == 2)
        thff::repeat_mfma_split<thff::SplitMode::kF32><<<grid, 256, 0, s>>>(
            static_cast<const float2*>(x), static_cast<float2*>(y), batch, tw, repeats);
    else if (precision == 3)
        thff::repeat_mfma_split<thff::SplitMode::kBf16x3><<<grid, 256, 0, s>>>(
            static_cast<const float2*>(x), static_cast<float2*>(y), batch, tw, repeats);
    else if (precision == THFF_FLOAT)
        thff::repeat_valu<float2, N><<<grid, 256, 0, s>>>(static_cast<const float2*>(x),
                                                          static_cast<float2*>(y), batch, tw,
                                                          repeats);
    else
        thff::repeat_mfma<4><<<grid, 256, 0, s>>>(static_cast<const __half2*>(x),
                                                  static_cast<__half2*>(y), batch, tw, repeats);
    return hipGetLastError() == hipSuccess ? 0 : -5;
}
