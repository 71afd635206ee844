// fft_tile.hpp -- building blocks of the batched transforms on gfx950:
// the per-length plan, the in-register Stockham passes, per-lane twiddles and
// the staging of 4096-value tiles between HBM and the pass layout.
//
// Transform convention (include/thunderfft/thunderfft.cuh:129-141 of the
// reference): forward X[k] = sum_n x[n] exp(-2*pi*i*n*k/N), inverse uses
// exp(+...), neither is normalized; natural order in and out.
//
// Work decomposition.  A workgroup is 256 lanes (4 wave64s) and processes
// "tiles" of 4096 contiguous complex values (4096/N whole transforms), 16
// values per lane.  Every transform is owned by TPF = N/16 lanes; lane t of a
// transform holds x[t + TPF*j], j < 16, before the first pass and X[t + TPF*j]
// after the last one (natural_order), so a forward transform, a pointwise
// product and an inverse transform chain in registers with no reordering.
//
//   N <= 1024: each wave owns 1024/N whole transforms and a private LDS
//              region, synchronised at wave scope (no workgroup barriers).
//   N >= 2048: a transform spans 2 or 4 waves and passes synchronise the
//              workgroup.
//
// Passes are self-sorting Stockham decimation-in-time passes: radix 16 first,
// then R1 (and R2).  A pass of radix R after sub-transforms of length L
// treats butterfly b (0 <= b < N/R): k = b mod L, inputs x[b + j*N/R] (j < R)
// are multiplied by W_{L*R}^{j*k}, an R-point DFT gives outputs y_m written to
// (b - k)*R + k + m*L.
//
// Twiddles W_{LR}^{j*k} depend only on the lane: each lane loads a few base
// factors once (PassTwiddles) and keeps them in registers.
#pragma once

#include "fft_core.hpp"

namespace thff {

template <int N>
struct C2CPlan {
    static_assert(N == 64 || N == 128 || N == 256 || N == 512 || N == 1024 || N == 2048 ||
                      N == 4096,
                  "unsupported transform length");
    static constexpr int kE = 16;                 // complex values per lane
    static constexpr int kWG = 256;               // lanes per workgroup
    static constexpr int kTile = kWG * kE;        // complex values per tile
    static constexpr int kTPF = N / kE;           // lanes per transform
    static constexpr int kFPB = kTile / N;        // transforms per tile
    static constexpr int kR0 = 16;
    static constexpr int kR1 = N == 64 ? 4 : N == 128 ? 8 : 16;
    static constexpr int kR2 = N / (kR0 * kR1);   // 1 when two passes suffice
    static constexpr int kRLast = kR2 > 1 ? kR2 : kR1;
    static constexpr bool kWaveLocal = kTPF <= 64;
    static constexpr int kSlot = N + N / 16;      // padded LDS slots per transform
    static constexpr int kLdsSlots = kFPB * kSlot;
};

__device__ __forceinline__ int lds_pad(int i) { return i + (i >> 4); }

// A transform's LDS slot: element i of a contiguous slot sits at lds_pad(i);
// a strided slot holds element i at base[i * stride] (a column of an image
// kept row-major in LDS, transformed where it lies).
__device__ __forceinline__ cpx& slot_at(cpx* slot, int i) { return slot[lds_pad(i)]; }
struct StridedSlot {
    cpx* base;
    int stride;
};
__device__ __forceinline__ cpx& slot_at(StridedSlot s, int i) { return s.base[i * s.stride]; }

template <bool WaveLocal>
__device__ __forceinline__ void region_sync() {
    if constexpr (WaveLocal)
        wave_lds_sync();
    else
        __syncthreads();
}

// Twiddles of the pass of radix R that follows sub-transforms of length L.
// Butterfly b = t + TPF*q (q < 16/R) multiplies input j by W_{LR}^{j*k},
// k = b mod L.  Whenever q > 0 occurs, t + TPF*q < L and L*R = 16*TPF, so
// W_{LR}^{j*k} = W_{LR}^{j*(t mod L)} * W_16^{j*q}: only the lane's base
// factors W_{LR}^{j*(t mod L)} are kept in registers and W_16^{j*q} is a
// compile-time rotation.  For R = 16 the 15 bases are rebuilt per use from
// 6 stored ones, W^{(4a+c)k} = W^{4ak} * W^{ck}.  Values carry the positive
// angle (cos, sin)(2*pi*m/N) of the fp32 table (as the reference's table,
// thunderfft_impl_twiddle.cuh:76-91) and are conjugated at use for the
// forward direction, so one set serves both directions.
template <int N, int R, int L>
struct PassTwiddles {
    static constexpr bool kCompact = R == 16;
    static constexpr int kStored = kCompact ? 6 : R - 1;
    cpx b[kStored];

    __device__ __forceinline__ void load(int t, const float2* __restrict__ tw) {
        const int k = t % L;
        auto w = [&](int j) {
            const float2 x = tw[(j * k * (N / (L * R))) & (N - 1)];
            return cpx{x.x, x.y};
        };
        if constexpr (kCompact) {
            b[0] = w(1), b[1] = w(2), b[2] = w(3);
            b[3] = w(4), b[4] = w(8), b[5] = w(12);
        } else {
#pragma unroll
            for (int j = 1; j < R; ++j) b[j - 1] = w(j);
        }
    }

    // The same factors from cis_rev, with no table access.
    __device__ __forceinline__ void build(int t) {
        const int k = t % L;
        auto w = [&](int j) { return cis_rev(j * k * (N / (L * R)), N); };
        if constexpr (kCompact) {
            b[0] = w(1), b[1] = w(2), b[2] = w(3);
            b[3] = w(4), b[4] = w(8), b[5] = w(12);
        } else {
#pragma unroll
            for (int j = 1; j < R; ++j) b[j - 1] = w(j);
        }
    }

    // All R-1 bases W_{LR}^{j*(t mod L)}, j = 1..R-1.
    __device__ __forceinline__ void expand(cpx* w) const {
        if constexpr (kCompact) {
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int j = 4 * a + c;
                    if (j == 0) continue;
                    w[j - 1] = a == 0 ? b[c - 1] : (c == 0 ? b[2 + a] : cmul(b[2 + a], b[c - 1]));
                }
        } else {
#pragma unroll
            for (int j = 0; j < R - 1; ++j) w[j] = b[j];
        }
    }
};

template <int N>
struct LaneTwiddles {
    using P = C2CPlan<N>;
    PassTwiddles<N, P::kR1, 16> p1;
    PassTwiddles<N, (P::kR2 > 1 ? P::kR2 : 2), 16 * P::kR1> p2;  // unused when kR2 == 1
    const float2* table = nullptr;  // the table itself (read by the device API's MFMA path)
    __device__ __forceinline__ void load(int t, const float2* __restrict__ tw) {
        table = tw;
        p1.load(t, tw);
        if constexpr (P::kR2 > 1) p2.load(t, tw);
    }
    // The factors from cis_rev, with no table (the device API's fp16
    // coefficients, unit_fp16::make_reg_b_precompute).
    __device__ __forceinline__ void build(int t) {
        table = nullptr;
        p1.build(t);
        if constexpr (P::kR2 > 1) p2.build(t);
    }
};

// One Stockham pass p >= 1: write the previous pass's outputs to LDS, read
// this pass's inputs, twiddle, DFT.
template <int N, bool FWD, int R, int L, int RPrev, int LPrev, class Slot>
__device__ __forceinline__ void stockham_pass(cpx (&v)[16], Slot slot, int t,
                                              const PassTwiddles<N, R, L>& tw) {
    using P = C2CPlan<N>;
    // previous outputs: butterfly b = t + TPF*q, output m -> (b/LPrev)*LPrev*RPrev + b%LPrev + m*LPrev
    region_sync<P::kWaveLocal>();
#pragma unroll
    for (int q = 0; q < 16 / RPrev; ++q) {
        const int b = t + P::kTPF * q;
        const int base = (b / LPrev) * LPrev * RPrev + (b % LPrev);
#pragma unroll
        for (int m = 0; m < RPrev; ++m) slot_at(slot, base + m * LPrev) = v[q * RPrev + m];
    }
    region_sync<P::kWaveLocal>();
    cpx w[R - 1];
    tw.expand(w);
    static_for<0, 16 / R>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        const int b = t + P::kTPF * q;
        v[q * R] = slot_at(slot, b);
        static_for<1, R>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const cpx x = slot_at(slot, b + j * (N / R));
            v[q * R + j] = rot<16, j * q, FWD>(FWD ? cmulc(x, w[j - 1]) : cmul(x, w[j - 1]));
        });
        Dft<R, FWD>::run(v + q * R);
    });
}

// The whole transform of the lane's transform slot: v[j] = x[t + TPF*j] in,
// v[j] = X[t + TPF*j] out.  `slot` is the transform's LDS slot (cpx* or
// StridedSlot).
template <int N, bool FWD, class Slot>
__device__ __forceinline__ void fft_registers(cpx (&v)[16], Slot slot, int t,
                                              const LaneTwiddles<N>& w) {
    using P = C2CPlan<N>;
    Dft<16, FWD>::run(v);
    stockham_pass<N, FWD, P::kR1, 16, 16, 1>(v, slot, t, w.p1);
    if constexpr (P::kR2 > 1) stockham_pass<N, FWD, P::kR2, 16 * P::kR1, P::kR1, 16>(v, slot, t, w.p2);
    // last pass: output m of butterfly b = t + TPF*q is X[b + m*N/RLast]
    //          = X[t + TPF*(q + m*16/RLast)]
    constexpr int kRL = P::kRLast;
    cpx o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = v[i];
#pragma unroll
    for (int q = 0; q < 16 / kRL; ++q)
#pragma unroll
        for (int m = 0; m < kRL; ++m) v[q + m * (16 / kRL)] = o[q * kRL + m];
}

// N = 64 with exact per-lane twiddles: the radix-4 pass multiplies input j of
// butterfly t + 4q by W_64^(j (t + 4 q)), all 12 of them kept in registers
// (24 VGPRs), instead of a base factor W_64^(j t) times a compile-time W_16^(j q)
// rotation: 32 fewer VALU instructions per transform.  Same LDS exchange and
// register order as fft_registers<64>.
struct LaneTwiddles64Exact {
    cpx e[4][3];  // e[q][j - 1] = W_64^(j (t + 4 q)), positive angle
    __device__ __forceinline__ void load(int t, const float2* __restrict__ tw) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                const float2 x = tw[(j * (t + 4 * q)) & 63];
                e[q][j - 1] = cpx{x.x, x.y};
            }
    }
};

template <int N, bool FWD>
__device__ __forceinline__ void fft_registers(cpx (&v)[16], cpx* slot, int t,
                                              const LaneTwiddles64Exact& w) {
    static_assert(N == 64, "exact lane twiddles: N = 64");
    using P = C2CPlan<64>;
    Dft<16, FWD>::run(v);
    // the radix-16 outputs of butterfly t go to 16 t + m
    region_sync<P::kWaveLocal>();
#pragma unroll
    for (int m = 0; m < 16; ++m) slot[lds_pad(16 * t + m)] = v[m];
    region_sync<P::kWaveLocal>();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int b = t + 4 * q;
        v[4 * q] = slot[lds_pad(b)];
#pragma unroll
        for (int j = 1; j < 4; ++j) {
            const cpx x = slot[lds_pad(b + 16 * j)];
            v[4 * q + j] = FWD ? cmulc(x, w.e[q][j - 1]) : cmul(x, w.e[q][j - 1]);
        }
        Dft<4, FWD>::run(v + 4 * q);
    }
    // output m of butterfly t + 4q is X[t + 4 (q + 4 m)]
    cpx o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = v[i];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int m = 0; m < 4; ++m) v[q + 4 * m] = o[4 * q + m];
}

// Raw per-lane data of one tile as loaded from global memory: 16/kVec
// 16-byte vectors of kVec consecutive complex values.  Lane l of wave w
// holds tile elements 1024*w + kVec*l + 64*kVec*i, i < 16/kVec.
template <class IO>
struct TileRaw {
    using W = typename Io<IO>::W4;
    static constexpr int kCount = 16 / Io<IO>::kVec;
    W w[kCount];
};

// Moves 4096-value tiles between HBM and the pass layout (`batch` counts
// transforms of length N).  Tile element e
// sits at LDS position lds_pad(e) while staged, which is also where transform
// f's element i sits in its slot (f*kSlot + lds_pad(i)).  The last tile of a
// batch may hold fewer than kFPB transforms: missing inputs read as zero and
// missing outputs are not written.
template <class IO, int N>
struct TileIO {
    using P = C2CPlan<N>;
    using I = Io<IO>;
    using Raw = TileRaw<IO>;
    using W = typename Raw::W;
    static constexpr int kVec = I::kVec;

    int wave, lane, f, t;
    cpx* slot;   // this lane's transform slot
    cpx* chunk;  // this wave's quarter of the tile

    __device__ __forceinline__ TileIO(cpx* lds, int tid)
        : wave(tid >> 6), lane(tid & 63), f(tid / P::kTPF), t(tid % P::kTPF),
          slot(lds + (tid / P::kTPF) * P::kSlot), chunk(lds + (tid >> 6) * (1024 + 64)) {}

    // Valid values (0..1024) in this wave's quarter of tile tl.
    __device__ __forceinline__ int valid(long long tl, long long batch) const {
        long long left = batch - tl * P::kFPB;
        left = left < P::kFPB ? left : P::kFPB;
        const long long v = left * N - 1024LL * wave;
        return v <= 0 ? 0 : (v >= 1024 ? 1024 : static_cast<int>(v));
    }

    __device__ __forceinline__ void load(Raw& r, const IO* __restrict__ base, long long tl,
                                         long long batch) const {
        const int nv = valid(tl, batch);
        const IO* src = base + tl * P::kTile + 1024 * wave;
#pragma unroll
        for (int i = 0; i < Raw::kCount; ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            r.w[i] = e < nv ? ld_nt(reinterpret_cast<const W*>(src + e)) : W{};
        }
    }

    // Raw tile -> LDS -> v[j] = x[t + TPF*j] of this lane's transform.
    __device__ __forceinline__ void stage(const Raw& r, cpx (&v)[16]) const {
        region_sync<P::kWaveLocal>();  // earlier reads of the region are done
#pragma unroll
        for (int i = 0; i < Raw::kCount; ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            cpx q[kVec];
            I::decode4(r.w[i], q);
#pragma unroll
            for (int c = 0; c < kVec; ++c) chunk[lds_pad(e + c)] = q[c];
        }
        region_sync<P::kWaveLocal>();
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = slot[lds_pad(t + j * P::kTPF)];
    }

    // v[j] = y[t + TPF*j] -> LDS -> 16-byte non-temporal stores of tile tl.
    __device__ __forceinline__ void store(const cpx (&v)[16], IO* __restrict__ base, long long tl,
                                          long long batch) const {
        region_sync<P::kWaveLocal>();
#pragma unroll
        for (int j = 0; j < 16; ++j) slot[lds_pad(t + j * P::kTPF)] = v[j];
        region_sync<P::kWaveLocal>();
        const int nv = valid(tl, batch);
        IO* dst = base + tl * P::kTile + 1024 * wave;
#pragma unroll
        for (int i = 0; i < Raw::kCount; ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            if (e < nv) {
                cpx q[kVec];
#pragma unroll
                for (int c = 0; c < kVec; ++c) q[c] = chunk[lds_pad(e + c)];
                st_nt(reinterpret_cast<W*>(dst + e), I::encode4(q));
            }
        }
    }
};

// Direct movement between HBM and the first-pass layout, with no LDS
// staging: lane t of transform f loads x[t + TPF*j] (j < 16) into its
// registers, and stores y[t + TPF*j] from them.  One instruction of a wave
// covers 64/TPF whole runs of TPF consecutive values (N >= 1024: 64
// consecutive values of one transform), so every access is a full line.  A
// transform past the end of the batch reads zeros and is not written.
template <class IO, int N>
struct DirectIO {
    using P = C2CPlan<N>;
    using W = typename Io<IO>::W1;
    struct Raw {
        W w[16];
    };
    int f, t;
    __device__ __forceinline__ explicit DirectIO(int tid) : f(tid / P::kTPF), t(tid % P::kTPF) {}

    __device__ __forceinline__ void load(Raw& r, const IO* __restrict__ base, long long tl,
                                         long long batch) const {
        const long long tr = tl * P::kFPB + f;
        const W* p = reinterpret_cast<const W*>(base + tr * N + t);
#pragma unroll
        for (int j = 0; j < 16; ++j) r.w[j] = tr < batch ? ld_nt(p + j * P::kTPF) : W{};
    }
    __device__ __forceinline__ static void decode(const Raw& r, cpx (&v)[16]) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = Io<IO>::decode1(r.w[j]);
    }
    __device__ __forceinline__ void store(const cpx (&v)[16], IO* __restrict__ base, long long tl,
                                          long long batch) const {
        const long long tr = tl * P::kFPB + f;
        if (tr >= batch) return;
        W* p = reinterpret_cast<W*>(base + tr * N + t);
#pragma unroll
        for (int j = 0; j < 16; ++j) st_nt(p + j * P::kTPF, Io<IO>::encode1(v[j]));
    }
};

// Wave issue priority (s_setprio) from the share of this workgroup's tiles
// still to do, `left` of `total` (including the current one): 3 while more
// than three quarters remain, down to 0 in the last quarter.  Workgroups of a
// grid-stride walk start together but the SIMD's arbitration favours the
// oldest waves, so without it the last workgroups of a CU run alone at the
// end; with it a workgroup that gets ahead yields issue slots to those behind.
// Measured for the VALU-bound fp32 convolutions (conv1d of 16384 signals of
// 2048 with per-signal filters: 151 against 156-157 us; conv2d of 8192
// images: 1.5%; the valid conv1d: 1.8%) and the fp16 conv1d kernels at
// N = 2048 and 4096 (1-4%); the fp16 conv2d uses it too, neutral within one
// box's noise (59.4-61.7 against 60.8 us); at N <= 1024 the MFMA conv1d kernels
// measured neutral or slower with it (real conv1d N = 256: 61.5 against
// 58 us), the fp16 C2C kernels slower (N = 2048: 106 against 89 us) and the
// fp32 real conv1d neutral or slower (N = 256: 105 against 99-100 us), so
// those do not use it.
// The level is floor((4 left - 1) / total), decided by comparing `left`
// with three thresholds computed once (left >= ceil((l total + 1) / 4) for
// level >= l), so a walk pays no division per tile.
struct ProgressPriority {
    long long t1, t2, t3;
    __device__ __forceinline__ explicit ProgressPriority(long long total)
        : t1((total + 4) / 4), t2((2 * total + 4) / 4), t3((3 * total + 4) / 4) {}
    __device__ __forceinline__ void set(long long left) const {
        if (left >= t3)
            __builtin_amdgcn_s_setprio(3);
        else if (left >= t2)
            __builtin_amdgcn_s_setprio(2);
        else if (left >= t1)
            __builtin_amdgcn_s_setprio(1);
        else
            __builtin_amdgcn_s_setprio(0);
    }
};

// The tiles of workgroup blockIdx.x: first, first + step, ... while < end
// (first >= end when it has none).
//   tiles_per_block > 0: a contiguous run of that many (grids sized to the batch).
//   tiles_per_block = 0: grid-stride, tiles b, b + G, b + 2G, ... (grids sized to
//     the device).  The workgroups resident at any moment then work on
//     neighbouring tiles, so their traffic spreads over the HBM channels;
//     contiguous per-workgroup shares put the concurrent accesses a share apart
//     and measured 3-10% slower on MI355X.
__device__ __forceinline__ void tile_walk(long long ntiles, int tiles_per_block, long long& first,
                                          long long& end, long long& step) {
    if (tiles_per_block > 0) {
        first = static_cast<long long>(blockIdx.x) * tiles_per_block;
        end = first + tiles_per_block < ntiles ? first + tiles_per_block : ntiles;
        step = 1;
    } else {
        first = blockIdx.x;
        end = ntiles;
        step = gridDim.x;
    }
}

// Quotient and remainder of a walk index g by d (g = q d + r), advanced by
// the walk's constant step without a 64-bit division per step.
struct DivPos {
    long long q, r;
};
struct DivWalk {
    long long d, adv_q, adv_r;
    __device__ __forceinline__ DivWalk(long long step, long long divisor)
        : d(divisor), adv_q(step / divisor), adv_r(step - (step / divisor) * divisor) {}
    __device__ __forceinline__ DivPos at(long long g) const {
        const long long q = g / d;
        return {q, g - q * d};
    }
    // (adv_r < d and p.r < d: at most one carry)
    __device__ __forceinline__ DivPos advance(DivPos p) const {
        p.q += adv_q;
        p.r += adv_r;
        if (p.r >= d) p.r -= d, ++p.q;
        return p;
    }
};

}  // namespace thff
