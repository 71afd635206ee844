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
// Twiddles W_{LR}^{j*k} depend only on the lane, so each lane loads its (at
// most 30) factors once and keeps them in registers; they are stored with the
// positive angle and conjugated at use for the forward direction, so one set
// serves both directions.
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
    static constexpr int kTw1 = (16 / kR1) * (kR1 - 1);                  // pass-1 factors per lane
    static constexpr int kTw2 = kR2 > 1 ? (16 / kR2) * (kR2 - 1) : 0;   // pass-2 factors per lane
};

__device__ __forceinline__ int lds_pad(int i) { return i + (i >> 4); }

template <bool WaveLocal>
__device__ __forceinline__ void region_sync() {
    if constexpr (WaveLocal)
        wave_lds_sync();
    else
        __syncthreads();
}

// Per-lane twiddles of the pass of radix R that follows sub-transforms of
// length L: for butterfly b = t + TPF*q (q < 16/R) and input j (1 <= j < R),
// (cos, sin)(2*pi*j*(b mod L)/(L*R)), read from the fp32 table
// tw[m] = (cos, sin)(2*pi*m/N) (positive angle, as the reference's table,
// thunderfft_impl_twiddle.cuh:76-91).
template <int N, int R, int L>
__device__ __forceinline__ void pass_twiddles(cpx* w, int t, const float2* __restrict__ tw) {
    using P = C2CPlan<N>;
#pragma unroll
    for (int q = 0; q < 16 / R; ++q) {
        const int k = (t + P::kTPF * q) % L;
#pragma unroll
        for (int j = 1; j < R; ++j) {
            const float2 x = tw[(j * k * (N / (L * R))) & (N - 1)];
            w[q * (R - 1) + j - 1] = cpx{x.x, x.y};
        }
    }
}

template <int N>
struct LaneTwiddles {
    using P = C2CPlan<N>;
    cpx w1[P::kTw1];
    cpx w2[P::kTw2 > 0 ? P::kTw2 : 1];
    __device__ __forceinline__ void load(int t, const float2* __restrict__ tw) {
        pass_twiddles<N, P::kR1, 16>(w1, t, tw);
        if constexpr (P::kR2 > 1) pass_twiddles<N, P::kR2, 16 * P::kR1>(w2, t, tw);
    }
};

// One Stockham pass p >= 1: write the previous pass's outputs to LDS, read
// this pass's inputs, twiddle, DFT.
template <int N, bool FWD, int R, int L, int RPrev, int LPrev>
__device__ __forceinline__ void stockham_pass(cpx (&v)[16], cpx* slot, int t, const cpx* w) {
    using P = C2CPlan<N>;
    // previous outputs: butterfly b = t + TPF*q, output m -> (b/LPrev)*LPrev*RPrev + b%LPrev + m*LPrev
    region_sync<P::kWaveLocal>();
#pragma unroll
    for (int q = 0; q < 16 / RPrev; ++q) {
        const int b = t + P::kTPF * q;
        const int base = (b / LPrev) * LPrev * RPrev + (b % LPrev);
#pragma unroll
        for (int m = 0; m < RPrev; ++m) slot[lds_pad(base + m * LPrev)] = v[q * RPrev + m];
    }
    region_sync<P::kWaveLocal>();
#pragma unroll
    for (int q = 0; q < 16 / R; ++q) {
        const int b = t + P::kTPF * q;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const cpx x = slot[lds_pad(b + j * (N / R))];
            if (j == 0) {
                v[q * R] = x;
            } else {
                const cpx ww = w[q * (R - 1) + j - 1];
                v[q * R + j] = FWD ? cmulc(x, ww) : cmul(x, ww);
            }
        }
        Dft<R, FWD>::run(v + q * R);
    }
}

// The whole transform of the lane's transform slot: v[j] = x[t + TPF*j] in,
// v[j] = X[t + TPF*j] out.  `slot` is the transform's LDS slot.
template <int N, bool FWD>
__device__ __forceinline__ void fft_registers(cpx (&v)[16], cpx* slot, int t,
                                              const LaneTwiddles<N>& w) {
    using P = C2CPlan<N>;
    Dft<16, FWD>::run(v);
    stockham_pass<N, FWD, P::kR1, 16, 16, 1>(v, slot, t, w.w1);
    if constexpr (P::kR2 > 1) stockham_pass<N, FWD, P::kR2, 16 * P::kR1, P::kR1, 16>(v, slot, t, w.w2);
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

// Tiles [first, end) of the workgroup; first >= end when it has none.
__device__ __forceinline__ void block_tiles(long long ntiles, int tiles_per_block, long long& first,
                                            long long& end) {
    first = static_cast<long long>(blockIdx.x) * tiles_per_block;
    end = first + tiles_per_block < ntiles ? first + tiles_per_block : ntiles;
}

}  // namespace thff
