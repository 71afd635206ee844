// fft_c2c.hpp -- the batched out-of-place C2C kernel for one (storage, N, direction).
//
// Replaces detail::ThunderFFT_global_kernel<T,N,fwd> of the reference
// (include/thunderfft/detail/kernel/global_kernel.cuh:21-100): natural-order
// signals of N complex values at in[b*N], out[b*N]; the last tile may hold
// fewer than kFPB valid transforms, whose inputs are never read (they are
// zero-filled) and whose outputs are never written.
//
// Work decomposition.  A workgroup is 256 lanes (4 wave64s) and processes
// "tiles" of 4096 contiguous complex values (4096/N whole transforms), 16
// values per lane.  Every transform is owned by TPF = N/16 lanes.  Each wave
// reads its quarter of the tile with 16-byte non-temporal loads and
// redistributes it through LDS into the first pass's layout; the output
// leaves the same way, so all global traffic is fully coalesced dwordx4.
//
//   N <= 1024: each wave owns 1024/N whole transforms and a private LDS
//              region, synchronised at wave scope (no workgroup barriers).
//   N >= 2048: a transform spans 2 or 4 waves and passes synchronise the
//              workgroup.
//
// A workgroup walks `tiles_per_block` consecutive tiles; kPrefetch keeps the
// next tile's loads in flight while the current one is transformed.
//
// Twiddles W_{LR}^{j*k} of every Stockham pass depend only on the lane, so
// each lane computes its (at most 30) factors once from the device table
// and keeps them in registers for all the tiles it processes.
//
// Global loads and stores are non-temporal: every byte is touched exactly
// once, so the data should not displace anything in the caches.
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
// W_{LR}^{j*(b mod L)}, read from the fp32 table tw[m] = (cos, sin)(2*pi*m/N)
// (positive angle, as the reference's table, thunderfft_impl_twiddle.cuh:
// 76-91) and conjugated once here for the forward direction.
template <int N, bool FWD, int R, int L>
__device__ __forceinline__ void pass_twiddles(cpx* w, int t, const float2* __restrict__ tw) {
    using P = C2CPlan<N>;
#pragma unroll
    for (int q = 0; q < 16 / R; ++q) {
        const int k = (t + P::kTPF * q) % L;
#pragma unroll
        for (int j = 1; j < R; ++j) {
            const float2 x = tw[(j * k * (N / (L * R))) & (N - 1)];
            w[q * (R - 1) + j - 1] = FWD ? cpx{x.x, -x.y} : cpx{x.x, x.y};
        }
    }
}

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
            v[q * R + j] = j == 0 ? x : cmul(x, w[q * (R - 1) + j - 1]);
        }
        Dft<R, FWD>::run(v + q * R);
    }
}

// Raw per-lane input of one tile as loaded from global memory: 16/kVec
// 16-byte vectors of kVec consecutive complex values.  Lane l of wave w
// holds tile elements 1024*w + kVec*l + 64*kVec*i, i < 16/kVec.
template <class IO>
struct TileRaw {
    using W = typename Io<IO>::W4;
    static constexpr int kCount = 16 / Io<IO>::kVec;
    W w[kCount];
};

// Every tile is 4096 contiguous complex values (kFPB whole transforms).
// Tile element e lives in LDS at lds_pad(e) while it is staged, which is
// also where transform f's element i sits in its slot (f*kSlot + lds_pad(i)).
//
// kPrefetch: keep the next tile's loads in flight while transforming the
// current one (costs 2*16/kVec*4 VGPRs; pays off when occupancy is low).
template <class IO, int N, bool FWD, bool kPrefetch>
__global__ __launch_bounds__(256) void c2c_kernel(const IO* __restrict__ in, IO* __restrict__ out,
                                                  int batch, const float2* __restrict__ tw,
                                                  int tiles_per_block) {
    using P = C2CPlan<N>;
    using I = Io<IO>;
    using Raw = TileRaw<IO>;
    using W = typename Raw::W;
    __shared__ cpx lds[P::kLdsSlots];
    const int tid = threadIdx.x;
    const int f = tid / P::kTPF;  // transform slot within the tile
    const int t = tid % P::kTPF;  // lane within the transform
    const int wave = tid >> 6, lane = tid & 63;
    constexpr int kVec = I::kVec;
    cpx* slot = lds + f * P::kSlot;
    cpx* chunk = lds + wave * (1024 + 64);  // the wave's quarter of the tile

    cpx w1[P::kTw1];
    cpx w2[P::kTw2 > 0 ? P::kTw2 : 1];
    pass_twiddles<N, FWD, P::kR1, 16>(w1, t, tw);
    if constexpr (P::kR2 > 1) pass_twiddles<N, FWD, P::kR2, 16 * P::kR1>(w2, t, tw);

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile = static_cast<long long>(blockIdx.x) * tiles_per_block;
    const long long tile_end = tile + tiles_per_block < ntiles ? tile + tiles_per_block : ntiles;
    if (tile >= tile_end) return;  // uniform over the workgroup

    // Valid values (0..1024) in this wave's quarter of tile tl: the tile's
    // last transforms may lie past the batch.
    auto chunk_valid = [&](long long tl) {
        long long left = static_cast<long long>(batch) - tl * P::kFPB;
        left = left < P::kFPB ? left : P::kFPB;
        const long long v = left * N - 1024LL * wave;
        return v <= 0 ? 0 : (v >= 1024 ? 1024 : static_cast<int>(v));
    };
    auto load_tile = [&](Raw& r, long long tl) {
        const int valid = chunk_valid(tl);
        const IO* src = in + tl * P::kTile + 1024 * wave;
#pragma unroll
        for (int i = 0; i < Raw::kCount; ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            r.w[i] = e < valid ? ld_nt(reinterpret_cast<const W*>(src + e)) : W{};
        }
    };

    Raw next;
    if constexpr (kPrefetch) load_tile(next, tile);
    for (; tile < tile_end; ++tile) {
        Raw cur;
        if constexpr (kPrefetch) {
            cur = next;
            if (tile + 1 < tile_end) load_tile(next, tile + 1);
        } else {
            load_tile(cur, tile);
        }

        // ---- stage: tile -> LDS, then pass-0 inputs x[t + j*TPF], j < 16 ----
        region_sync<P::kWaveLocal>();  // the previous tile's reads of the region are done
#pragma unroll
        for (int i = 0; i < Raw::kCount; ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            cpx q[kVec];
            I::decode4(cur.w[i], q);
#pragma unroll
            for (int c = 0; c < kVec; ++c) chunk[lds_pad(e + c)] = q[c];
        }
        region_sync<P::kWaveLocal>();
        cpx v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = slot[lds_pad(t + j * P::kTPF)];

        // ---- pass 0: radix 16 over stride-TPF inputs (L = 1, no twiddle) ----
        Dft<16, FWD>::run(v);
        // ---- pass 1 ----
        stockham_pass<N, FWD, P::kR1, 16, 16, 1>(v, slot, t, w1);
        // ---- pass 2 ----
        if constexpr (P::kR2 > 1) stockham_pass<N, FWD, P::kR2, 16 * P::kR1, P::kR1, 16>(v, slot, t, w2);

        // ---- store: last pass output m of butterfly b = t + TPF*q is y[b + m*N/RLast] ----
        constexpr int kRL = P::kRLast;
        region_sync<P::kWaveLocal>();
#pragma unroll
        for (int q = 0; q < 16 / kRL; ++q) {
            const int b = t + P::kTPF * q;
#pragma unroll
            for (int m = 0; m < kRL; ++m) slot[lds_pad(b + m * (N / kRL))] = v[q * kRL + m];
        }
        region_sync<P::kWaveLocal>();
        const int valid = chunk_valid(tile);
        IO* dst = out + tile * P::kTile + 1024 * wave;
#pragma unroll
        for (int i = 0; i < Raw::kCount; ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            if (e < valid) {
                cpx q[kVec];
#pragma unroll
                for (int c = 0; c < kVec; ++c) q[c] = chunk[lds_pad(e + c)];
                st_nt(reinterpret_cast<W*>(dst + e), I::encode4(q));
            }
        }
    }
}

}  // namespace thff
