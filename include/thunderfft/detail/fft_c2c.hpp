// fft_c2c.hpp -- the batched out-of-place C2C kernel for one (storage, N, direction).
//
// Replaces detail::ThunderFFT_global_kernel<T,N,fwd> of the reference
// (include/thunderfft/detail/kernel/global_kernel.cuh:21-100): natural-order
// signals of N complex values at in[b*N], out[b*N]; the last tile may hold
// fewer than kFPB valid transforms, whose inputs are never read (they are
// zero-filled) and whose outputs are never written.
//
// A workgroup walks `tiles_per_block` consecutive tiles of 4096 values, or
// with 0 every G-th tile of a device-sized grid (tile_walk, fft_tile.hpp).  Each wave reads its quarter of a tile with 16-byte
// non-temporal loads and redistributes it through LDS into the first pass's
// layout; the output leaves the same way, so all global traffic is fully
// coalesced dwordx4.  With kDirect the tile instead moves straight between
// HBM and the first (last) pass's registers (DirectIO, fft_tile.hpp): no
// staging, whole lines per wave instruction for N >= 256.  kPrefetch keeps
// the next tile's loads in flight while the current one is transformed.  Arithmetic is fp32 for both storage
// types: half inputs are widened on load and rounded once (to nearest even)
// on store.
#pragma once

#include "fft_tile.hpp"

namespace thff {

// Lengths up to 1024 are held to <= 168 VGPRs (3 waves per SIMD) without
// spilling; the longer ones keep the compiler's choice.  Held to 128 (4 waves,
// 4 one-tile workgroups per CU) the fp32 N = 1024 kernel does not spill either
// but measured slower: 174.7 against 172.3-172.4 us.
template <int N>
inline constexpr int kMinWavesPerEU = N <= 1024 ? 3 : 1;

template <class IO, int N, bool FWD, bool kPrefetch, bool kDirect = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kMinWavesPerEU<N>))) void
c2c_kernel(const IO* __restrict__ in, IO* __restrict__ out, int batch, const float2* __restrict__ tw,
           int tiles_per_block) {
    using P = C2CPlan<N>;
    using T = TileIO<IO, N>;
    __shared__ cpx lds[P::kLdsSlots];
    const T io(lds, threadIdx.x);

    LaneTwiddles<N> w;
    w.load(io.t, tw);

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
    if (tile >= tile_end) return;  // uniform over the workgroup

    if constexpr (kDirect) {
        const DirectIO<IO, N> dio(threadIdx.x);
        typename DirectIO<IO, N>::Raw next;
        if constexpr (kPrefetch) dio.load(next, in, tile, batch);
        for (; tile < tile_end; tile += step) {
            typename DirectIO<IO, N>::Raw cur;
            if constexpr (kPrefetch) {
                cur = next;
                if (tile + step < tile_end) dio.load(next, in, tile + step, batch);
            } else {
                dio.load(cur, in, tile, batch);
            }
            cpx v[16];
            dio.decode(cur, v);
            fft_registers<N, FWD>(v, io.slot, io.t, w);
            dio.store(v, out, tile, batch);
        }
        return;
    }
    typename T::Raw next;
    if constexpr (kPrefetch) io.load(next, in, tile, batch);
    for (; tile < tile_end; tile += step) {
        typename T::Raw cur;
        if constexpr (kPrefetch) {
            cur = next;
            if (tile + step < tile_end) io.load(next, in, tile + step, batch);
        } else {
            io.load(cur, in, tile, batch);
        }
        cpx v[16];
        io.stage(cur, v);
        fft_registers<N, FWD>(v, io.slot, io.t, w);
        io.store(v, out, tile, batch);
    }
}

}  // namespace thff
