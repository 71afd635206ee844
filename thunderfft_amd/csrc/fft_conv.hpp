// fft_conv.hpp -- fused FFT convolutions: forward FFT, pointwise product and
// inverse FFT in one kernel, so the spectra never touch HBM.
//
// conv1d: y[b] = IFFT(FFT(x[b]) * FFT(h[b or 0])) / N, i.e. the circular
// convolution y[b][k] = sum_m x[b][m] * h[(k - m) mod N] of every signal with
// its own filter (per-signal) or with one shared filter.  The reference's
// fused convolution (sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331)
// runs forward FFT -> multiply by a pre-permuted filter spectrum -> reorder
// -> inverse FFT inside one block; here the transforms keep lane t's values
// at x[t + TPF*j] both before the first pass and after the last one
// (fft_tile.hpp), so the product and the inverse transform need neither a
// spectrum permutation nor a reorder.  The 1/N of the inverse is folded into
// the filter spectrum.
#pragma once

#include "fft_tile.hpp"

namespace thff {

template <class IO, int N, bool kPerSignal>
__global__ __launch_bounds__(256) void conv1d_kernel(const IO* __restrict__ x,
                                                     const IO* __restrict__ h, IO* __restrict__ y,
                                                     int batch, const float2* __restrict__ tw,
                                                     int tiles_per_block) {
    using P = C2CPlan<N>;
    using T = TileIO<IO, N>;
    __shared__ cpx lds[P::kLdsSlots];
    const T io(lds, threadIdx.x);

    LaneTwiddles<N> w;
    w.load(io.t, tw);
    constexpr float kScale = 1.0f / N;

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end;
    block_tiles(ntiles, tiles_per_block, tile, tile_end);
    if (tile >= tile_end) return;  // uniform over the workgroup

    cpx hs[16];  // this lane's share of the scaled filter spectrum, H[t + TPF*j] / N
    if constexpr (!kPerSignal) {
        // Every transform slot transforms the shared filter once.
#pragma unroll
        for (int j = 0; j < 16; ++j) hs[j] = Io<IO>::decode1(
            *reinterpret_cast<const typename Io<IO>::W1*>(h + io.t + j * P::kTPF));
        fft_registers<N, true>(hs, io.slot, io.t, w);
#pragma unroll
        for (int j = 0; j < 16; ++j) hs[j] = {hs[j].re * kScale, hs[j].im * kScale};
    }

    for (; tile < tile_end; ++tile) {
        typename T::Raw rx, rh;
        io.load(rx, x, tile, batch);
        cpx v[16];
        if constexpr (kPerSignal) {
            io.load(rh, h, tile, batch);
            io.stage(rh, hs);
            fft_registers<N, true>(hs, io.slot, io.t, w);
#pragma unroll
            for (int j = 0; j < 16; ++j) hs[j] = {hs[j].re * kScale, hs[j].im * kScale};
        }
        io.stage(rx, v);
        fft_registers<N, true>(v, io.slot, io.t, w);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = cmul(v[j], hs[j]);
        fft_registers<N, false>(v, io.slot, io.t, w);
        io.store(v, y, tile, batch);
    }
}

}  // namespace thff
