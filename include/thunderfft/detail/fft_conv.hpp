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

namespace thff {

// ---------------------------------------------------------------------------
// conv2d: y[b] = IFFT2(FFT2(x[b]) * FFT2(h)) / (64*64) for 64 x 64 row-major
// images and one shared 64 x 64 filter h, i.e. the 2-D circular convolution
// y[b][r][c] = sum x[b][r'][c'] * h[(r - r') mod 64][(c - c') mod 64].
//
// One image is one 4096-value tile.  Rows are 64-point transforms (transform
// slot f = row, lane t holds columns t + 4j).  A workgroup-wide LDS transpose
// writes row f's element c into column transform c's slot at position f, so
// the column transforms run with the same 64-point machinery; the product
// with the filter spectrum (computed once per workgroup by the same steps,
// so its lane layout matches) and the inverse column transforms stay in
// registers, then the transpose runs back and the inverse row transforms
// finish.  Reference: sample/conv2d/thunder.cu:70-207 (row FFT, column FFT x H
// x column IFFT, row IFFT as three launches over a 1024 x 1024 image) and
// the unbuilt 64 x 64 tile sketch sample/conv2d/thunder_tile64.cu:33-208.
// ---------------------------------------------------------------------------

// Rows <-> columns of the 64 x 64 tile held as v[j] = A[f][t + 4j].
__device__ __forceinline__ void transpose64(cpx (&v)[16], cpx* lds, int f, int t) {
    using P = C2CPlan<64>;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) lds[(t + 4 * j) * P::kSlot + lds_pad(f)] = v[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = lds[f * P::kSlot + lds_pad(t + 4 * j)];
}

// v[j] = A[f][t + 4j] -> v[j] = X[kr = t + 4j][kc = f] (transposed spectrum).
template <bool FWD>
__device__ __forceinline__ void fft2_64(cpx (&v)[16], cpx* lds, cpx* slot, int f, int t,
                                        const LaneTwiddles<64>& w) {
    fft_registers<64, FWD>(v, slot, t, w);  // rows
    transpose64(v, lds, f, t);
    fft_registers<64, FWD>(v, slot, t, w);  // columns
}

// The inverse of fft2_64's layout change: transposed spectrum in, image out.
__device__ __forceinline__ void ifft2_64(cpx (&v)[16], cpx* lds, cpx* slot, int f, int t,
                                         const LaneTwiddles<64>& w) {
    fft_registers<64, false>(v, slot, t, w);  // columns
    transpose64(v, lds, f, t);
    fft_registers<64, false>(v, slot, t, w);  // rows
}

template <class IO>
__global__ __launch_bounds__(256) void conv2d64_kernel(const IO* __restrict__ x,
                                                       const IO* __restrict__ h,
                                                       IO* __restrict__ y, int batch,
                                                       const float2* __restrict__ tw,
                                                       int tiles_per_block) {
    using P = C2CPlan<64>;
    using T = TileIO<IO, 64>;
    __shared__ cpx lds[P::kLdsSlots];
    const T io(lds, threadIdx.x);

    LaneTwiddles<64> w;
    w.load(io.t, tw);
    constexpr float kScale = 1.0f / 4096.0f;

    long long tile, tile_end;
    block_tiles(batch, tiles_per_block, tile, tile_end);
    if (tile >= tile_end) return;  // uniform over the workgroup

    cpx hs[16];  // FFT2(h) / 4096 in the transposed-spectrum layout
    {
        typename T::Raw r;
        io.load(r, h, 0, 64);
        io.stage(r, hs);
        fft2_64<true>(hs, lds, io.slot, io.f, io.t, w);
#pragma unroll
        for (int j = 0; j < 16; ++j) hs[j] = {hs[j].re * kScale, hs[j].im * kScale};
    }
    const long long rows = 64LL * batch;  // TileIO counts 64-point row transforms
    for (; tile < tile_end; ++tile) {
        typename T::Raw r;
        io.load(r, x, tile, rows);
        cpx v[16];
        io.stage(r, v);
        fft2_64<true>(v, lds, io.slot, io.f, io.t, w);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = cmul(v[j], hs[j]);
        ifft2_64(v, lds, io.slot, io.f, io.t, w);
        io.store(v, y, tile, rows);
    }
}

}  // namespace thff
