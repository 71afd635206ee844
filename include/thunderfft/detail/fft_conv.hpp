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

#include <type_traits>

namespace thff {

// Next-tile prefetch of the VALU convolutions: none; early, the next tile's
// loads issued before the current tile is staged; or late, issued after the
// current tile's product with the filter spectrum, before its inverse
// transform.  Loads return in order, so a load issued after a prefetch waits
// for it: the late form keeps the spectrum's loads ahead of the prefetch.
enum class Prefetch { kNone, kEarly, kLate };

// Waves per SIMD the fused 1-D convolution is held to (168 VGPRs for 3): 3
// fits without spilling up to N = 2048 and measured 7-12% faster than the 2
// the compiler picks on its own (16384 x 2048, MI355X).
template <int N>
inline constexpr int kConvMinWavesPerEU = N <= 2048 ? 3 : 1;

// kDirect (per-signal filters, no prefetch): signal and filter load straight
// into the first pass's registers and the output is stored from the last
// pass's, with no LDS staging (DirectIO): 16384 x 2048 fp32 158 vs 164 us.
template <class IO, int N, bool kPerSignal, Prefetch kPf = Prefetch::kNone, bool kDirect = false>
__global__ __launch_bounds__(256) __attribute__((
    amdgpu_waves_per_eu(kPf != Prefetch::kNone ? 2 : kConvMinWavesPerEU<N>))) void
conv1d_kernel(const IO* __restrict__ x, const IO* __restrict__ h, IO* __restrict__ y, int batch,
              const float2* __restrict__ tw, int tiles_per_block) {
    using P = C2CPlan<N>;
    using T = TileIO<IO, N>;
    __shared__ cpx lds[P::kLdsSlots];
    const T io(lds, threadIdx.x);

    LaneTwiddles<N> w;
    w.load(io.t, tw);
    constexpr float kScale = 1.0f / N;

    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
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

    // Prefetch::kEarly: the next tile's raw signal (and filter) load while
    // the current tile is transformed.
    constexpr bool kPrefetch = kPf == Prefetch::kEarly;
    typename T::Raw nx, nh;
    if constexpr (kPrefetch) {
        io.load(nx, x, tile, batch);
        if constexpr (kPerSignal) io.load(nh, h, tile, batch);
    }
    long long left = (tile_end - tile + step - 1) / step;  // tiles still to do, this one included
    const ProgressPriority priority(left);
    for (; tile < tile_end; tile += step, --left) {
        priority.set(left);
        cpx v[16];
        if constexpr (kPrefetch) {
            typename T::Raw rx = nx, rh;
            if constexpr (kPerSignal) rh = nh;
            if (tile + step < tile_end) {
                io.load(nx, x, tile + step, batch);
                if constexpr (kPerSignal) io.load(nh, h, tile + step, batch);
            }
            if constexpr (kPerSignal) {
                io.stage(rh, hs);
                fft_registers<N, true>(hs, io.slot, io.t, w);
            }
            io.stage(rx, v);
        } else if constexpr (kPerSignal && kDirect) {
            const DirectIO<IO, N> dio(threadIdx.x);
            {
                typename DirectIO<IO, N>::Raw rh;
                dio.load(rh, h, tile, batch);
                dio.decode(rh, hs);
            }
            typename DirectIO<IO, N>::Raw rx;
            dio.load(rx, x, tile, batch);
            fft_registers<N, true>(hs, io.slot, io.t, w);
            dio.decode(rx, v);
        } else if constexpr (kPerSignal) {
            // The filter first, so its raw tile is dead before the signal's
            // arrives; float2 issues the signal's loads before transforming
            // the filter, half2 (tighter on registers) after.
            {
                typename T::Raw rh;
                io.load(rh, h, tile, batch);
                io.stage(rh, hs);
            }
            typename T::Raw rx;
            if constexpr (std::is_same_v<IO, float2>) {
                io.load(rx, x, tile, batch);
                fft_registers<N, true>(hs, io.slot, io.t, w);
            } else {
                fft_registers<N, true>(hs, io.slot, io.t, w);
                io.load(rx, x, tile, batch);
            }
            io.stage(rx, v);
        } else {
            typename T::Raw rx;
            io.load(rx, x, tile, batch);
            io.stage(rx, v);
        }
        fft_registers<N, true>(v, io.slot, io.t, w);
#pragma unroll
        for (int j = 0; j < 16; ++j)
            v[j] = kPerSignal ? cmul(v[j], cpx{hs[j].re * kScale, hs[j].im * kScale})
                             : cmul(v[j], hs[j]);
        fft_registers<N, false>(v, io.slot, io.t, w);
        if constexpr (kDirect)
            DirectIO<IO, N>(threadIdx.x).store(v, y, tile, batch);
        else
            io.store(v, y, tile, batch);
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// conv2d: y[b] = IFFT2(FFT2(x[b]) * FFT2(h)) / (64*64) for 64 x 64 row-major
// images and one shared 64 x 64 filter h, i.e. the 2-D circular convolution
// y[b][r][c] = sum x[b][r'][c'] * h[(r - r') mod 64][(c - c') mod 64].
// Reference: sample/conv2d/thunder.cu:70-207 (row FFT, column FFT x H, column
// IFFT, row IFFT as three launches over a 1024 x 1024 image) and the unbuilt
// 64 x 64 tile sketch sample/conv2d/thunder_tile64.cu:33-208.
//
// One image is one workgroup tile.  Both indices split as r = r0 + 4 r1,
// c = c0 + 4 c1 (r0, c0 < 4; r1, c1 < 16), and the 2-D DFT runs as four
// stages, two 16-point and two 4-point ones, in three lane layouts:
//   L0  wave r0, lane c:            v[r1]  = x[r0 + 4 r1][c]
//       DFT16 over r1 -> kr1; wave-local LDS exchange E1 ->
//   L1  wave r0, lane (c0, kr1):    v[c1]
//       DFT16 over c1 -> kc1; workgroup LDS exchange E2 ->
//   L2  lane (kr1, kc1):            v[4 r0 + c0]
//       twiddles W64^(c0 kc1), DFT4 over c0; W64^(r0 kr1), DFT4 over r0:
//       v[4 kr0 + kc0] = X[kr1 + 16 kr0][kc1 + 16 kc0].
// The filter spectrum is built by the same steps once per workgroup, so the
// product is lane-local, and the inverse runs the stages backwards through
// the same layouts (X[k][l] -> exp(+2 pi i (r k + c l)/64) factors the same
// way).  Loads and stores move whole rows: in L0 one instruction of a wave
// reads or writes 64 consecutive values of row r0 + 4 r1, so images go from
// HBM to registers and back with no staging, and a 2-D transform takes two
// LDS exchanges (the row/column form takes three plus the staging).
// ---------------------------------------------------------------------------
namespace conv2d {
// E1: per-wave region, row kr1 of 64 values at kr1 * kE1 (66 = 2 mod 32
// 8-byte words: the L1 reads of 32 lanes (c0 in {0,1} or {2,3}, kr1 < 16) hit
// 32 distinct word positions mod 32, i.e. all 64 banks once).
inline constexpr int kE1 = 66;
inline constexpr int kE1Wave = 16 * kE1;
// E2: value (r0, c0, kr1, kc1) at (4 r0 + c0) * kM + 17 kr1 + kc1.  L1 writes
// of 32 lanes (c0 parity fixed, kr1 < 16) land on 17 kr1 + 16 c0 mod 32, all
// distinct; L2 reads of 32 lanes (two kr1, kc1 < 16) share one word position.
inline constexpr int kM = 272;
inline constexpr int kLds = 16 * kM > 4 * kE1Wave ? 16 * kM : 4 * kE1Wave;

// The lane's twiddle bases (positive angle, conjugated at use for forward):
// wr[i] = W64^((i + 1) kr1), wc[i] = W64^((i + 1) kc1) of its L2 position.
struct Twiddles {
    cpx wr[3], wc[3];
    __device__ __forceinline__ void load(int tid, const float2* __restrict__ tw) {
        const int kr1 = tid >> 4, kc1 = tid & 15;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const float2 a = tw[((i + 1) * kr1) & 63], b = tw[((i + 1) * kc1) & 63];
            wr[i] = {a.x, a.y};
            wc[i] = {b.x, b.y};
        }
    }
};

template <bool FWD>
__device__ __forceinline__ cpx twiddle(cpx a, cpx w) {
    return FWD ? cmulc(a, w) : cmul(a, w);
}

// DFT4 over c0 (stride 1 in v) for every r0, or over r0 (stride 4) for every c0.
template <bool FWD, int kStride, int kStep>
__device__ __forceinline__ void dft4s(cpx (&v)[16]) {
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        cpx t[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] = v[o * kStep + i * kStride];
        Dft<4, FWD>::run(t);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[o * kStep + i * kStride] = t[i];
    }
}

// L0 image -> L2 spectrum.
__device__ __forceinline__ void forward(cpx (&v)[16], cpx* lds, int tid, const Twiddles& w) {
    const int wave = tid >> 6, lane = tid & 63, c0 = lane >> 4, kr1 = lane & 15;
    cpx* e1 = lds + wave * kE1Wave;
    Dft<16, true>::run(v);  // over r1
#pragma unroll
    for (int k = 0; k < 16; ++k) e1[k * kE1 + lane] = v[k];
    wave_lds_sync();
#pragma unroll
    for (int c1 = 0; c1 < 16; ++c1) v[c1] = e1[kr1 * kE1 + c0 + 4 * c1];
    Dft<16, true>::run(v);  // over c1
    __syncthreads();        // every wave is done with its E1 reads
    cpx* m = lds + (4 * wave + c0) * kM + 17 * kr1;
#pragma unroll
    for (int k = 0; k < 16; ++k) m[k] = v[k];
    __syncthreads();
    const cpx* q = lds + 17 * (tid >> 4) + (tid & 15);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = q[i * kM];
#pragma unroll
    for (int r0 = 0; r0 < 4; ++r0)
#pragma unroll
        for (int c = 1; c < 4; ++c) v[4 * r0 + c] = twiddle<true>(v[4 * r0 + c], w.wc[c - 1]);
    dft4s<true, 1, 4>(v);  // over c0
#pragma unroll
    for (int r0 = 1; r0 < 4; ++r0)
#pragma unroll
        for (int k = 0; k < 4; ++k) v[4 * r0 + k] = twiddle<true>(v[4 * r0 + k], w.wr[r0 - 1]);
    dft4s<true, 4, 1>(v);  // over r0
}

// L2 spectrum -> L0 image (unnormalized inverse).  The caller's next LDS use
// must follow a __syncthreads() or be this wave's own E1 region.
__device__ __forceinline__ void inverse(cpx (&v)[16], cpx* lds, int tid, const Twiddles& w) {
    const int wave = tid >> 6, lane = tid & 63, c0 = lane >> 4, kr1 = lane & 15;
    dft4s<false, 4, 1>(v);  // over kr0
#pragma unroll
    for (int r0 = 1; r0 < 4; ++r0)
#pragma unroll
        for (int k = 0; k < 4; ++k) v[4 * r0 + k] = twiddle<false>(v[4 * r0 + k], w.wr[r0 - 1]);
    dft4s<false, 1, 4>(v);  // over kc0
#pragma unroll
    for (int r0 = 0; r0 < 4; ++r0)
#pragma unroll
        for (int c = 1; c < 4; ++c) v[4 * r0 + c] = twiddle<false>(v[4 * r0 + c], w.wc[c - 1]);
    __syncthreads();  // every wave is done with its E2 reads
    cpx* q = lds + 17 * (tid >> 4) + (tid & 15);
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i * kM] = v[i];
    __syncthreads();
    const cpx* m = lds + (4 * wave + c0) * kM + 17 * kr1;
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = m[k];
    Dft<16, false>::run(v);  // over kc1
    __syncthreads();         // every wave is done with its E2' reads
    cpx* e1 = lds + wave * kE1Wave;
#pragma unroll
    for (int c1 = 0; c1 < 16; ++c1) e1[kr1 * kE1 + c0 + 4 * c1] = v[c1];
    wave_lds_sync();
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = e1[k * kE1 + lane];
    Dft<16, false>::run(v);  // over kr1
}

// Image `img` of `base` in L0, as loaded (raw[r1] = base[img][wave + 4 r1][lane])
// and decoded to v[r1].
template <class IO>
struct Raw {
    typename Io<IO>::W1 w[16];
};

// Image img as a buffer resource of its 4096 values: one lane offset serves
// all 16 accesses of a lane, the 256-element steps go in the scalar offset
// (cache policy 2: non-temporal).  With 64-bit per-lane pointers instead, the
// fp32 kernel kept one in scratch at its 128-VGPR budget and reloaded it
// behind an s_waitcnt vmcnt(0) each image: 96.4 against 97.8-98.4 us for
// 8192 images.  Every offset stays inside the image (tid * 8 + 15 * 2048 + 8
// <= 32 KiB), so the resource's bounds never clip an access.
template <class IO>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t image_rsrc(const IO* base, long long img) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<IO*>(base + img * 4096), 0,
                                             static_cast<int>(4096 * sizeof(IO)), 0x00020000);
}

template <class IO>
__device__ __forceinline__ void load(Raw<IO>& r, const IO* __restrict__ base, long long img,
                                     int tid) {
    using W = typename Io<IO>::W1;
    const __amdgpu_buffer_rsrc_t rs = image_rsrc(base, img);
    const int off = tid * static_cast<int>(sizeof(W));
#pragma unroll
    for (int r1 = 0; r1 < 16; ++r1) {
        if constexpr (sizeof(W) == 8)
            r.w[r1] = __builtin_bit_cast(W, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 256 * 8 * r1, 2));
        else
            r.w[r1] = __builtin_bit_cast(W, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 256 * 4 * r1, 2));
    }
}

template <class IO>
__device__ __forceinline__ void decode(const Raw<IO>& r, cpx (&v)[16]) {
#pragma unroll
    for (int r1 = 0; r1 < 16; ++r1) v[r1] = Io<IO>::decode1(r.w[r1]);
}

template <class IO>
__device__ __forceinline__ void store(const cpx (&v)[16], IO* __restrict__ base, long long img,
                                      int tid) {
    using W = typename Io<IO>::W1;
    const __amdgpu_buffer_rsrc_t rs = image_rsrc<IO>(base, img);
    const int off = tid * static_cast<int>(sizeof(W));
#pragma unroll
    for (int r1 = 0; r1 < 16; ++r1) {
        const W w = Io<IO>::encode1(v[r1]);
        if constexpr (sizeof(W) == 8)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, w), rs, off, 256 * 8 * r1, 2);
        else
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, w), rs, off, 256 * 4 * r1, 2);
    }
}
}  // namespace conv2d

// The next image's loads are issued before the current image is transformed.
// Held to 4 waves per SIMD (4 workgroups per CU), which the fp32 kernel fits
// without spilling since its image accesses are buffer instructions (above).
// Measured on MI355X, 8192 fp32 images, when it still kept 2 dwords in
// scratch: 101-104 us, against 103-106 us at its natural 129 VGPRs (3 per CU)
// and 104-107 us without the prefetch.
template <class IO>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void
conv2d64_kernel(const IO* __restrict__ x, const IO* __restrict__ h, IO* __restrict__ y,
                int batch, const float2* __restrict__ tw, int tiles_per_block) {
    __shared__ cpx lds[conv2d::kLds];
    const int tid = threadIdx.x;
    conv2d::Twiddles w;
    w.load(tid, tw);
    constexpr float kScale = 1.0f / 4096.0f;

    long long img, img_end, step;
    tile_walk(batch, tiles_per_block, img, img_end, step);
    if (img >= img_end) return;  // uniform over the workgroup

    conv2d::Raw<IO> raw;
    cpx hs[16];  // FFT2(h) / 4096 in the L2 layout
    conv2d::load(raw, h, 0, tid);
    conv2d::decode(raw, hs);
    conv2d::load(raw, x, img, tid);
    conv2d::forward(hs, lds, tid, w);
#pragma unroll
    for (int i = 0; i < 16; ++i) hs[i] = {hs[i].re * kScale, hs[i].im * kScale};
    __syncthreads();  // the filter's E2 reads are done before the first E1 writes
    long long left = (img_end - img + step - 1) / step;  // tiles still to do, this one included
    const ProgressPriority priority(left);
    for (; img < img_end; img += step, --left) {
        priority.set(left);
        cpx v[16];
        conv2d::decode(raw, v);
        if (img + step < img_end) conv2d::load(raw, x, img + step, tid);
        conv2d::forward(v, lds, tid, w);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = cmul(v[i], hs[i]);
        conv2d::inverse(v, lds, tid, w);
        conv2d::store(v, y, img, tid);
    }
}

// ---------------------------------------------------------------------------
// fp32 2-D circular convolution of 128 x 128 images with one shared filter
// (y = IFFT2(FFT2(x) * FFT2(h)) / 16384, the contract of conv2d64_kernel; the
// reference's 128-tile sketch is sample/conv2d/thunder_tile128.cu:64-237) in
// four lane layouts, one image per 1024-lane workgroup, 16 values per lane.
// Both indices split as r = r0 + 8 r1, c = c0 + 8 c1 (r0, c0 < 8), and each
// wave has one digit u = w mod 8 that is constant over its lanes, so every
// twiddle it applies is one of 16 wave-uniform values W128^(u k):
//   L0  lane (r0 = u, c = 64 (w / 8) + l): x[r0 + 8 j][c], j = r1 -- loaded
//       and stored straight from registers, each instruction 64 consecutive
//       values of one row; DFT16 over r1, times W128^(r0 kr1);
//   L1  lane (kr1 in {u, u + 8}, c): the 8 values over r0 of both kr1 (an
//       exchange within the 8 waves of one column half); two DFT8 over r0
//       -> X[kr = kr1 + 16 kr0][c];
//   L2  lane (c0 = u, kr = 64 (w / 8) + l): X[kr][c0 + 8 j], j = c1 (the
//       transpose, through a column-major buffer of stride 129); DFT16 over
//       c1, times W128^(c0 kc1);
//   L3  lane (kc1 in {u, u + 8}, kr): the 8 values over c0 of both kc1; two
//       DFT8 over c0 -> spectrum S[kr][kc1 + 16 kc0].
// The product with the filter spectrum (the same steps on h once per
// workgroup, x 1/16384, fp32 registers) is lane-local, and the inverse runs
// the steps backwards.  Every exchange moves 8-byte values with 64
// consecutive lanes on 64 consecutive (or 129-strided) slots: no bank
// conflicts.  One 129 KiB buffer serves all six exchanges, each between two
// workgroup barriers; the next image is loaded into registers while the
// current one is transformed (half before the forward transform, half
// before the inverse: 127 VGPRs, no spill).  2048 images on MI355X: 134 us,
// against 183 us for a row/column form that kept the image in LDS (two
// barriers per image, but only a quarter of the next image prefetched).
// ---------------------------------------------------------------------------
namespace conv2d128l {
constexpr int kN = 128;
constexpr int kT = 129;  // column stride of the transpose buffer
constexpr int kLds = kN * kT;

// a[k] *= t[k] (forward) or conj(t[k]) for k = 1..15 (the wave-uniform
// factors of this layout).
template <bool FWD>
__device__ __forceinline__ void twiddle(cpx (&a)[16], const cpx (&t)[16]) {
#pragma unroll
    for (int k = 1; k < 16; ++k) a[k] = FWD ? cmul(a[k], t[k]) : cmulc(a[k], t[k]);
}

// The forward 2-D DFT of the image held in L0 order (a[j] = x[u + 8 j][c]),
// through L: on return a[8 s + kc0] = S[kr][u + 8 s + 16 kc0], kr = c.
__device__ __forceinline__ void forward(cpx (&a)[16], cpx* L, int u, int c, const cpx (&t)[16]) {
    Dft<16, true>::run(a);
    twiddle<true>(a, t);
    __syncthreads();  // earlier readers of L are done
#pragma unroll
    for (int k = 0; k < 16; ++k) L[(u * 16 + k) * kN + c] = a[k];
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 8; ++r) a[8 * s + r] = L[(r * 16 + u + 8 * s) * kN + c];
    Dft<8, true>::run(a);
    Dft<8, true>::run(a + 8);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int k = 0; k < 8; ++k) L[c * kT + u + 8 * s + 16 * k] = a[8 * s + k];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) a[j] = L[(u + 8 * j) * kT + c];
    Dft<16, true>::run(a);
    twiddle<true>(a, t);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) L[(u * 16 + k) * kN + c] = a[k];
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 8; ++r) a[8 * s + r] = L[(r * 16 + u + 8 * s) * kN + c];
    Dft<8, true>::run(a);
    Dft<8, true>::run(a + 8);
}

// The inverse of forward (unnormalized): spectrum order in, L0 order out.
__device__ __forceinline__ void inverse(cpx (&a)[16], cpx* L, int u, int c, const cpx (&t)[16]) {
    Dft<8, false>::run(a);
    Dft<8, false>::run(a + 8);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 8; ++r) L[(r * 16 + u + 8 * s) * kN + c] = a[8 * s + r];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) a[k] = L[(u * 16 + k) * kN + c];
    twiddle<false>(a, t);
    Dft<16, false>::run(a);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) L[(u + 8 * j) * kT + c] = a[j];
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int k = 0; k < 8; ++k) a[8 * s + k] = L[c * kT + u + 8 * s + 16 * k];
    Dft<8, false>::run(a);
    Dft<8, false>::run(a + 8);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 8; ++r) L[(r * 16 + u + 8 * s) * kN + c] = a[8 * s + r];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) a[k] = L[(u * 16 + k) * kN + c];
    twiddle<false>(a, t);
    Dft<16, false>::run(a);
}
}  // namespace conv2d128l

template <int kUnused = 0>
__global__ __launch_bounds__(1024) void conv2d128_lanes_kernel(const float2* __restrict__ x,
                                                               const float2* __restrict__ h,
                                                               float2* __restrict__ y, int batch,
                                                               const float2* __restrict__ tw) {
    using namespace conv2d128l;
    constexpr int kImg = kN * kN;
    __shared__ cpx L[kLds];
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u = w & 7;
    const int c = 64 * (w >> 3) + (tid & 63);
    // W128^(u k) (forward: the conjugate of the positive-angle table).
    cpx t[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float2 v = tw[(u * k) & (kN - 1)];
        t[k] = {v.x, -v.y};
    }
    long long img, img_end, step;
    tile_walk(batch, 0, img, img_end, step);
    if (img >= img_end) return;  // uniform over the workgroup

    auto load = [&](const float2* src, cpx (&a)[16]) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const u32x2 v = ld_nt(reinterpret_cast<const u32x2*>(src + (u + 8 * j) * kN + c));
            a[j] = Io<float2>::decode1(v);
        }
    };
    // The image's values and the next image's alternate between two register
    // sets (the loop is unrolled by two, so no set is copied): the next
    // image's loads are issued before the current one is transformed, with
    // no branch (the last pass's go through a resource of no bytes and read
    // zeros without touching memory), and 16 stores to a
    // resource of no bytes after the first loads make the loop's entry look
    // like every later pass (the loads followed by 16 stores in flight), so
    // the compiler waits at the top of a pass for that pass's loads only,
    // not for the previous image's stores.
    // Buffer accesses: the image's resource in scalar registers, the lane's
    // offset in one VGPR, the row step j in the scalar offset.
    const int voff = 8 * (u * kN + c);
    auto load_img = [&](long long im, cpx (&a)[16], int j0 = 0, int j1 = 16, bool live = true) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float2*>(x + im * kImg), 0, live ? kImg * 8 : 0, 0x00020000);
#pragma unroll
        for (int j = j0; j < j1; ++j)
            a[j] = Io<float2>::decode1(__builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, voff, 64 * kN * j, 2)));
    };
    cpx hs[16], va[16], vb[16];
    load(h, hs);
    load_img(img, va);
    {
        const __amdgpu_buffer_rsrc_t none =
            __builtin_amdgcn_make_buffer_rsrc(y, 0, batch < 0 ? 16 : 0, 0x00020000);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 16; ++j)
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{}, none, 0, 64 * kN * j, 2);
    }
    forward(hs, L, u, c, t);
    constexpr float kScale = 1.0f / kImg;
#pragma unroll
    for (int k = 0; k < 16; ++k) hs[k] = {hs[k].re * kScale, hs[k].im * kScale};
    auto pass = [&](cpx (&a)[16], cpx (&nxt)[16]) {
        const bool live = img + step < img_end;
        const long long nim = live ? img + step : img;
        load_img(nim, nxt, 0, 8, live);
        forward(a, L, u, c, t);
#pragma unroll
        for (int k = 0; k < 16; ++k) a[k] = cmul(a[k], hs[k]);
        load_img(nim, nxt, 8, 16, live);
        inverse(a, L, u, c, t);
        const __amdgpu_buffer_rsrc_t ys =
            __builtin_amdgcn_make_buffer_rsrc(y + img * kImg, 0, kImg * 8, 0x00020000);
#pragma unroll
        for (int j = 0; j < 16; ++j)
            __builtin_amdgcn_raw_buffer_store_b64(Io<float2>::encode1(a[j]), ys, voff, 64 * kN * j, 2);
        img += step;
    };
    while (img < img_end) {
        pass(va, vb);
        if (img >= img_end) break;
        pass(vb, va);
    }
}

// ---------------------------------------------------------------------------
// Column pass of the multi-pass 2-D convolution of images too large for one
// workgroup (R x C = 1024 x 1024 here; the reference's built 2-D convolution
// is the same split, sample/conv2d/thunder.cu:70-207: row FFT kernel, a
// column kernel that runs FFT x H x IFFT, an inverse row kernel).  The row
// passes are the library's C2C kernels; this kernel does the columns.
// A workgroup of 512 lanes takes 8 adjacent columns of one image (a unit):
// it loads the R x 8 block in 16-byte pieces of whole rows (64 bytes per row
// fp32, 32 half), stages it column by column into LDS slots, and wave w
// transforms column c0 + w (R / 16 = 64 lanes, 16 values each) in its slot:
//   kConv:  out = IFFT_col(FFT_col(in) * H[., c0 + w])  (H fp32, R x C)
//   !kConv: out = scale * FFT_col(in)                   (a filter's spectrum)
// then stages the results back and stores them the way they came.  In and
// out may be the same buffer (each unit reads its block before writing it).
// Units are walked grid-stride; with a grid that is a multiple of the column
// blocks per image, a workgroup keeps one column block for every image, so
// its H column is loaded once and held in registers.  Slots are kSlotStride
// apart (2 kSlotStride = 8 mod 64 banks), so the staging accesses of a
// half-wave (4 columns x 8 rows) fall on distinct banks.  The next unit's
// pieces are loaded before the current unit is transformed: held to 2 waves
// per SIMD (one workgroup per CU), the kernel keeps its block, the next
// block and the H column in registers without spilling (at 4 per SIMD the
// forward and inverse column transforms alone spill).
// ---------------------------------------------------------------------------
namespace conv2dcols {
template <int R>
inline constexpr int kSlotStride = C2CPlan<R>::kSlot + 4;

// Cols columns per unit, moved by kLanes lanes in 16-byte row pieces.
template <class IO, int R, int Cols, int kLanes = 64 * Cols>
struct Block {
    static constexpr int kVec = Io<IO>::kVec;
    static constexpr int kPer = Cols / kVec;                 // pieces per row
    static constexpr int kRowsPerStep = kLanes / kPer;       // rows per lane step
    static constexpr int kCount = R / kRowsPerStep;     // pieces per lane
    typename Io<IO>::W4 w[kCount];
};

template <int First, int Last, int C, class IO, int R, int Cols, int L>
__device__ __forceinline__ void load(Block<IO, R, Cols, L>& b, const IO* in, long long base, int tid) {
    constexpr long long cols = C;
    using B = Block<IO, R, Cols, L>;
    const int p = tid % B::kPer, r0 = tid / B::kPer;
#pragma unroll
    for (int i = First; i < Last; ++i) {
        const long long e = base + static_cast<long long>(r0 + B::kRowsPerStep * i) * cols + B::kVec * p;
        b.w[i] = ld_nt(reinterpret_cast<const typename Io<IO>::W4*>(in + e));
    }
}

template <class IO, int R, int Cols, int L>
__device__ __forceinline__ void stage(const Block<IO, R, Cols, L>& b, cpx* lds, int tid) {
    using B = Block<IO, R, Cols, L>;
    const int p = tid % B::kPer, r0 = tid / B::kPer;
#pragma unroll
    for (int i = 0; i < B::kCount; ++i) {
        cpx q[B::kVec];
        Io<IO>::decode4(b.w[i], q);
#pragma unroll
        for (int c = 0; c < B::kVec; ++c)
            lds[(B::kVec * p + c) * kSlotStride<R> + lds_pad(r0 + B::kRowsPerStep * i)] = q[c];
    }
}

template <int C, class IO, int R, int Cols, int L = 64 * Cols>
__device__ __forceinline__ void store(IO* out, long long base, const cpx* lds, int tid) {
    constexpr long long cols = C;
    using B = Block<IO, R, Cols, L>;
    const int p = tid % B::kPer, r0 = tid / B::kPer;
#pragma unroll
    for (int i = 0; i < B::kCount; ++i) {
        cpx q[B::kVec];
#pragma unroll
        for (int c = 0; c < B::kVec; ++c)
            q[c] = lds[(B::kVec * p + c) * kSlotStride<R> + lds_pad(r0 + B::kRowsPerStep * i)];
        const long long e = base + static_cast<long long>(r0 + B::kRowsPerStep * i) * cols + B::kVec * p;
        st_nt(reinterpret_cast<typename Io<IO>::W4*>(out + e), Io<IO>::encode4(q));
    }
}
}  // namespace conv2dcols

// Waves per SIMD: 8 columns per unit (512 lanes, one wave per column) hold
// two, with the next unit's block prefetched; 16 columns (512 lanes, two
// columns per wave) two, loading each block when its unit starts (the
// prefetch would spill there); 4 columns (256 lanes) three, likewise.
template <int Cols>
inline constexpr int kColsWavesPerEU = Cols == 8 || Cols == 16 ? 2 : 3;
template <int Cols>
inline constexpr bool kColsPrefetch = Cols == 8;
// Lanes per workgroup: one wave per column up to 8 columns; 16 columns are
// 8 waves of two columns each.
template <int Cols>
inline constexpr int kColsLanes = Cols <= 8 ? 64 * Cols : 512;

template <class In, class Out, int R, int C, bool kConv, int Cols>
__global__ __launch_bounds__(kColsLanes<Cols>) __attribute__((amdgpu_waves_per_eu(kColsWavesPerEU<Cols>))) void
conv2d_cols_kernel(const In* in, Out* out, const float2* __restrict__ H, long long units,
                   float scale, const float2* __restrict__ tw) {
    using P = C2CPlan<R>;
    static_assert(P::kTPF == 64, "one wave per column");
    using namespace conv2dcols;
    constexpr int kL = kColsLanes<Cols>;
    constexpr int kWaves = kL / 64;
    constexpr int kCPW = Cols / kWaves;  // columns per wave
    __shared__ __align__(16) cpx lds[Cols * kSlotStride<R>];
    const int tid = threadIdx.x, wave = tid >> 6, t = tid & 63;
    LaneTwiddles<R> w;
    w.load(t, tw);
    constexpr long long cols = C;
    constexpr long long blocks_per_image = C / Cols;
    constexpr int kAll = Block<In, R, Cols, kL>::kCount;

    // A 128-byte line of a row holds kShare adjacent column blocks.  Work
    // items u = b + k G are renamed within aligned groups of 8 kShare so that
    // workgroups b, b + 8, b + 16, ... -- dispatched to the same XCD -- take
    // the kShare blocks of one line: the line is then fetched into one XCD's
    // L2 once instead of once per XCD (with consecutive blocks on consecutive
    // XCDs, FETCH_SIZE read 2x the data for fp32, 4x for half).
    constexpr int kShare = 128 / (Cols * static_cast<int>(sizeof(In))) > 1
                               ? 128 / (Cols * static_cast<int>(sizeof(In))) : 1;
    constexpr int kGroup = 8 * kShare;
    static_assert(blocks_per_image % kGroup == 0, "column blocks per image: whole groups");
    auto where = [&](long long u0, long long& base, int& c0) {
        const int i = static_cast<int>(u0 % kGroup);
        const long long u = u0 - i + kShare * (i % 8) + i / 8;
        const long long img = u / blocks_per_image;
        c0 = static_cast<int>(u - img * blocks_per_image) * Cols;
        base = img * R * static_cast<long long>(cols) + c0;
    };
    long long u = blockIdx.x;
    if (u >= units) return;  // uniform over the workgroup
    long long base;
    int c0;
    where(u, base, c0);
    Block<In, R, Cols, kL> raw;
    if constexpr (kColsPrefetch<Cols>) load<0, kAll, C>(raw, in, base, tid);
    int h_c0 = -1;
    cpx hs[kCPW][kConv ? 16 : 1];
    for (; u < units; u += gridDim.x) {
        const long long next_u = u + gridDim.x;
        long long next_base = 0;
        int next_c0 = 0;
        if (next_u < units) where(next_u, next_base, next_c0);
        if constexpr (!kColsPrefetch<Cols>) load<0, kAll, C>(raw, in, base, tid);
        __syncthreads();  // the previous unit's reads of the slots are done
        stage(raw, lds, tid);
        if constexpr (kColsPrefetch<Cols>)
            if (next_u < units) load<0, kAll, C>(raw, in, next_base, tid);
        if constexpr (kConv) {
            if (c0 != h_c0) {  // uniform: this workgroup's column block changed
#pragma unroll
                for (int v = 0; v < kCPW; ++v) {
                    const float2* hc = H + c0 + wave + kWaves * v;
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float2 hk = hc[static_cast<long long>(t + 64 * j) * cols];
                        hs[v][j] = {hk.x, hk.y};
                    }
                }
                h_c0 = c0;
            }
        }
        __syncthreads();
#pragma unroll
        for (int cv = 0; cv < kCPW; ++cv) {
            cpx* const slot = lds + (wave + kWaves * cv) * kSlotStride<R>;
            cpx v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = slot[lds_pad(t + 64 * j)];
            fft_registers<R, true>(v, slot, t, w);
            if constexpr (kConv) {
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = cmul(v[j], hs[cv][j]);
                fft_registers<R, false>(v, slot, t, w);
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = {v[j].re * scale, v[j].im * scale};
            }
            wave_lds_sync();
#pragma unroll
            for (int j = 0; j < 16; ++j) slot[lds_pad(t + 64 * j)] = v[j];
        }
        __syncthreads();
        store<C, Out, R, Cols, kL>(out, base, lds, tid);
        base = next_base;
        c0 = next_c0;
    }
}

// ---------------------------------------------------------------------------
// Real-input, real-output fused convolution with one real filter per channel
// (the reference's thunder_convN_block_kernel_realin_realout,
// sample/conv1d/conv1d_fullfft_l4096_thunder.cu:280-331, generalised to all
// seven lengths and both storage types):
//   y[b][d] = IFFT(FFT(x[b][d]) * H[d])   (length N), x, y real [batch][D][N].
// Because h is real, two signals of one channel share a complex transform:
// z = x[2p][d] + i x[2p+1][d] gives z (*) h = x[2p][d] (*) h + i x[2p+1][d] (*) h,
// so complex transform tau = p*D + d carries both, and the real and
// imaginary parts of its result are the two outputs.  The filter spectra
// H[d][k] = scale * FFT(h[d])[k] (fp32 complex, natural order) are prepared
// once by conv1d_real_filter_kernel; the convolution kernel then writes
// IFFT(FFT(x) * H) unnormalized, which with scale = 1 is N * (x (*) h), the
// reference's output, and with scale = 1/N is x (*) h itself.  The pairing
// needs H[d] to be Hermitian (H[k] = conj H[N - k]), which every spectrum of a
// real filter is.
// ---------------------------------------------------------------------------

// Real scalars of one storage type: 16-byte vectors of kVec values.
template <class IO>
struct RealIo;
template <>
struct RealIo<float2> {
    using S = float;
    static constexpr int kVec = 4;
    __device__ __forceinline__ static void decode(u32x4 w, float* v) {
        v[0] = as_f32(w.x), v[1] = as_f32(w.y), v[2] = as_f32(w.z), v[3] = as_f32(w.w);
    }
    __device__ __forceinline__ static u32x4 encode(const float* v) {
        return u32x4{as_u32(v[0]), as_u32(v[1]), as_u32(v[2]), as_u32(v[3])};
    }
};
template <>
struct RealIo<__half2> {
    using S = __half;
    static constexpr int kVec = 8;
    __device__ __forceinline__ static void decode(u32x4 w, float* v) {
        const unsigned u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 f = __half22float2(__builtin_bit_cast(__half2, u[i]));
            v[2 * i] = f.x, v[2 * i + 1] = f.y;
        }
    }
    __device__ __forceinline__ static u32x4 encode(const float* v) {
        unsigned u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            u[i] = __builtin_bit_cast(unsigned, __floats2half2_rn(v[2 * i], v[2 * i + 1]));
        return u32x4{u[0], u[1], u[2], u[3]};
    }
};

// Position of transform tau = p * channels + d of the real convolutions
// (row pair p, channel d) on a tile walk whose successive tiles are `adv`
// transforms apart: positions advance without a 64-bit division per tile,
// and transform tau + k (k small) is located with one 32-bit division.
struct ChannelPos {
    long long p;
    int d;
};
struct ChannelWalk {
    long long adv_p;
    int adv_d;
    int channels;
    __host__ __device__ __forceinline__ ChannelWalk(long long adv, int ch) : channels(ch) {
        adv_p = adv / ch;
        adv_d = static_cast<int>(adv - adv_p * ch);
    }
    __host__ __device__ __forceinline__ ChannelPos at(long long tau) const {
        const long long p = tau / channels;
        return {p, static_cast<int>(tau - p * channels)};
    }
    // (adv_d < channels and q.d < channels: at most one carry)
    __host__ __device__ __forceinline__ ChannelPos advance(ChannelPos q) const {
        q.p += adv_p;
        q.d += adv_d;
        if (q.d >= channels) q.d -= channels, ++q.p;
        return q;
    }
    __host__ __device__ __forceinline__ void locate(ChannelPos q, int k, long long& pair, int& chan) const {
        const unsigned s = static_cast<unsigned>(q.d) + static_cast<unsigned>(k);
        const unsigned c = static_cast<unsigned>(channels);
        const unsigned j = s / c;
        pair = q.p + j;
        chan = static_cast<int>(s - j * c);
    }
};

// H[d][k] = scale * FFT(h[d])[k] for `channels` real fp32 filters h[d] of N
// taps (fp32 for both storage types, so half convolutions keep exact taps).
template <int N>
__global__ __launch_bounds__(256) void conv1d_real_filter_kernel(const float* __restrict__ h,
                                                                 float2* __restrict__ spectrum,
                                                                 int channels, float scale,
                                                                 const float2* __restrict__ tw) {
    using P = C2CPlan<N>;
    __shared__ cpx lds[P::kLdsSlots];
    const int tid = threadIdx.x, f = tid / P::kTPF, t = tid % P::kTPF;
    cpx* slot = lds + f * P::kSlot;
    LaneTwiddles<N> w;
    w.load(t, tw);
    const long long d = static_cast<long long>(blockIdx.x) * P::kFPB + f;
    const bool ok = d < channels;
    cpx v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        v[j] = {ok ? h[d * N + t + j * P::kTPF] : 0.f, 0.f};
    }
    fft_registers<N, true>(v, slot, t, w);
    if (ok) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
            spectrum[d * N + t + j * P::kTPF] = make_float2(v[j].re * scale, v[j].im * scale);
    }
}

// kDirect (float, N >= 1024; used for N >= 2048): lane t of a transform loads samples
// t + TPF*j of both rows straight into its first-pass registers (4-byte
// accesses, 64 consecutive samples per wave instruction) and stores the
// real and imaginary parts of its last-pass registers the same way, with no
// LDS staging.
template <class IO, int N, Prefetch kPf = Prefetch::kNone, bool kDirect = false>
__global__ __launch_bounds__(256) void conv1d_real_kernel(
    const typename RealIo<IO>::S* __restrict__ x, const float2* __restrict__ spectrum,
    typename RealIo<IO>::S* __restrict__ y, int batch, int channels,
    const float2* __restrict__ tw, int tiles_per_block) {
    using P = C2CPlan<N>;
    using R = RealIo<IO>;
    constexpr int kVec = R::kVec;
    // A tile is kFPB complex transforms = 4096 complex values; value e
    // (transform e / N, element e % N) is staged at LDS position lds_pad(e),
    // which is where the transform's slot expects it.  Wave w moves values
    // [1024 w, 1024 (w + 1)), which for N <= 1024 are exactly the transforms
    // its own lanes compute; lane l takes kVec of them per step, from the
    // same offset of both rows of a pair.
    constexpr int kSteps = 1024 / (64 * kVec);
    __shared__ cpx lds[P::kLdsSlots];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int f = tid / P::kTPF, t = tid % P::kTPF;
    cpx* slot = lds + f * P::kSlot;
    LaneTwiddles<N> w;
    w.load(t, tw);

    const long long pairs = (static_cast<long long>(batch) + 1) / 2;
    const long long transforms = pairs * channels;
    const long long ntiles = (transforms + P::kFPB - 1) / P::kFPB;
    long long tile, tile_end, step;
    tile_walk(ntiles, tiles_per_block, tile, tile_end, step);
    // N = 4096 (one transform per tile, device-sized grids, 2 waves per SIMD
    // already): the channel's spectrum stays in registers while the channel
    // does not change, instead of being read from L2 per tile.
    constexpr bool kKeepSpectrum = N == 4096;
    int spec_d = -1;
    cpx spec[kKeepSpectrum ? 16 : 1];

    // Position of a tile's first transform tau = tl * kFPB (ChannelWalk).
    using Pos = ChannelPos;
    const ChannelWalk walk(step * P::kFPB, channels);
    Pos pos = walk.at(tile * P::kFPB);
    auto advance = [&](Pos q) { return walk.advance(q); };
    auto locate = [&](Pos q, int k, long long& pair, int& chan) { walk.locate(q, k, pair, chan); };

    // This lane's kSteps 16-byte pieces of tile tl in both rows.  Piece i is
    // tile element e = u_i + kVec lane, u_i = 1024 wave + 64 kVec i: element
    // e % N of transform tl * kFPB + e / N.  For N >= 64 kVec the 64 lanes'
    // pieces i lie in one transform, so the row offsets of u_i are
    // wave-uniform (scalar) and a lane adds kVec lane; for N >= 1024 a wave's
    // 1024 elements lie in one transform and one offset per row serves every
    // piece.  Shorter transforms keep per-lane offsets.  -1: no such row.
    constexpr bool kUniform = N >= 64 * kVec;
    constexpr int kRowOffsets = N >= 1024 ? 1 : kSteps;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    struct Rows {
        long long o0[kRowOffsets], o1[kRowOffsets];
        u32x4 r0[kSteps], r1[kSteps];
    };
    auto piece = [&](const long long* o, int i) -> long long {
        if constexpr (N >= 1024)
            return o[0] < 0 ? -1 : o[0] + 64 * kVec * i + kVec * lane;
        else if constexpr (kUniform)
            return o[i] < 0 ? -1 : o[i] + kVec * lane;
        else
            return o[i];
    };
    auto fetch = [&](long long tl, Pos q, Rows& rw) {
#pragma unroll
        for (int i = 0; i < kRowOffsets; ++i) {
            const int e = kUniform ? 1024 * wave_u + (N >= 1024 ? 0 : 64 * kVec * i)
                                   : 1024 * wave + kVec * lane + 64 * kVec * i;
            const int k = e / N;
            const long long tau = tl * P::kFPB + k;
            long long pair;
            int chan;
            locate(q, k, pair, chan);
            const long long b0 = 2 * pair, b1 = b0 + 1;
            const int n = e % N;
            rw.o0[i] = tau < transforms ? (b0 * channels + chan) * N + n : -1;
            rw.o1[i] = tau < transforms && b1 < batch ? (b1 * channels + chan) * N + n : -1;
        }
#pragma unroll
        for (int i = 0; i < kSteps; ++i) {
            const long long a0 = piece(rw.o0, i), a1 = piece(rw.o1, i);
            rw.r0[i] = a0 >= 0 ? ld_nt(reinterpret_cast<const u32x4*>(x + a0)) : u32x4{};
            rw.r1[i] = a1 >= 0 ? ld_nt(reinterpret_cast<const u32x4*>(x + a1)) : u32x4{};
        }
    };
    static_assert(!kDirect || (std::is_same_v<IO, float2> && N >= 1024),
                  "direct real-conv movement: float, N >= 1024");
    // Direct movement: this lane's 16 samples of both rows of transform f of
    // tile tl (o0 / o1: offset of sample t of the row, -1: no such row).
    struct DRows {
        long long o0, o1;
        float r0[16], r1[16];
    };
    auto dfetch = [&](long long tl, Pos q, DRows& rw) {
        const long long tau = tl * P::kFPB + f;
        long long pair;
        int chan;
        locate(q, f, pair, chan);
        const long long b0 = 2 * pair, b1 = b0 + 1;
        rw.o0 = tau < transforms ? (b0 * channels + chan) * N + t : -1;
        rw.o1 = tau < transforms && b1 < batch ? (b1 * channels + chan) * N + t : -1;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            rw.r0[j] = rw.o0 >= 0 ? ld_nt(reinterpret_cast<const float*>(x) + rw.o0 + j * P::kTPF)
                                  : 0.f;
            rw.r1[j] = rw.o1 >= 0 ? ld_nt(reinterpret_cast<const float*>(x) + rw.o1 + j * P::kTPF)
                                  : 0.f;
        }
    };
    using RowsT = std::conditional_t<kDirect, DRows, Rows>;
    auto fetch_any = [&](long long tl, Pos q, RowsT& rw) {
        if constexpr (kDirect)
            dfetch(tl, q, rw);
        else
            fetch(tl, q, rw);
    };
    // The next tile's pieces load while the current tile is transformed
    // (kPf): early, right after the current tile's pieces are taken, or
    // late, after its product with the spectrum.
    RowsT next;
    if constexpr (kPf != Prefetch::kNone)
        if (tile < tile_end) fetch_any(tile, pos, next);

    for (; tile < tile_end; tile += step) {
        // ---- both rows of each transform -> (re, im) = (row 0, row 1) ----
        RowsT cur;
        const Pos at = pos;
        pos = advance(pos);
        if constexpr (kPf == Prefetch::kEarly) {
            cur = next;
            if (tile + step < tile_end) fetch_any(tile + step, pos, next);
        } else if constexpr (kPf == Prefetch::kLate) {
            if constexpr (kDirect) {
                cur.o0 = next.o0, cur.o1 = next.o1;
            } else {
#pragma unroll
                for (int i = 0; i < kRowOffsets; ++i) cur.o0[i] = next.o0[i], cur.o1[i] = next.o1[i];
            }
        } else {
            fetch_any(tile, at, cur);
        }
        const RowsT& src = kPf == Prefetch::kLate ? next : cur;
        cpx v[16];
        if constexpr (kDirect) {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = cpx{src.r0[j], src.r1[j]};
        } else {
            region_sync<P::kWaveLocal>();
#pragma unroll
            for (int i = 0; i < kSteps; ++i) {
                const int e = 1024 * wave + kVec * lane + 64 * kVec * i;
                float a[kVec], b[kVec];
                R::decode(src.r0[i], a);
                R::decode(src.r1[i], b);
#pragma unroll
                for (int c = 0; c < kVec; ++c) lds[lds_pad(e + c)] = cpx{a[c], b[c]};
            }
            region_sync<P::kWaveLocal>();
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = slot[lds_pad(t + j * P::kTPF)];
        }

        // ---- FFT, product with the channel's spectrum, inverse FFT ----
        // (a channel past the last transform too: always a valid spectrum row)
        long long pair_f;
        int d;
        locate(at, f, pair_f, d);
        fft_registers<N, true>(v, slot, t, w);
        if constexpr (kKeepSpectrum) {
            if (d != spec_d) {
                const float2* hs = spectrum + static_cast<long long>(d) * N + t;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float2 hk = hs[j * P::kTPF];
                    spec[j] = cpx{hk.x, hk.y};
                }
                spec_d = d;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = cmul(v[j], spec[j]);
        } else {
            const float2* hs = spectrum + static_cast<long long>(d) * N + t;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float2 hk = hs[j * P::kTPF];
                v[j] = cmul(v[j], cpx{hk.x, hk.y});
            }
        }
        if constexpr (kPf == Prefetch::kLate)
            if (tile + step < tile_end) fetch_any(tile + step, pos, next);
        fft_registers<N, false>(v, slot, t, w);

        // ---- real part -> row 0, imaginary part -> row 1 ----
        if constexpr (kDirect) {
            float* yf = reinterpret_cast<float*>(y);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (cur.o0 >= 0) st_nt(yf + cur.o0 + j * P::kTPF, v[j].re);
                if (cur.o1 >= 0) st_nt(yf + cur.o1 + j * P::kTPF, v[j].im);
            }
        } else {
            region_sync<P::kWaveLocal>();
#pragma unroll
            for (int j = 0; j < 16; ++j) slot[lds_pad(t + j * P::kTPF)] = v[j];
            region_sync<P::kWaveLocal>();
#pragma unroll
            for (int i = 0; i < kSteps; ++i) {
                const int e = 1024 * wave + kVec * lane + 64 * kVec * i;
                float a[kVec], b[kVec];
#pragma unroll
                for (int c = 0; c < kVec; ++c) {
                    const cpx z = lds[lds_pad(e + c)];
                    a[c] = z.re, b[c] = z.im;
                }
                const long long a0 = piece(cur.o0, i), a1 = piece(cur.o1, i);
                if (a0 >= 0) st_nt(reinterpret_cast<u32x4*>(y + a0), R::encode(a));
                if (a1 >= 0) st_nt(reinterpret_cast<u32x4*>(y + a1), R::encode(b));
            }
        }
    }
}

}  // namespace thff

namespace thff {

// ---------------------------------------------------------------------------
// Tiled valid 1-D correlation with 64-point FFTs (overlap-save), the
// reference's conv1d_direct_fft_kernel (sample/conv1d/main.cu:38-128):
//   y[b][i] = sum_{k < F} x[b][i + k] * f[k],   i < L - F + 1,  1 <= F <= 64,
// complex x, f, no conjugation.  Window w of a signal is x[w*V .. w*V + 63]
// with V = 65 - F; its circular convolution with g[m] = f[(64 - m) mod 64] / 64
// (the reversed filter, main.cu:145-154) equals y[w*V + j] for j < V, since
// those outputs never wrap.  Each wave owns 16 consecutive windows: it stages
// their input span (15 V + 64 <= 1024 values) in its own LDS region, gathers
// every window into its transform slot's registers, runs FFT * G * IFFT and
// writes the V valid outputs of each window back contiguously.  Nothing
// crosses waves, so the kernel has no workgroup barrier after its set-up:
// every workgroup transforms the filter once (fp32 taps) into a 64-value LDS
// table G, then walks groups of 64 windows (one per transform slot) with
// tile_walk: groups_per_block consecutive groups, or 0 for grid-stride over a
// device-sized grid.
// Inputs past the end of a signal read as zero; no valid output uses them.
// Spans and output runs start at multiples of 16 values of their signal, so
// signals that start on a 16-byte boundary move as whole 16-byte vectors
// (one partial vector at a signal's end); others value by value.
// float2: the next group's span is loaded into registers while the current
// one is transformed (when every signal starts on a 16-byte boundary), at 2
// waves per SIMD: 2^26 values, 9 taps, 232 us against 261 us without.  The
// library runs half2 on conv1d_valid_mfma_kernel (fft_conv_mfma.hpp:
// 256-point windows on MFMA, 112 us against 162 us for this kernel in half2,
// which keeps 3 waves per SIMD and no prefetch).
// ---------------------------------------------------------------------------
template <class IO>
inline constexpr bool kValidPrefetch = std::is_same_v<IO, float2>;
template <class IO>
inline constexpr int kValidMinWavesPerEU = kValidPrefetch<IO> ? 2 : 3;

// kExact: the 64-point passes use exact per-lane twiddles (LaneTwiddles64Exact,
// 610 instead of 666 VALU instructions per window group, 243 VGPRs): float2
// only, which already runs at 2 waves per SIMD; 227 vs 233 us at 2^26 values.
template <class IO, bool kExact = kValidPrefetch<IO>>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kValidMinWavesPerEU<IO>))) void conv1d_valid_kernel(
    const IO* __restrict__ x, const float2* __restrict__ taps, IO* __restrict__ y,
    long long len, int ntaps, int batch, const float2* __restrict__ tw, int groups_per_block) {
    using P = C2CPlan<64>;
    using I = Io<IO>;
    using W1 = typename I::W1;
    using W4 = typename I::W4;
    constexpr int kVec = I::kVec;      // complex values per 16-byte vector
    constexpr int kWindowsPerWave = 16;
    constexpr int kSpan = 1024;        // values staged per wave, >= 15 V + 64 and >= 16 V
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int t = tid & 3;             // lane within its window's transform
    const int fl = (tid >> 2) & 15;    // window within the wave
    __shared__ __align__(16) cpx lds[P::kLdsSlots];
    __shared__ cpx spectrum[64];  // G, natural order
    cpx* const region = lds + wave * kWindowsPerWave * P::kSlot;  // 16 slots = 1088 >= kSpan
    cpx* const slot = region + fl * P::kSlot;

    std::conditional_t<kExact, LaneTwiddles64Exact, LaneTwiddles<64>> w;
    w.load(t, tw);

    const int V = 65 - ntaps;                            // valid outputs per window
    const unsigned rcpV = (65536u + V - 1) / V;          // e / V == (e * rcpV) >> 16 for e < 1024
    const long long out_len = len - ntaps + 1;
    const long long windows = (out_len + V - 1) / V;     // per signal
    const long long groups_per_signal = (windows + P::kFPB - 1) / P::kFPB;
    const long long groups = groups_per_signal * batch;
    const bool x16 = (reinterpret_cast<unsigned long long>(x) & 15) == 0;
    const bool y16 = (reinterpret_cast<unsigned long long>(y) & 15) == 0;

    // G = FFT(g), g[m] = f[(64 - m) mod 64] / 64, m = t + 4 j, computed by
    // every slot and published once by the first slot.
    {
        cpx G[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int m = t + 4 * j;
            const int k = m == 0 ? 0 : 64 - m;
            const float2 c = k < ntaps ? taps[k] : make_float2(0.f, 0.f);
            G[j] = {c.x * (1.0f / 64), c.y * (1.0f / 64)};
        }
        fft_registers<64, true>(G, slot, t, w);
        if (tid < 4)
#pragma unroll
            for (int j = 0; j < 16; ++j) spectrum[t + 4 * j] = G[j];
        __syncthreads();
    }

    long long g, g_end, step;
    tile_walk(groups, groups_per_block, g, g_end, step);
    // A wave's 16 windows read 15 V + 64 values of its span; nothing past
    // that is loaded (it is the next wave's, which may run on another XCD).
    const int need = 15 * V + 64;
    // The span of group gg (this wave's windows) as 16-byte vectors, zero past
    // the signal's end; for signals that start on a 16-byte boundary.
    constexpr int kLoads = kSpan / (64 * kVec);
    // Signal and group within it of the walk's groups, advanced per step.
    const DivWalk walk(step, groups_per_signal);
    DivPos pos = walk.at(g);
    auto span_load = [&](DivPos gp, W4 (&r)[kLoads]) {
        const long long bb = gp.q;
        const long long s0 = (gp.r * P::kFPB + wave * kWindowsPerWave) * V;
        const long long av = len - s0 < need ? len - s0 : need;
        const IO* sp = x + bb * len + s0;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int e = kVec * (lane + 64 * i);
            if (s0 < out_len && e + kVec <= av) {
                r[i] = ld_nt(reinterpret_cast<const W4*>(sp + e));
            } else {
                W4 z{};
                if (s0 < out_len)
#pragma unroll
                    for (int c = 0; c < kVec; ++c)
                        if (e + c < av)
                            reinterpret_cast<W1*>(&z)[c] = *reinterpret_cast<const W1*>(sp + e + c);
                r[i] = z;
            }
        }
    };
    // Prefetch only when every signal starts on a 16-byte boundary.
    const bool prefetch = kValidPrefetch<IO> && x16 && len % kVec == 0;
    W4 next[kLoads];
    if (prefetch && g < g_end) span_load(pos, next);
    // A wave's issue priority falls as its workgroup gets ahead of the others
    // (ProgressPriority): 223.5 against 227.3-227.5 us for 2^26 values (the
    // fp16 MFMA valid kernel measured 1.5% slower with it and does not use it).
    long long left = (g_end - g + step - 1) / step;
    const ProgressPriority priority(left);
    for (; g < g_end; g += step, --left) {
        priority.set(left);
        const long long b = pos.q;
        // This wave's first window, and where its input span and its outputs
        // start in signal b (both w0 * V, a multiple of 16 values).
        const long long w0 = pos.r * P::kFPB + wave * kWindowsPerWave;
        const long long span0 = w0 * V;
        pos = walk.advance(pos);
        W4 cur[kLoads];
        if (prefetch) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) cur[i] = next[i];
            if (g + step < g_end) span_load(pos, next);
        }
        if (span0 >= out_len) continue;  // no window of this wave has an output
        const long long avail = len - span0 < need ? len - span0 : need;  // > 0
        const IO* src = x + b * len + span0;
        // Whole 16-byte vectors when the signal starts on one (always for b = 0).
        const bool in_vec = x16 && (b * len) % kVec == 0;
        const bool out_vec = y16 && (b * out_len) % kVec == 0;

        wave_lds_sync();  // the previous group's reads of the region are done
        if (prefetch) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                const int e = kVec * (lane + 64 * i);
                cpx q[kVec];
                I::decode4(cur[i], q);
#pragma unroll
                for (int c = 0; c < kVec; ++c) region[e + c] = q[c];
            }
        } else if (in_vec) {
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                const int e = kVec * (lane + 64 * i);
                cpx q[kVec];
                if (e + kVec <= avail) {
                    I::decode4(*reinterpret_cast<const W4*>(src + e), q);
                } else {
#pragma unroll
                    for (int c = 0; c < kVec; ++c)
                        q[c] = e + c < avail ? I::decode1(*reinterpret_cast<const W1*>(src + e + c))
                                             : cpx{0.f, 0.f};
                }
#pragma unroll
                for (int c = 0; c < kVec; ++c) region[e + c] = q[c];
            }
        } else {
#pragma unroll
            for (int i = 0; i < kSpan / 64; ++i) {
                const int e = lane + 64 * i;
                region[e] = e < avail ? I::decode1(*reinterpret_cast<const W1*>(src + e))
                                      : cpx{0.f, 0.f};
            }
        }
        wave_lds_sync();
        cpx v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = region[fl * V + t + 4 * j];
        wave_lds_sync();  // the gather is done before the transform reuses the region

        fft_registers<64, true>(v, slot, t, w);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = cmul(v[j], spectrum[t + 4 * j]);
        fft_registers<64, false>(v, slot, t, w);

        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < 16; ++j) slot[lds_pad(t + 4 * j)] = v[j];
        wave_lds_sync();
        // Output e of the wave (e < 16 V) is element e mod V of window e / V.
        const long long left = out_len - span0;
        const int count = left < kWindowsPerWave * V ? static_cast<int>(left) : kWindowsPerWave * V;
        IO* dst = y + b * out_len + span0;
        auto value = [&](int e) {
            const int q = static_cast<int>((static_cast<unsigned>(e) * rcpV) >> 16);
            return region[q * P::kSlot + lds_pad(e - q * V)];
        };
        if (out_vec) {
#pragma unroll 1
            for (int i = 0; i < kSpan / (64 * kVec); ++i) {
                const int e = kVec * (lane + 64 * i);
                if (e + kVec <= count) {
                    cpx q[kVec];
#pragma unroll
                    for (int c = 0; c < kVec; ++c) q[c] = value(e + c);
                    st_nt(reinterpret_cast<W4*>(dst + e), I::encode4(q));
                } else {
#pragma unroll
                    for (int c = 0; c < kVec; ++c)
                        if (e + c < count)
                            *reinterpret_cast<W1*>(dst + e + c) = I::encode1(value(e + c));
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kSpan / 64; ++i) {
                const int e = lane + 64 * i;
                if (e < count) *reinterpret_cast<W1*>(dst + e) = I::encode1(value(e));
            }
        }
    }
}

}  // namespace thff
