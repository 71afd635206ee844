// thunderfft_device.hpp -- the reference's device-side fusion API on gfx950.
//
// Mirrors the device half of mcrl/thunderfft's include/thunderfft/thunderfft.cuh
// (layout_t :35-44, the movement helpers :81-126, ThunderFFT_kernel_reg
// :200-202, batch_per_block / warp_per_block / threads_per_warp / pad_h) so a
// caller can run batched FFTs inside its own kernel and keep them fused with
// other work.  These are the same building blocks the library's own kernels
// use (thunderfft/detail/fft_tile.hpp).
//
// Contract (wave64 / gfx950 values; the reference's warp-32 figures differ):
//  * A block is 256 lanes (any dim3 whose product is 256, e.g. 256 or
//    (64, 4)), and processes batch_per_block<N> = 4096 / N transforms of
//    length N.  Every lane holds 16 complex values ("the fragment").
//  * Fragment order: lane tid belongs to transform f = tid / (N/16) and
//    holds elements t + (N/16)*j, j = 0..15, of it, t = tid % (N/16).  The
//    same order holds before and after ThunderFFT_kernel_reg, in both
//    directions, so a forward transform, a pointwise product and an inverse
//    transform chain in registers with no reordering (the reference needs a
//    size-specific reorder between them).
//  * The workspace is caller-owned LDS of workspace_bytes<N, batch> bytes
//    (8 bytes per complex value for both storage types: the FFT computes in
//    fp32), 8-byte aligned.  All helpers are collective over the block, do
//    no bounds checks and insert no barrier before their first access:
//    __syncthreads() between a producer and a consumer of the same LDS, as
//    in the reference.
//  * Twiddles: ThunderFFTInitialize<T>(N) builds the device table; pass its
//    pointer (ThunderFFT_twiddle_table<T>() on the host) to
//    ThunderFFT_load_twiddles once per kernel, or straight to
//    ThunderFFT_kernel_reg, which then loads the lane's factors itself.
//  * layout_t::Reversed must be false: fragments here are natural-order.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "thunderfft/detail/fft_tile.hpp"
#include "thunderfft/thunderfft.hpp"

namespace thunderfft {

// Wave64s per block (the reference's warp_per_block<N>, thunderfft_impl.cuh:24-32).
template <int N>
inline constexpr int warp_per_block = 4;

// Padding per transform in the workspace (the reference's pad_h, util_arith.h:123-136).
__host__ __device__ constexpr int pad_h(int N) { return N / 16; }

// Complex values per lane in a fragment.
inline constexpr int elements_per_thread = 16;

// LDS bytes ThunderFFT_kernel_reg<T, N, batch, fwd> needs as workspace.
template <int N, int batch>
inline constexpr int workspace_bytes = 8 * (N + N / 16) * batch;

// Block-local shared-memory layout (reference thunderfft.cuh:35-44): logical
// element i of transform j is at idx = i*ElemStride + j*BatchStride, stored
// at idx + (idx / PadPeriod) * Pad.
template <int N_, int Batch_, int ElemStride_, int BatchStride_, int PadPeriod_, int Pad_,
          bool Reversed_>
struct layout_t {
    static constexpr int N = N_;
    static constexpr int batch = Batch_;
    static constexpr int elem_stride = ElemStride_;
    static constexpr int batch_stride = BatchStride_;
    static constexpr int pad_period = PadPeriod_;
    static constexpr int pad = Pad_;
    static constexpr int reversed = Reversed_;
    static_assert(PadPeriod_ > 0, "layout_t: PadPeriod must be positive");
    static_assert(!Reversed_, "layout_t: fragments are natural-order; Reversed is not used");
    __host__ __device__ static constexpr int at(int i, int j) {
        const int idx = i * ElemStride_ + j * BatchStride_;
        return idx + (idx / PadPeriod_) * Pad_;
    }
};

// Per-lane twiddle factors of length N (a few registers; see fft_tile.hpp).
template <int N>
using lane_twiddles = thff::LaneTwiddles<N>;

namespace detail {

__device__ __forceinline__ int block_tid() {
    return threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z);
}

template <class T>
__device__ __forceinline__ thff::cpx to_cpx(vec2_t<T> v) {
    if constexpr (std::is_same_v<T, float>) {
        return {v.x, v.y};
    } else {
        const float2 f = __half22float2(v);
        return {f.x, f.y};
    }
}

template <class T>
__device__ __forceinline__ vec2_t<T> from_cpx(thff::cpx v) {
    if constexpr (std::is_same_v<T, float>)
        return make_float2(v.re, v.im);
    else
        return __floats2half2_rn(v.re, v.im);
}

template <int N, int batch>
__device__ __forceinline__ void check_shape() {
    static_assert(is_supported_length<N>, "Unsupported ThunderFFT length");
    static_assert(batch == batch_per_block<N>,
                  "batch must be batch_per_block<N> (4096 / N transforms per 256-lane block)");
}

}  // namespace detail

// Load this lane's twiddle factors for length N from the device table of
// ThunderFFTInitialize<T>(N) (N fp32 values (cos, sin)(2*pi*m/N)).
template <int N>
__device__ __forceinline__ void ThunderFFT_load_twiddles(lane_twiddles<N>& w,
                                                         const float2* __restrict__ table) {
    w.load(detail::block_tid() % (N / 16), table);
}

// Batched FFT of the block's fragment in place (reference thunderfft.cuh:200-202).
// Collective over the 256-lane block; workspace = workspace_bytes<N, batch>
// bytes of LDS that no other lane is still reading.  Unnormalized; forward
// uses exp(-2*pi*i*n*k/N).
template <typename T, int N, int batch, bool forward>
__device__ __forceinline__ void ThunderFFT_kernel_reg(vec2_t<T>* __restrict__ reg,
                                                      const lane_twiddles<N>& W, void* workspace) {
    detail::check_shape<N, batch>();
    using P = thff::C2CPlan<N>;
    const int tid = detail::block_tid();
    thff::cpx* slot = static_cast<thff::cpx*>(workspace) + (tid / P::kTPF) * P::kSlot;
    thff::cpx v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = detail::to_cpx<T>(reg[j]);
    thff::fft_registers<N, forward>(v, slot, tid % P::kTPF, W);
#pragma unroll
    for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(v[j]);
}

// As above, loading the lane's twiddles from the device table W first.
template <typename T, int N, int batch, bool forward>
__device__ __forceinline__ void ThunderFFT_kernel_reg(vec2_t<T>* __restrict__ reg,
                                                      const float2* __restrict__ W,
                                                      void* workspace) {
    lane_twiddles<N> w;
    ThunderFFT_load_twiddles<N>(w, W);
    ThunderFFT_kernel_reg<T, N, batch, forward>(reg, w, workspace);
}

// Global memory -> fragment (reference thunderfft.cuh:81-85).  gmem is the
// block-local base of `batch` contiguous natural-order signals of N values.
template <typename T, int N, int batch>
__device__ __forceinline__ void ThunderFFT_gmem2reg(vec2_t<T>* __restrict__ reg,
                                                    const vec2_t<T>* __restrict__ gmem) {
    detail::check_shape<N, batch>();
    constexpr int TPF = N / 16;
    const int tid = detail::block_tid();
    const vec2_t<T>* src = gmem + (tid / TPF) * N + tid % TPF;
#pragma unroll
    for (int j = 0; j < 16; ++j) reg[j] = src[j * TPF];
}

// Fragment -> global memory, natural order (reference thunderfft.cuh:88-92).
template <typename T, int N, int batch>
__device__ __forceinline__ void ThunderFFT_reg2gmem(vec2_t<T>* __restrict__ gmem,
                                                    const vec2_t<T>* __restrict__ reg) {
    detail::check_shape<N, batch>();
    constexpr int TPF = N / 16;
    const int tid = detail::block_tid();
    vec2_t<T>* dst = gmem + (tid / TPF) * N + tid % TPF;
#pragma unroll
    for (int j = 0; j < 16; ++j) dst[j * TPF] = reg[j];
}

// Shared memory described by sL -> fragment (reference thunderfft.cuh:97-101).
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_smem2reg(vec2_t<T>* __restrict__ reg,
                                                    const vec2_t<T>* __restrict__ smem) {
    detail::check_shape<sL::N, sL::batch>();
    constexpr int TPF = sL::N / 16;
    const int tid = detail::block_tid();
    const int f = tid / TPF, t = tid % TPF;
#pragma unroll
    for (int j = 0; j < 16; ++j) reg[j] = smem[sL::at(t + j * TPF, f)];
}

// Fragment -> shared memory described by sL (reference thunderfft.cuh:106-110).
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_reg2smem(vec2_t<T>* __restrict__ smem,
                                                    const vec2_t<T>* __restrict__ reg) {
    detail::check_shape<sL::N, sL::batch>();
    constexpr int TPF = sL::N / 16;
    const int tid = detail::block_tid();
    const int f = tid / TPF, t = tid % TPF;
#pragma unroll
    for (int j = 0; j < 16; ++j) smem[sL::at(t + j * TPF, f)] = reg[j];
}

// Contiguous global tile -> shared memory described by sL (reference
// thunderfft.cuh:114-118); consecutive lanes read consecutive elements.
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_gmem2smem(vec2_t<T>* __restrict__ smem,
                                                     const vec2_t<T>* __restrict__ gmem) {
    const int tid = detail::block_tid();
#pragma unroll 4
    for (int e = tid; e < sL::N * sL::batch; e += 256) smem[sL::at(e % sL::N, e / sL::N)] = gmem[e];
}

// Shared memory described by sL -> contiguous global tile (reference
// thunderfft.cuh:122-126).
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_smem2gmem(vec2_t<T>* __restrict__ gmem,
                                                     const vec2_t<T>* __restrict__ smem) {
    const int tid = detail::block_tid();
#pragma unroll 4
    for (int e = tid; e < sL::N * sL::batch; e += 256) gmem[e] = smem[sL::at(e % sL::N, e / sL::N)];
}

}  // namespace thunderfft
