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
//  * Fragment order: register j of lane tid holds element
//    fragment_element<T, N>(tid, j) of transform fragment_transform<T, N>(tid, j)
//    of the block.  For float, and for half at N = 64, 128 (VALU
//    transforms): transform tid / (N/16), element t + (N/16)*j,
//    t = tid % (N/16).  For half at N = 256 ... 4096 the transform
//    runs on the matrix cores (v_mfma_f32_16x16x32_f16, as the library's own
//    kernels) and the fragment is the MFMA layout: wave w = tid/64, lane
//    n + 16q, j = 4b + r; N = 256C (C = 1, 2, 4): transform w*(4/C) + b/C,
//    element n + 16*(b%C) + 16C*(q+4r); N = 2048: transform w/2, element
//    4*(w%2) + b + 8n + 128*(q+4r); N = 4096: element
//    4w + b + 16n + 256*(q+4r).  Either way the same order holds before and after
//    ThunderFFT_kernel_reg, in both directions, so a forward transform, a
//    pointwise product and an inverse transform chain in registers with no
//    reordering (the reference needs a size-specific reorder between them);
//    the movement helpers below follow the order.
//  * The workspace is caller-owned LDS of workspace_bytes<N, batch> bytes
//    (8 bytes per complex value for both storage types: the FFT computes in
//    fp32), 16-byte aligned (the MFMA transforms move 16-byte chunks through
//    it; __shared__ __align__(16)).  All helpers are collective over the block, do
//    no bounds checks and insert no barrier before their first access:
//    __syncthreads() between a producer and a consumer of the same LDS, as
//    in the reference.
//  * Twiddles: ThunderFFTInitialize<T>(N) builds the device table; pass its
//    pointer (ThunderFFT_twiddle_table<T>() on the host) to
//    ThunderFFT_load_twiddles once per kernel, or straight to
//    ThunderFFT_kernel_reg, which then loads the lane's factors itself.  For
//    half, as in the reference's fused samples, a kernel can instead build
//    its coefficients once with unit_fp16::make_reg_b_precompute<N, fwd>(W)
//    (vec2_t<half> W[36], or W[28] for N <= 128, the reference's sizes;
//    unit_fp16::coefficient_count<N> is never more; no table needed) and
//    pass W to ThunderFFT_kernel_reg: the MFMA transforms then build no
//    operand and read no twiddle table per call.
//  * layout_t::Reversed on an input layout selects the permutation the
//    transforms expect, which here is the identity (natural order).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "thunderfft/detail/fft_mfma.hpp"
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
// at idx + (idx / PadPeriod) * Pad.  Reversed requests "the input
// permutation each size-specific transform expects" (the reference's
// documented meaning, thunderfft.cuh:29-32; its transforms take base-4
// digit-reversed input for N outside {512, 2048, 4096}).  Every transform
// here takes natural order, so that permutation is the identity: a fused
// kernel written for the reference with a reversed input layout runs
// unchanged.  As in the reference (thunderfft_impl_helper.cuh:51-56), an
// output layout must not be reversed: ThunderFFT_smem2gmem rejects it at
// compile time.
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
    __host__ __device__ static constexpr int at(int i, int j) {
        const int idx = i * ElemStride_ + j * BatchStride_;
        return idx + (idx / PadPeriod_) * Pad_;
    }
};

// A bank-conflict-free shared-memory layout of the block's batch_per_block<N>
// transforms for the fragment order of (T, N): ThunderFFT_smem2reg /
// reg2smem through it read and write every LDS bank once per instruction.
// VALU order: one pad value per 16 (as pad_h); MFMA order (C = N/256): 16 pad
// values after every 16C, so the four lane groups q (16C apart) land on
// different banks; N = 2048 and 4096: one pad value per 64.
template <typename T, int N>
using fragment_layout = std::conditional_t<
    std::is_same_v<T, half> && (N == 2048 || N == 4096),
    layout_t<N, batch_per_block<N>, 1, N, 64, 1, false>,
    std::conditional_t<
    std::is_same_v<T, half> && (N == 512 || N == 1024),
    layout_t<N, batch_per_block<N>, 1, N, 16 * (N / 256), 16, false>,
    std::conditional_t<std::is_same_v<T, half> && N == 256,
                       layout_t<N, batch_per_block<N>, 1, N, 16, 0, false>,
                       layout_t<N, batch_per_block<N>, 1, N, 16, 1, false>>>>;

// Per-lane twiddle factors of length N (a few registers; see fft_tile.hpp),
// and the table they came from.
template <int N>
using lane_twiddles = thff::LaneTwiddles<N>;

// True where half fragments use the MFMA layout (see the contract above).
template <typename T, int N>
inline constexpr bool fragment_on_mfma =
    std::is_same_v<T, half> && (N == 256 || N == 512 || N == 1024 || N == 2048 || N == 4096);

// Transform (of the block's batch_per_block<N>) and element index held by
// register j of lane tid.
template <typename T, int N>
__device__ __forceinline__ int fragment_transform(int tid, int j) {
    if constexpr (fragment_on_mfma<T, N> && N == 4096) {
        return 0;
    } else if constexpr (fragment_on_mfma<T, N> && N == 2048) {
        return tid >> 7;
    } else if constexpr (fragment_on_mfma<T, N>) {
        constexpr int C = N / 256;
        return (tid >> 6) * (4 / C) + (j >> 2) / C;
    } else {
        return tid / (N / 16);
    }
}
template <typename T, int N>
__device__ __forceinline__ int fragment_element(int tid, int j) {
    if constexpr (fragment_on_mfma<T, N> && N == 4096) {
        const int lane = tid & 63;
        return 4 * (tid >> 6) + (j >> 2) + 16 * (lane & 15) + 256 * ((lane >> 4) + 4 * (j & 3));
    } else if constexpr (fragment_on_mfma<T, N> && N == 2048) {
        const int lane = tid & 63;
        return 4 * ((tid >> 6) & 1) + (j >> 2) + 8 * (lane & 15) + 128 * ((lane >> 4) + 4 * (j & 3));
    } else if constexpr (fragment_on_mfma<T, N>) {
        constexpr int C = N / 256;
        const int lane = tid & 63;
        return (lane & 15) + 16 * ((j >> 2) % C) + 16 * C * ((lane >> 4) + 4 * (j & 3));
    } else {
        return tid % (N / 16) + (N / 16) * j;
    }
}

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
    const int tid = detail::block_tid();
    if constexpr (fragment_on_mfma<T, N> && N == 4096) {
        // The library's three-stage MFMA transform (thff::mfma4096_fft_regs);
        // 17 KiB of the workspace; two workgroup barriers.
        thff::cpx y[4][4];
#pragma unroll
        for (int j = 0; j < 16; ++j) y[j >> 2][j & 3] = detail::to_cpx<T>(reg[j]);
        thff::mfma4096_fft_regs<forward>(static_cast<unsigned*>(workspace), W.table, tid, y);
#pragma unroll
        for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(y[j >> 2][j & 3]);
    } else if constexpr (fragment_on_mfma<T, N> && N == 2048) {
        // The three-stage MFMA transform of the library's N = 2048 kernel
        // (thff::mfma2048_fft_regs), both transforms of the block at once;
        // 16.5 KiB of the workspace; two workgroup barriers.
        thff::cpx y[4][4];
#pragma unroll
        for (int j = 0; j < 16; ++j) y[j >> 2][j & 3] = detail::to_cpx<T>(reg[j]);
        thff::mfma2048_fft_regs<forward>(static_cast<unsigned*>(workspace), W.table, tid, y);
#pragma unroll
        for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(y[j >> 2][j & 3]);
    } else if constexpr (fragment_on_mfma<T, N>) {
        // The library's MFMA transform (thff::mfma_fft_regs): f16 data into
        // each DFT16 stage, fp32 accumulation and twiddles; wave w uses 4 KiB
        // of the workspace at w * 4 KiB.
        constexpr int C = N / 256;
        thff::cpx y[4][4];
#pragma unroll
        for (int j = 0; j < 16; ++j) y[j >> 2][j & 3] = detail::to_cpx<T>(reg[j]);
        unsigned* region = static_cast<unsigned*>(workspace) + (tid >> 6) * 1024;
        thff::mfma_fft_regs<C, forward>(region, W.table, tid & 63, y);
#pragma unroll
        for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(y[j >> 2][j & 3]);
    } else {
        using P = thff::C2CPlan<N>;
        thff::cpx* slot = static_cast<thff::cpx*>(workspace) + (tid / P::kTPF) * P::kSlot;
        thff::cpx v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = detail::to_cpx<T>(reg[j]);
        thff::fft_registers<N, forward>(v, slot, tid % P::kTPF, W);
#pragma unroll
        for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(v[j]);
    }
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

namespace detail {

// The per-lane coefficients of the fp16 transform of length N in fp32 form:
// the MFMA transforms' operands and twiddles (N = 256 ... 4096) or the VALU
// passes' twiddle factors (N = 64, 128).
template <int N>
using half_coefficients = std::conditional_t<
    N == 4096, thff::Mfma4096Coeffs,
    std::conditional_t<N == 2048, thff::Mfma2048Coeffs,
    std::conditional_t<fragment_on_mfma<half, N>, thff::MfmaCoeffs<(N >= 256 ? N / 256 : 1)>,
                       thff::LaneTwiddles<N>>>>;

// The reference's slot budget for those coefficients: make_reg_b_precompute
// fills 28 half2 for N = 64, 128 and 36 for N = 256 ... 4096
// (unit_kernel_fp16.cuh:97-108), and its fused kernels declare arrays of
// exactly that size (sample/conv1d/main.cu:61, conv1d_fullfft_l4096_thunder.cu
// :298, sample/conv2d/thunder.cu:84,125).
template <int N>
inline constexpr int reference_coefficient_slots = N <= 128 ? 28 : 36;

// An MFMA transform's coefficients with every twiddle held as one f16 pair
// (real low, imaginary high), rounded once, and the DFT16 operands (f16
// already) as they are: at N = 1024 (19 twiddles) and 2048, 4096 (20) the
// fp32 form needs 56 slots, this one 36.  The f16 twiddle adds an error of
// the size of the f16 rounding the data already takes before every DFT16.
template <class Full>
struct PackedMfmaCoefficients {
    thff::f16x8 ops[4];
    unsigned tw[Full::kTwiddles];
    __device__ __forceinline__ void pack(Full& k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ops[i] = k.op(i);
#pragma unroll
        for (int i = 0; i < Full::kTwiddles; ++i) tw[i] = thff::pack_half2(k.twiddle(i));
    }
    __device__ __forceinline__ void unpack(Full& k) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) k.op(i) = ops[i];
#pragma unroll
        for (int i = 0; i < Full::kTwiddles; ++i) k.twiddle(i) = thff::unpack_half2(tw[i]);
    }
};

// What make_reg_b_precompute<N, fwd> stores in W: the fp32 form where it fits
// the reference's budget (N = 64 ... 512), else the packed one.
template <int N>
using half_coefficient_slots = std::conditional_t<
    sizeof(half_coefficients<N>) <= sizeof(unsigned) * reference_coefficient_slots<N>,
    half_coefficients<N>, PackedMfmaCoefficients<half_coefficients<N>>>;

template <int N>
inline constexpr bool half_coefficients_packed =
    !std::is_same_v<half_coefficient_slots<N>, half_coefficients<N>>;

}  // namespace detail

namespace unit_fp16 {

// half2 slots of per-lane coefficients that make_reg_b_precompute<N, fwd>
// writes and ThunderFFT_kernel_reg<half, N, batch, fwd>(reg, W, workspace)
// reads (a slot holds 32 bits: f16 operand pairs, an f16 twiddle pair or one
// fp32 twiddle component).  Never more than the reference's 28 (N <= 128) or
// 36 (N >= 256) half2 (unit_kernel_fp16.cuh:97-108): a kernel written for the
// reference keeps its W_fwd[36] / W_inv[36] arrays.
template <int N>
inline constexpr int coefficient_count =
    static_cast<int>(sizeof(detail::half_coefficient_slots<N>) / sizeof(unsigned));

// This lane's coefficients of the fp16 transform of length N in direction
// `forward` (the reference's unit_fp16::make_reg_b_precompute<N, fwd>,
// unit_kernel_fp16.cuh:97-108, and sample/README.md:406-409): the DFT16
// operands and every twiddle the transform needs, computed with the hardware
// transcendentals (no table, no memory access; their error is far below the
// f16 rounding of the data), once per kernel.  Call with the same block
// shape and lane numbering as ThunderFFT_kernel_reg.  W is a vec2_t<half>
// array or pointer to at least coefficient_count<N> slots, which is at most
// the reference's 28 / 36; an array is checked at compile time.
template <int N, bool forward, class Coeffs>
__device__ __forceinline__ void make_reg_b_precompute(Coeffs&& W_arg) {
    static_assert(coefficient_count<N> <= detail::reference_coefficient_slots<N>,
                  "the coefficients must fit the reference's W arrays");
    using A = std::remove_reference_t<Coeffs>;
    if constexpr (std::is_array_v<A>)
        static_assert(std::extent_v<A> >= static_cast<size_t>(coefficient_count<N>),
                      "make_reg_b_precompute: declare vec2_t<half> "
                      "W[thunderfft::unit_fp16::coefficient_count<N>] (28 for N <= 128, "
                      "36 otherwise, as in the reference)");
    vec2_t<half>* const W = W_arg;
    detail::check_shape<N, batch_per_block<N>>();
    const int tid = detail::block_tid();
    detail::half_coefficients<N> k;
    if constexpr (N == 2048 || N == 4096)
        k.template build<forward>(tid);
    else if constexpr (fragment_on_mfma<half, N>)
        k.template build<forward>(tid & 63);
    else
        k.build(tid % (N / 16));
    if constexpr (detail::half_coefficients_packed<N>) {
        detail::half_coefficient_slots<N> packed;
        packed.pack(k);
        __builtin_memcpy(static_cast<void*>(W), &packed, sizeof(packed));
    } else {
        __builtin_memcpy(static_cast<void*>(W), &k, sizeof(k));
    }
}

}  // namespace unit_fp16

// ThunderFFT_kernel_reg with the reference's argument types
// (thunderfft.cuh:200-202): for half, W holds this lane's coefficients from
// unit_fp16::make_reg_b_precompute<N, forward> (unit_fp16::coefficient_count<N>
// slots), so no table is read and no operand is built per call; for float, W
// is the ThunderFFTInitialize<float>(N) table, as in the overload above.
template <typename T, int N, int batch, bool forward>
__device__ __forceinline__ void ThunderFFT_kernel_reg(vec2_t<T>* __restrict__ reg,
                                                      vec2_t<T>* __restrict__ W, void* workspace) {
    if constexpr (std::is_same_v<T, float>) {
        ThunderFFT_kernel_reg<T, N, batch, forward>(reg, static_cast<const float2*>(W), workspace);
    } else {
        detail::check_shape<N, batch>();
        const int tid = detail::block_tid();
        detail::half_coefficients<N> k;
        if constexpr (detail::half_coefficients_packed<N>) {
            detail::half_coefficient_slots<N> packed;
            __builtin_memcpy(&packed, static_cast<const void*>(W), sizeof(packed));
            packed.unpack(k);
        } else {
            __builtin_memcpy(&k, static_cast<const void*>(W), sizeof(k));
        }
        if constexpr (N == 4096) {
            thff::cpx y[4][4];
#pragma unroll
            for (int j = 0; j < 16; ++j) y[j >> 2][j & 3] = detail::to_cpx<T>(reg[j]);
            thff::mfma4096_fft_regs<forward>(static_cast<unsigned*>(workspace), k, tid, y);
#pragma unroll
            for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(y[j >> 2][j & 3]);
        } else if constexpr (N == 2048) {
            thff::cpx y[4][4];
#pragma unroll
            for (int j = 0; j < 16; ++j) y[j >> 2][j & 3] = detail::to_cpx<T>(reg[j]);
            thff::mfma2048_fft_regs<forward>(static_cast<unsigned*>(workspace), k, tid, y);
#pragma unroll
            for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(y[j >> 2][j & 3]);
        } else if constexpr (fragment_on_mfma<T, N>) {
            constexpr int C = N / 256;
            thff::cpx y[4][4];
#pragma unroll
            for (int j = 0; j < 16; ++j) y[j >> 2][j & 3] = detail::to_cpx<T>(reg[j]);
            unsigned* region = static_cast<unsigned*>(workspace) + (tid >> 6) * 1024;
            thff::mfma_fft_regs<C, forward>(region, k, tid & 63, y);
#pragma unroll
            for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(y[j >> 2][j & 3]);
        } else {
            using P = thff::C2CPlan<N>;
            thff::cpx* slot = static_cast<thff::cpx*>(workspace) + (tid / P::kTPF) * P::kSlot;
            thff::cpx v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = detail::to_cpx<T>(reg[j]);
            thff::fft_registers<N, forward>(v, slot, tid % P::kTPF, k);
#pragma unroll
            for (int j = 0; j < 16; ++j) reg[j] = detail::from_cpx<T>(v[j]);
        }
    }
}

// Global memory -> fragment (reference thunderfft.cuh:81-85).  gmem is the
// block-local base of `batch` contiguous natural-order signals of N values.
template <typename T, int N, int batch>
__device__ __forceinline__ void ThunderFFT_gmem2reg(vec2_t<T>* __restrict__ reg,
                                                    const vec2_t<T>* __restrict__ gmem) {
    detail::check_shape<N, batch>();
    const int tid = detail::block_tid();
#pragma unroll
    for (int j = 0; j < 16; ++j)
        reg[j] = gmem[fragment_transform<T, N>(tid, j) * N + fragment_element<T, N>(tid, j)];
}

// Fragment -> global memory, natural order (reference thunderfft.cuh:88-92).
template <typename T, int N, int batch>
__device__ __forceinline__ void ThunderFFT_reg2gmem(vec2_t<T>* __restrict__ gmem,
                                                    const vec2_t<T>* __restrict__ reg) {
    detail::check_shape<N, batch>();
    const int tid = detail::block_tid();
#pragma unroll
    for (int j = 0; j < 16; ++j)
        gmem[fragment_transform<T, N>(tid, j) * N + fragment_element<T, N>(tid, j)] = reg[j];
}

// Shared memory described by sL -> fragment (reference thunderfft.cuh:97-101).
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_smem2reg(vec2_t<T>* __restrict__ reg,
                                                    const vec2_t<T>* __restrict__ smem) {
    detail::check_shape<sL::N, sL::batch>();
    constexpr int N = sL::N;
    const int tid = detail::block_tid();
#pragma unroll
    for (int j = 0; j < 16; ++j)
        reg[j] = smem[sL::at(fragment_element<T, N>(tid, j), fragment_transform<T, N>(tid, j))];
}

// Fragment -> shared memory described by sL (reference thunderfft.cuh:106-110).
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_reg2smem(vec2_t<T>* __restrict__ smem,
                                                    const vec2_t<T>* __restrict__ reg) {
    detail::check_shape<sL::N, sL::batch>();
    constexpr int N = sL::N;
    const int tid = detail::block_tid();
#pragma unroll
    for (int j = 0; j < 16; ++j)
        smem[sL::at(fragment_element<T, N>(tid, j), fragment_transform<T, N>(tid, j))] = reg[j];
}

// Contiguous global tile -> shared memory described by sL (reference
// thunderfft.cuh:114-118); consecutive lanes read consecutive elements.
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_gmem2smem(vec2_t<T>* __restrict__ smem,
                                                     const vec2_t<T>* __restrict__ gmem) {
    const int tid = detail::block_tid();
    constexpr int kTotal = sL::N * sL::batch;
    constexpr int kVec = 16 / static_cast<int>(sizeof(vec2_t<T>));  // values per 16-byte load
    constexpr bool kWhole = kTotal % (256 * kVec) == 0;
    if (kWhole && (reinterpret_cast<unsigned long long>(gmem) & 15) == 0) {
        // 16-byte loads of kVec consecutive values
#pragma unroll 4
        for (int e = kVec * tid; e < kTotal; e += 256 * kVec) {
            const thff::u32x4 w = thff::ld_nt(reinterpret_cast<const thff::u32x4*>(gmem + e));
            vec2_t<T> v[kVec];
            __builtin_memcpy(v, &w, 16);
#pragma unroll
            for (int c = 0; c < kVec; ++c) smem[sL::at((e + c) % sL::N, (e + c) / sL::N)] = v[c];
        }
    } else {
#pragma unroll 4
        for (int e = tid; e < kTotal; e += 256) smem[sL::at(e % sL::N, e / sL::N)] = gmem[e];
    }
}

// Shared memory described by sL -> contiguous global tile (reference
// thunderfft.cuh:122-126).
template <typename T, typename sL>
__device__ __forceinline__ void ThunderFFT_smem2gmem(vec2_t<T>* __restrict__ gmem,
                                                     const vec2_t<T>* __restrict__ smem) {
    static_assert(!sL::reversed, "ThunderFFT_smem2gmem: an output layout must not be reversed");
    const int tid = detail::block_tid();
    constexpr int kTotal = sL::N * sL::batch;
    constexpr int kVec = 16 / static_cast<int>(sizeof(vec2_t<T>));
    constexpr bool kWhole = kTotal % (256 * kVec) == 0;
    if (kWhole && (reinterpret_cast<unsigned long long>(gmem) & 15) == 0) {
#pragma unroll 4
        for (int e = kVec * tid; e < kTotal; e += 256 * kVec) {
            vec2_t<T> v[kVec];
#pragma unroll
            for (int c = 0; c < kVec; ++c) v[c] = smem[sL::at((e + c) % sL::N, (e + c) / sL::N)];
            thff::u32x4 w;
            __builtin_memcpy(&w, v, 16);
            thff::st_nt(reinterpret_cast<thff::u32x4*>(gmem + e), w);
        }
    } else {
#pragma unroll 4
        for (int e = tid; e < kTotal; e += 256) gmem[e] = smem[sL::at(e % sL::N, e / sL::N)];
    }
}

}  // namespace thunderfft
