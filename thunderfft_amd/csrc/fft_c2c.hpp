// fft_c2c.hpp -- the batched out-of-place C2C kernel for one (storage, N, direction).
//
// Replaces detail::ThunderFFT_global_kernel<T,N,fwd> of the reference
// (include/thunderfft/detail/kernel/global_kernel.cuh:21-100): natural-order
// signals of N complex values at in[b*N], out[b*N]; the last workgroup may
// hold fewer than FPB valid transforms, whose inputs are never read and whose
// outputs are never written.
//
// Layout per workgroup (256 lanes = 4 wave64s): every transform is owned by
// TPF = N/16 lanes holding 16 complex values each.  N <= 1024: each wave owns
// 1024/N whole transforms and a private LDS region, synchronised at wave
// scope; the wave's 1024 contiguous input values are staged through LDS with
// 16-byte loads when N < 1024, so global traffic stays fully coalesced.
// N = 2048/4096: a transform spans 2/4 waves and passes synchronise the
// workgroup.  LDS holds fp32 complex values padded by one slot every 16.
#pragma once

#include "fft_core.hpp"

namespace thff {

template <int N>
struct C2CPlan {
    static_assert(N == 64 || N == 128 || N == 256 || N == 512 || N == 1024 || N == 2048 ||
                      N == 4096,
                  "unsupported transform length");
    static constexpr int kE = 16;                 // complex values per lane
    static constexpr int kTPF = N / kE;           // lanes per transform
    static constexpr int kWG = 256;               // lanes per workgroup
    static constexpr int kFPB = kWG / kTPF;       // transforms per workgroup
    static constexpr int kR0 = 16;
    static constexpr int kR1 = N == 64 ? 4 : N == 128 ? 8 : 16;
    static constexpr int kR2 = N / (kR0 * kR1);   // 1 when two passes suffice
    static constexpr bool kWaveLocal = kTPF <= 64;
    static constexpr bool kStaged = kTPF < 64;
    static constexpr int kSlot = N + N / 16;      // padded LDS slots per transform
    static constexpr int kLdsSlots = kFPB * kSlot;
};

__device__ __forceinline__ int lds_pad(int i) { return i + (i >> 4); }

template <bool WaveLocal>
__device__ __forceinline__ void region_sync() {
    if constexpr (WaveLocal)
        wave_lds_sync();
    else
        __syncthreads();
}

// Twiddle W_{LR}^{e'} for the pass, read from the fp32 table tw[m] =
// (cos, sin)(2*pi*m/N) (positive angle, as the reference's table
// thunderfft_impl_twiddle.cuh:76-91) and conjugated for the forward direction.
template <int N, bool FWD>
__device__ __forceinline__ cpx apply_twiddle(cpx v, const float2* __restrict__ tw, int e) {
    const float2 w = tw[e & (N - 1)];
    return FWD ? cmulc(v, cpx{w.x, w.y}) : cmul(v, cpx{w.x, w.y});
}

// One Stockham pass p >= 1: write the previous pass's outputs to LDS, read
// this pass's inputs, twiddle, DFT.
template <int N, bool FWD, int R, int L, int RPrev, int LPrev>
__device__ __forceinline__ void stockham_pass(cpx (&v)[16], cpx* slot, int t,
                                              const float2* __restrict__ tw) {
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
        const int k = b % L;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            cpx x = slot[lds_pad(b + j * (N / R))];
            if (j > 0) x = apply_twiddle<N, FWD>(x, tw, j * k * (N / (L * R)));
            v[q * R + j] = x;
        }
        Dft<R, FWD>::run(v + q * R);
    }
}

template <class IO, int N, bool FWD>
__global__ __launch_bounds__(256) void c2c_kernel(const IO* __restrict__ in, IO* __restrict__ out,
                                                  int batch, const float2* __restrict__ tw) {
    using P = C2CPlan<N>;
    __shared__ cpx lds[P::kLdsSlots];
    const int tid = threadIdx.x;
    const int f = tid / P::kTPF;  // transform slot within the workgroup
    const int t = tid % P::kTPF;  // lane within the transform
    const long long first = static_cast<long long>(blockIdx.x) * P::kFPB;
    cpx* slot = lds + f * P::kSlot;
    cpx v[16];

    // ---- load pass-0 inputs: x[t + j*TPF], j < 16 ----
    if constexpr (P::kStaged) {
        constexpr int kFPW = 64 / P::kTPF;  // transforms per wave
        constexpr int kVec = Io<IO>::kVec;
        const int wave = tid >> 6, lane = tid & 63;
        const long long wfirst = first + wave * kFPW;
        const long long left = static_cast<long long>(batch) - wfirst;
        const int valid = left <= 0 ? 0 : (left >= kFPW ? 1024 : static_cast<int>(left) * N);
        cpx* chunk = lds + wave * kFPW * P::kSlot;
        const IO* src = in + wfirst * N;
#pragma unroll
        for (int i = 0; i < 1024 / (64 * kVec); ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            cpx q[kVec];
            if (e < valid) {
                Io<IO>::load_vec(src + e, q);
            } else {
#pragma unroll
                for (int c = 0; c < kVec; ++c) q[c] = {0.f, 0.f};
            }
#pragma unroll
            for (int c = 0; c < kVec; ++c) chunk[lds_pad(e + c)] = q[c];
        }
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = slot[lds_pad(t + j * P::kTPF)];
    } else {
        const bool active = first + f < batch;
        const IO* src = in + (first + f) * N;
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = active ? Io<IO>::load(src + t + j * P::kTPF) : cpx{0.f, 0.f};
    }

    // ---- pass 0: radix 16 over stride-TPF inputs (L = 1, no twiddle) ----
    Dft<16, FWD>::run(v);
    // ---- pass 1 ----
    stockham_pass<N, FWD, P::kR1, 16, 16, 1>(v, slot, t, tw);
    constexpr int kRLast = P::kR2 > 1 ? P::kR2 : P::kR1;
    // ---- pass 2 ----
    if constexpr (P::kR2 > 1) stockham_pass<N, FWD, P::kR2, 16 * P::kR1, P::kR1, 16>(v, slot, t, tw);

    // ---- store: last pass output m of butterfly b = t + TPF*q is y[b + m*N/RLast] ----
    if constexpr (P::kStaged) {
        region_sync<true>();
#pragma unroll
        for (int q = 0; q < 16 / kRLast; ++q) {
            const int b = t + P::kTPF * q;
#pragma unroll
            for (int m = 0; m < kRLast; ++m) slot[lds_pad(b + m * (N / kRLast))] = v[q * kRLast + m];
        }
        wave_lds_sync();
        constexpr int kFPW = 64 / P::kTPF;
        constexpr int kVec = Io<IO>::kVec;
        const int wave = tid >> 6, lane = tid & 63;
        const long long wfirst = first + wave * kFPW;
        const long long left = static_cast<long long>(batch) - wfirst;
        const int valid = left <= 0 ? 0 : (left >= kFPW ? 1024 : static_cast<int>(left) * N);
        const cpx* chunk = lds + wave * kFPW * P::kSlot;
        IO* dst = out + wfirst * N;
#pragma unroll
        for (int i = 0; i < 1024 / (64 * kVec); ++i) {
            const int e = kVec * lane + 64 * kVec * i;
            if (e < valid) {
                cpx q[kVec];
#pragma unroll
                for (int c = 0; c < kVec; ++c) q[c] = chunk[lds_pad(e + c)];
                Io<IO>::store_vec(dst + e, q);
            }
        }
    } else {
        if (first + f < batch) {
            IO* dst = out + (first + f) * N;
#pragma unroll
            for (int q = 0; q < 16 / kRLast; ++q) {
                const int b = t + P::kTPF * q;
#pragma unroll
                for (int m = 0; m < kRLast; ++m) Io<IO>::store(dst + b + m * (N / kRLast), v[q * kRLast + m]);
            }
        }
    }
}

}  // namespace thff
