// fft_core.hpp -- register/LDS building blocks of the gfx950 batched C2C FFT.
//
// Arithmetic is fp32 for both storage types (float2 and half2): half inputs
// are widened on load and rounded once, round-to-nearest-even, on store.
//
// Transform convention (include/thunderfft/thunderfft.cuh:129-141 of the
// reference): forward X[k] = sum_n x[n] exp(-2*pi*i*n*k/N), inverse uses
// exp(+...), neither is normalized; natural order in and out.
//
// Algorithm: self-sorting (Stockham) decimation-in-time passes.  A pass of
// radix R after sub-transforms of length L have been formed treats butterfly
// b (0 <= b < N/R): k = b mod L, inputs x[b + j*N/R] (j < R) are multiplied
// by W_{L*R}^{j*k}, an R-point DFT gives outputs y_m written to
// (b - k)*R + k + m*L.  Inputs of every pass are unit-stride across
// threads, so pass 0 reads global memory coalesced and the last pass
// (L*R = N) writes y[b + m*N/R], also coalesced.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

namespace thff {

struct cpx {
    float re, im;
};

__device__ __forceinline__ cpx cadd(cpx a, cpx b) { return {a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ cpx csub(cpx a, cpx b) { return {a.re - b.re, a.im - b.im}; }

// a * w  (w = c + i s)
__device__ __forceinline__ cpx cmul(cpx a, cpx w) {
    return {a.re * w.re - a.im * w.im, a.re * w.im + a.im * w.re};
}
// a * conj(w)
__device__ __forceinline__ cpx cmulc(cpx a, cpx w) {
    return {a.re * w.re + a.im * w.im, a.im * w.re - a.re * w.im};
}

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// cos(2*pi*e/16), sin(2*pi*e/16), e = 0..15 (correctly rounded constants)
constexpr float kCos16[16] = {
    1.0f, 0.92387953251128675613f, 0.70710678118654752440f, 0.38268343236508977173f,
    0.0f, -0.38268343236508977173f, -0.70710678118654752440f, -0.92387953251128675613f,
    -1.0f, -0.92387953251128675613f, -0.70710678118654752440f, -0.38268343236508977173f,
    0.0f, 0.38268343236508977173f, 0.70710678118654752440f, 0.92387953251128675613f};
constexpr float kSin16[16] = {
    0.0f, 0.38268343236508977173f, 0.70710678118654752440f, 0.92387953251128675613f,
    1.0f, 0.92387953251128675613f, 0.70710678118654752440f, 0.38268343236508977173f,
    0.0f, -0.38268343236508977173f, -0.70710678118654752440f, -0.92387953251128675613f,
    -1.0f, -0.92387953251128675613f, -0.70710678118654752440f, -0.38268343236508977173f};

// (cos, sin)(2 pi num / den) for a power-of-two den, computed with the
// hardware transcendentals (v_cos_f32 / v_sin_f32, whose argument is in
// revolutions) with no memory access: num is reduced mod den first, so the
// argument num/den in [0, 1) is exact.  Used where the result is rounded to
// f16 or applied to data that is (the device API's fp16 coefficients): the
// table of ThunderFFTInitialize stays the source of every fp32 twiddle.
__device__ __forceinline__ cpx cis_rev(int num, int den) {
    const float r = static_cast<float>(num & (den - 1)) / static_cast<float>(den);
    return {__builtin_amdgcn_cosf(r), __builtin_amdgcn_sinf(r)};
}

// a * W_R^E with W_R = exp(-2*pi*i/R) (forward) or exp(+2*pi*i/R) (inverse).
// R divides 16; multiplications by +-1 and +-i cost no multiplies.
template <int R, int E, bool FWD>
__device__ __forceinline__ cpx rot(cpx a) {
    constexpr int e = ((E % R) + R) % R;
    constexpr int e16 = e * (16 / R);
    if constexpr (e16 == 0) {
        return a;
    } else if constexpr (e16 == 8) {
        return {-a.re, -a.im};
    } else if constexpr (e16 == 4) {  // forward: * (-i)
        return FWD ? cpx{a.im, -a.re} : cpx{-a.im, a.re};
    } else if constexpr (e16 == 12) {  // forward: * (+i)
        return FWD ? cpx{-a.im, a.re} : cpx{a.im, -a.re};
    } else {
        constexpr float c = kCos16[e16], s = kSin16[e16];
        if constexpr (FWD)
            return {a.re * c + a.im * s, a.im * c - a.re * s};
        else
            return {a.re * c - a.im * s, a.im * c + a.re * s};
    }
}

// In-register R-point DFT, natural order in and out, R in {1,2,4,8,16}.
template <int R, bool FWD>
struct Dft {
    // R = P * Q four-step: n = Q*n1 + n2, k = k1 + P*k2.
    static constexpr int Q = 4;
    static constexpr int P = R / Q;
    static_assert(R == 8 || R == 16, "Dft: unsupported radix");
    __device__ __forceinline__ static void run(cpx* x) {
        cpx a[Q][P];
        static_for<0, Q>([&](auto n2) {
            constexpr int N2 = decltype(n2)::value;
            static_for<0, P>([&](auto n1) { a[N2][decltype(n1)::value] = x[Q * decltype(n1)::value + N2]; });
            Dft<P, FWD>::run(a[N2]);
            static_for<0, P>([&](auto k1) {
                constexpr int K1 = decltype(k1)::value;
                a[N2][K1] = rot<R, N2 * K1, FWD>(a[N2][K1]);
            });
        });
        static_for<0, P>([&](auto k1) {
            constexpr int K1 = decltype(k1)::value;
            cpx b[Q];
            static_for<0, Q>([&](auto n2) { b[decltype(n2)::value] = a[decltype(n2)::value][K1]; });
            Dft<Q, FWD>::run(b);
            static_for<0, Q>([&](auto k2) { x[K1 + P * decltype(k2)::value] = b[decltype(k2)::value]; });
        });
    }
};

template <bool FWD>
struct Dft<1, FWD> {
    __device__ __forceinline__ static void run(cpx*) {}
};

template <bool FWD>
struct Dft<2, FWD> {
    __device__ __forceinline__ static void run(cpx* x) {
        const cpx a = x[0], b = x[1];
        x[0] = cadd(a, b);
        x[1] = csub(a, b);
    }
};

template <bool FWD>
struct Dft<4, FWD> {
    __device__ __forceinline__ static void run(cpx* x) {
        const cpx t0 = cadd(x[0], x[2]), t1 = csub(x[0], x[2]);
        const cpx t2 = cadd(x[1], x[3]), t3 = rot<4, 1, FWD>(csub(x[1], x[3]));
        x[0] = cadd(t0, t2);
        x[2] = csub(t0, t2);
        x[1] = cadd(t1, t3);
        x[3] = csub(t1, t3);
    }
};

// ---------------------------------------------------------------------------
// Storage types.  float2 holds (re, im); __half2 holds low = re, high = im
// (the reference's vec2_t<half>, include/thunderfft/detail/util_cuda.h:46-49).
// ---------------------------------------------------------------------------
using u32x2 = unsigned __attribute__((ext_vector_type(2)));
using u32x4 = unsigned __attribute__((ext_vector_type(4)));

// Non-temporal global accesses (streamed data, touched once).
template <class W>
__device__ __forceinline__ W ld_nt(const W* p) {
    return __builtin_nontemporal_load(p);
}
template <class W>
__device__ __forceinline__ void st_nt(W* p, W w) {
    __builtin_nontemporal_store(w, p);
}

// Bit casts taken on plain scalars: clang mis-evaluates __builtin_bit_cast
// applied directly to an ext-vector element (w.y read as w.x), so elements
// are always passed by value first.
__device__ __forceinline__ float as_f32(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ unsigned as_u32(float f) { return __builtin_bit_cast(unsigned, f); }

template <class IO>
struct Io;

// W1 holds one complex value, W4 one 16-byte vector of kVec values.
template <>
struct Io<float2> {
    static constexpr int kVec = 2;
    using W1 = u32x2;
    using W4 = u32x4;
    __device__ __forceinline__ static cpx decode1(W1 w) { return {as_f32(w.x), as_f32(w.y)}; }
    __device__ __forceinline__ static W1 encode1(cpx v) { return W1{as_u32(v.re), as_u32(v.im)}; }
    __device__ __forceinline__ static void decode4(W4 w, cpx* v) {
        v[0] = {as_f32(w.x), as_f32(w.y)};
        v[1] = {as_f32(w.z), as_f32(w.w)};
    }
    __device__ __forceinline__ static W4 encode4(const cpx* v) {
        return W4{as_u32(v[0].re), as_u32(v[0].im), as_u32(v[1].re), as_u32(v[1].im)};
    }
};

template <>
struct Io<__half2> {
    static constexpr int kVec = 4;
    using W1 = unsigned;
    using W4 = u32x4;
    __device__ __forceinline__ static cpx unpack(unsigned w) {
        const float2 f = __half22float2(__builtin_bit_cast(__half2, w));
        return {f.x, f.y};
    }
    // Round to nearest even, low half = real.
    __device__ __forceinline__ static unsigned pack(cpx v) {
        return __builtin_bit_cast(unsigned, __floats2half2_rn(v.re, v.im));
    }
    __device__ __forceinline__ static cpx decode1(W1 w) { return unpack(w); }
    __device__ __forceinline__ static W1 encode1(cpx v) { return pack(v); }
    __device__ __forceinline__ static void decode4(W4 w, cpx* v) {
        v[0] = unpack(w.x);
        v[1] = unpack(w.y);
        v[2] = unpack(w.z);
        v[3] = unpack(w.w);
    }
    __device__ __forceinline__ static W4 encode4(const cpx* v) {
        return W4{pack(v[0]), pack(v[1]), pack(v[2]), pack(v[3])};
    }
};

// Synchronisation of an LDS region that only one wavefront touches.  LDS
// operations of one wavefront are performed in program order, so only the
// compiler must be kept from moving LDS accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima, gfx9
// encoding): every vector memory access of the wave has completed.  Placed
// inside a rarely taken branch that loads, it keeps the compiler from
// waiting for everything at the branch's join on every pass: after the join
// it counts only the accesses the common path issued.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

}  // namespace thff
