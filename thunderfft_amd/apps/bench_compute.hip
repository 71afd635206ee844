// bench_compute.hip -- in-register repeat kernels for the reference-style
// differential compute time (sample/bench/paper_fft.cu:131-148 and
// sample/bench/baseline/thunderfft_bench.h:7-57): each block loads its tile
// once, runs the transform `repeats` times on it and stores once, so
// (t(2R) - t(R)) / R is the time of one pass of the transform over the batch
// without global-memory traffic.  The repeated values are not meaningful
// (they grow without bound and may overflow) and are never checked, as in
// the reference.  Built into libthff_bench_compute.so for bench.py.
#include "thunderfft/detail/fft_c2c.hpp"
#include "thunderfft/detail/fft_mfma.hpp"
#include "thunderfft/thunderfft.h"

namespace thff {
namespace {

// fp32 arithmetic, VALU passes (the kernel the library runs for float).
template <class IO, int N>
__global__ __launch_bounds__(256) void repeat_valu(const IO* in, IO* out, int batch,
                                                   const float2* tw, int repeats) {
    using P = C2CPlan<N>;
    using T = TileIO<IO, N>;
    __shared__ cpx lds[P::kLdsSlots];
    const T io(lds, threadIdx.x);
    LaneTwiddles<N> w;
    w.load(io.t, tw);
    typename T::Raw r;
    io.load(r, in, blockIdx.x, batch);
    cpx v[16];
    io.stage(r, v);
#pragma unroll 1
    for (int i = 0; i < repeats; ++i) fft_registers<N, true>(v, io.slot, io.t, w);
    io.store(v, out, blockIdx.x, batch);
}

// half2 on MFMA (the kernel the library runs for half, N = 256*C): steps 1-6
// from the LDS staging, the result written back there in natural order.
template <int C>
__global__ __launch_bounds__(256) void repeat_mfma(const __half2* in, __half2* out, int batch,
                                                   const float2* tw, int repeats) {
    using P = MfmaPlan<C>;
    constexpr int N = P::N;
    constexpr int kRaw = P::kVals / 4;
    __shared__ unsigned lds[4 * P::kRegion];
    __shared__ cpx w1[P::kTw1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, q = lane >> 4;
    unsigned* region = lds + wave * P::kRegion;
    f16x8 a[2];
    cpx w2[C > 1 ? C - 1 : 1];
    mfma_setup<C, true>(a, w1, nullptr, w2, tw);
    const Stage3Plain<false> s3{a, w2};
    const long long first = static_cast<long long>(blockIdx.x) * P::kFPB + wave * P::kFPW;
    const bool valid = first + P::kFPW <= batch;
    const __half2* src = in + first * N;
#pragma unroll
    for (int i = 0; i < kRaw; ++i)
        *reinterpret_cast<u32x4*>(region + P::in_pad(4 * lane + 256 * i)) =
            valid ? ld_nt(reinterpret_cast<const u32x4*>(src + 4 * lane + 256 * i)) : u32x4{};
    cpx y[P::kBlocks][4];
#pragma unroll 1
    for (int i = 0; i < repeats; ++i) {
        wave_lds_sync();
        mfma_fft_staged<C, true>(region, a, w1, s3, lane, y);
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < P::kBlocks; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                region[P::in_pad((b / C) * N + n + 16 * (b % C) + P::kM * (q + 4 * r))] =
                    pack_half2(y[b][r]);
    }
    wave_lds_sync();
    if (valid) {
        __half2* dst = out + first * N;
#pragma unroll
        for (int i = 0; i < kRaw; ++i)
            st_nt(reinterpret_cast<u32x4*>(dst + 4 * lane + 256 * i),
                  *reinterpret_cast<const u32x4*>(region + P::in_pad(4 * lane + 256 * i)));
    }
}

}  // namespace
}  // namespace thff

// One launch of the repeat kernel for N = 1024 over `batch` transforms
// (a multiple of the tile size); precision 0 float (VALU), 1 half (MFMA).
// Returns 0, -22 (bad argument: no table for N = 1024, batch not a multiple)
// or -5 (launch error).  Asynchronous on `stream`.
extern "C" int thffx_compute_repeat(int precision, const void* x, void* y, int batch,
                                    int repeats, void* stream) {
    constexpr int N = 1024;
    const void* table = nullptr;
    int tn = 0;
    if (thff_twiddle_info(precision, &table, &tn) != 0 || tn != N || !table) return -22;
    if (!x || !y || x == y || batch <= 0 || repeats < 0 || batch % 4) return -22;
    const auto* tw = static_cast<const float2*>(table);
    auto s = static_cast<hipStream_t>(stream);
    const unsigned grid = batch / 4;
    if (precision == THFF_FLOAT)
        thff::repeat_valu<float2, N><<<grid, 256, 0, s>>>(static_cast<const float2*>(x),
                                                          static_cast<float2*>(y), batch, tw,
                                                          repeats);
    else
        thff::repeat_mfma<4><<<grid, 256, 0, s>>>(static_cast<const __half2*>(x),
                                                  static_cast<__half2*>(y), batch, tw, repeats);
    return hipGetLastError() == hipSuccess ? 0 : -5;
}
