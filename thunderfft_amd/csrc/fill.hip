// fill.hip -- device generator for the seeded U[-1,1) benchmark/test inputs.
// Component c gets 2 * (splitmix64(seed ^ c) >> 40) * 2^-24 - 1 (exact in
// fp32); half storage rounds it to nearest-even.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "launch.hpp"

namespace thff {
namespace {

__device__ __forceinline__ unsigned long long splitmix64(unsigned long long z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float uniform_component(unsigned long long seed, unsigned long long c) {
    const unsigned long long r = splitmix64(seed ^ c) >> 40;
    return static_cast<float>(r) * (1.0f / 8388608.0f) - 1.0f;
}

template <class IO>
__global__ __launch_bounds__(256) void fill_uniform_kernel(IO* out, long long count,
                                                           unsigned long long seed,
                                                           long long first_element) {
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long e = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; e < count;
         e += stride) {
        const unsigned long long c = 2ull * static_cast<unsigned long long>(first_element + e);
        const float re = uniform_component(seed, c);
        const float im = uniform_component(seed, c + 1);
        if constexpr (sizeof(IO) == 8)
            out[e] = make_float2(re, im);
        else
            out[e] = __floats2half2_rn(re, im);
    }
}

// Streaming copy: one 16-byte vector per lane, non-temporal load and store.
// Of 1, 2, 4 and 8 vectors per lane (all loads before all stores), one
// streams best on MI355X: 512 MiB each way at 6.60 TB/s against 6.20, 6.11
// and 5.85 TB/s.
using u32x4v = unsigned __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void copy_nt_kernel(const u32x4v* __restrict__ src,
                                                      u32x4v* __restrict__ dst, long long n16) {
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

hipError_t launch_copy_nt(void* dst, const void* src, long long bytes, hipStream_t stream) {
    const long long n16 = bytes / 16;
    if (n16 <= 0) return hipSuccess;
    const long long blocks = (n16 + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    copy_nt_kernel<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(
        static_cast<const u32x4v*>(src), static_cast<u32x4v*>(dst), n16);
    return hipGetLastError();
}

hipError_t launch_fill_uniform(int precision, void* out, long long count, unsigned long long seed,
                               long long first_element, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    long long blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (precision == 0)
        fill_uniform_kernel<float2><<<static_cast<unsigned>(blocks), 256, 0, stream>>>(
            static_cast<float2*>(out), count, seed, first_element);
    else
        fill_uniform_kernel<__half2><<<static_cast<unsigned>(blocks), 256, 0, stream>>>(
            static_cast<__half2*>(out), count, seed, first_element);
    return hipGetLastError();
}

}  // namespace thff
