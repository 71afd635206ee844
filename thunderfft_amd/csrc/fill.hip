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

}  // namespace

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
