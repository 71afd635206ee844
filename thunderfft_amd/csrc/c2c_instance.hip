// c2c_instance.hip -- instantiates the C2C kernels of one length THFF_N
// (compiled once per length, -DTHFF_N=64 ... 4096, so the lengths build in
// parallel).
#include "fft_c2c.hpp"
#include "launch.hpp"

#ifndef THFF_N
#error "compile with -DTHFF_N=<transform length>"
#endif

namespace thff {

// Tiles per workgroup, measured on MI355X at batch = 2^26/N (one tile per
// workgroup leaves the most waves resident; two amortise the per-lane
// twiddle setup where a tile holds few transforms).
template <int N>
constexpr int preferred_tiles(int precision) {
    return precision == 0 && N <= 1024 ? 1 : 2;
}

template <int N>
hipError_t launch_c2c(int precision, bool forward, const void* in, void* out, int batch,
                      const float2* tw, int num_cus, hipStream_t stream) {
    using P = C2CPlan<N>;
    const long long ntiles = (static_cast<long long>(batch) + P::kFPB - 1) / P::kFPB;
    // Small batches spread one tile per workgroup over the whole device.
    const int tpb = ntiles >= 16LL * (num_cus > 0 ? num_cus : 256) ? preferred_tiles<N>(precision) : 1;
    const unsigned grid = static_cast<unsigned>((ntiles + tpb - 1) / tpb);
    const dim3 block(P::kWG);
    if (precision == 0) {
        const auto* x = static_cast<const float2*>(in);
        auto* y = static_cast<float2*>(out);
        if (forward)
            c2c_kernel<float2, N, true, false><<<grid, block, 0, stream>>>(x, y, batch, tw, tpb);
        else
            c2c_kernel<float2, N, false, false><<<grid, block, 0, stream>>>(x, y, batch, tw, tpb);
    } else {
        const auto* x = static_cast<const __half2*>(in);
        auto* y = static_cast<__half2*>(out);
        if (forward)
            c2c_kernel<__half2, N, true, false><<<grid, block, 0, stream>>>(x, y, batch, tw, tpb);
        else
            c2c_kernel<__half2, N, false, false><<<grid, block, 0, stream>>>(x, y, batch, tw, tpb);
    }
    return hipGetLastError();
}

template hipError_t launch_c2c<THFF_N>(int, bool, const void*, void*, int, const float2*, int,
                                       hipStream_t);

}  // namespace thff
