// device_example.hip -- kernels written against the public device-side API
// (<thunderfft/thunderfft.cuh>), as a caller of the library would write them;
// built into libthff_device_example.so for the GPU tests.
//
//   thffx_device_fft      gmem -> smem (layout_t) -> fragment -> ThunderFFT_kernel_reg
//                         -> smem -> gmem, with 64 sentinel values after the
//                         workspace that must survive (the reference's
//                         validate_core, sample/validation/fft_validation.cu:84-123);
//   thffx_device_fft_reg  the same through ThunderFFT_gmem2reg / reg2gmem only;
//   thffx_fused_filter    forward FFT x per-bin filter x inverse FFT / N in one
//                         kernel (the reference's fused-convolution pattern);
//   thffx_device_fft_reversed_in
//                         thffx_device_fft with a Reversed = true input layout;
//   thffx_device_fft_w, thffx_fused_filter_w
//                         the same two with ThunderFFT_kernel_reg(reg, W, ws) in
//                         the reference's argument types: for half, W from
//                         unit_fp16::make_reg_b_precompute<N, fwd> (built once
//                         per kernel, no table), for float the table.
// Every entry point requires batch to be a multiple of batch_per_block<N>
// and returns 0, -22 (bad argument) or -5 (launch error).
#include <thunderfft/thunderfft.cuh>

#include <type_traits>

namespace {

constexpr int kGuard = 64;
constexpr float kGuardRe = 299.f, kGuardIm = -299.f;

// kReversedIn: the input is staged through a layout_t with Reversed = true
// (a reference fused kernel's input layout), the output through the same
// layout with Reversed = false.
template <class T, int N, bool FWD, bool kReversedIn = false>
__global__ __launch_bounds__(256) void device_fft(const vec2_t<T>* in, vec2_t<T>* out,
                                                  const float2* tw, int* guard_changes) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    using L = thunderfft::layout_t<N, BPB, 1, N + thunderfft::pad_h(N), 16, 1, false>;
    using Lin = thunderfft::layout_t<N, BPB, 1, N + thunderfft::pad_h(N), 16, 1, kReversedIn>;
    constexpr int kWorkBytes = thunderfft::workspace_bytes<N, BPB>;
    // The staging tile (L) and the FFT workspace share one LDS buffer.
    constexpr int kStageBytes = (L::at(N - 1, BPB - 1) + 1) * sizeof(vec2_t<T>);
    constexpr int kBytes = kWorkBytes > kStageBytes ? kWorkBytes : kStageBytes;
    __shared__ __align__(16) unsigned char raw[kBytes + kGuard * sizeof(float2)];
    auto* stage = reinterpret_cast<vec2_t<T>*>(raw);
    auto* guard = reinterpret_cast<float2*>(raw + kBytes);
    const int tid = threadIdx.x;
    if (tid < kGuard) guard[tid] = make_float2(kGuardRe, kGuardIm);

    thunderfft::lane_twiddles<N> w;
    thunderfft::ThunderFFT_load_twiddles<N>(w, tw);
    vec2_t<T> reg[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_gmem2smem<T, Lin>(stage, in + blockIdx.x * BPB * N);
    __syncthreads();
    thunderfft::ThunderFFT_smem2reg<T, Lin>(reg, stage);
    __syncthreads();
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, FWD>(reg, w, raw);
    __syncthreads();
    thunderfft::ThunderFFT_reg2smem<T, L>(stage, reg);
    __syncthreads();
    thunderfft::ThunderFFT_smem2gmem<T, L>(out + blockIdx.x * BPB * N, stage);
    if (tid < kGuard) {
        const float2 g = guard[tid];
        if (g.x != kGuardRe || g.y != kGuardIm) atomicAdd(guard_changes, 1);
    }
}

template <class T, int N, bool FWD>
__global__ __launch_bounds__(256) void device_fft_reg(const vec2_t<T>* in, vec2_t<T>* out,
                                                      const float2* tw) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    __shared__ __align__(16) unsigned char work[thunderfft::workspace_bytes<N, BPB>];
    vec2_t<T> reg[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_gmem2reg<T, N, BPB>(reg, in + blockIdx.x * BPB * N);
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, FWD>(reg, tw, work);
    thunderfft::ThunderFFT_reg2gmem<T, N, BPB>(out + blockIdx.x * BPB * N, reg);
}

// y = IFFT(FFT(x) * H) / N, H given per frequency bin in natural order.
template <class T, int N>
__global__ __launch_bounds__(256) void fused_filter(const vec2_t<T>* in, vec2_t<T>* out,
                                                    const float2* H, const float2* tw) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    __shared__ __align__(16) unsigned char work[thunderfft::workspace_bytes<N, BPB>];
    thunderfft::lane_twiddles<N> w;
    thunderfft::ThunderFFT_load_twiddles<N>(w, tw);
    vec2_t<T> reg[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_gmem2reg<T, N, BPB>(reg, in + blockIdx.x * BPB * N);
    // fp32 product; register j holds bin fragment_element<T, N>(tid, j)
    float2 spec[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, true>(reg, w, work);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        float2 a;
        if constexpr (sizeof(vec2_t<T>) == 8)
            a = reinterpret_cast<const float2&>(reg[j]);
        else
            a = __half22float2(reinterpret_cast<const __half2&>(reg[j]));
        const float2 h = H[thunderfft::fragment_element<T, N>(threadIdx.x, j)];
        spec[j] = make_float2((a.x * h.x - a.y * h.y) / N, (a.x * h.y + a.y * h.x) / N);
        if constexpr (sizeof(vec2_t<T>) == 8)
            reinterpret_cast<float2&>(reg[j]) = spec[j];
        else
            reinterpret_cast<__half2&>(reg[j]) = __floats2half2_rn(spec[j].x, spec[j].y);
    }
    __syncthreads();  // the forward transform's workspace reads are done
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, false>(reg, w, work);
    thunderfft::ThunderFFT_reg2gmem<T, N, BPB>(out + blockIdx.x * BPB * N, reg);
}

// The coefficient argument of ThunderFFT_kernel_reg(reg, W, ws) in the
// reference's types: half -> this lane's precomputed coefficients in an
// array of the size the reference's fused kernels declare (W_fwd[28] for
// N <= 128, sample/conv1d/main.cu:61; W_fwd[36] otherwise,
// conv1d_fullfft_l4096_thunder.cu:298), float -> the table.
template <class T, int N, bool FWD>
struct KernelRegW {
    vec2_t<T> coeffs[std::is_same_v<T, half> ? (N <= 128 ? 28 : 36) : 1];
    vec2_t<T>* w;
    __device__ explicit KernelRegW(const float2* tw) {
        if constexpr (std::is_same_v<T, half>) {
            thunderfft::unit_fp16::make_reg_b_precompute<N, FWD>(coeffs);
            w = coeffs;
        } else {
            w = const_cast<float2*>(tw);
        }
    }
};

template <class T, int N, bool FWD>
__global__ __launch_bounds__(256) void device_fft_w(const vec2_t<T>* in, vec2_t<T>* out,
                                                    const float2* tw) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    __shared__ __align__(16) unsigned char work[thunderfft::workspace_bytes<N, BPB>];
    KernelRegW<T, N, FWD> W(tw);
    vec2_t<T> reg[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_gmem2reg<T, N, BPB>(reg, in + blockIdx.x * BPB * N);
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, FWD>(reg, W.w, work);
    thunderfft::ThunderFFT_reg2gmem<T, N, BPB>(out + blockIdx.x * BPB * N, reg);
}

// fused_filter with precomputed coefficients of both directions.
template <class T, int N>
__global__ __launch_bounds__(256) void fused_filter_w(const vec2_t<T>* in, vec2_t<T>* out,
                                                      const float2* H, const float2* tw) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    __shared__ __align__(16) unsigned char work[thunderfft::workspace_bytes<N, BPB>];
    KernelRegW<T, N, true> Wf(tw);
    KernelRegW<T, N, false> Wi(tw);
    vec2_t<T> reg[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_gmem2reg<T, N, BPB>(reg, in + blockIdx.x * BPB * N);
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, true>(reg, Wf.w, work);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        float2 a;
        if constexpr (sizeof(vec2_t<T>) == 8)
            a = reinterpret_cast<const float2&>(reg[j]);
        else
            a = __half22float2(reinterpret_cast<const __half2&>(reg[j]));
        const float2 h = H[thunderfft::fragment_element<T, N>(threadIdx.x, j)];
        const float2 p = make_float2((a.x * h.x - a.y * h.y) / N, (a.x * h.y + a.y * h.x) / N);
        if constexpr (sizeof(vec2_t<T>) == 8)
            reinterpret_cast<float2&>(reg[j]) = p;
        else
            reinterpret_cast<__half2&>(reg[j]) = __floats2half2_rn(p.x, p.y);
    }
    __syncthreads();  // the forward transform's workspace reads are done
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, false>(reg, Wi.w, work);
    thunderfft::ThunderFFT_reg2gmem<T, N, BPB>(out + blockIdx.x * BPB * N, reg);
}

// (transform, element) of every (lane, register) of one block:
// map[2 * (16 * tid + j)] = fragment_transform, [... + 1] = fragment_element.
template <class T, int N>
__global__ __launch_bounds__(256) void fragment_map(int* map) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < thunderfft::elements_per_thread; ++j) {
        map[2 * (16 * tid + j)] = thunderfft::fragment_transform<T, N>(tid, j);
        map[2 * (16 * tid + j) + 1] = thunderfft::fragment_element<T, N>(tid, j);
    }
}

template <class T>
int launch_map(int n, int* map, hipStream_t s) {
    switch (n) {
    case 64: fragment_map<T, 64><<<1, 256, 0, s>>>(map); break;
    case 128: fragment_map<T, 128><<<1, 256, 0, s>>>(map); break;
    case 256: fragment_map<T, 256><<<1, 256, 0, s>>>(map); break;
    case 512: fragment_map<T, 512><<<1, 256, 0, s>>>(map); break;
    case 1024: fragment_map<T, 1024><<<1, 256, 0, s>>>(map); break;
    case 2048: fragment_map<T, 2048><<<1, 256, 0, s>>>(map); break;
    case 4096: fragment_map<T, 4096><<<1, 256, 0, s>>>(map); break;
    default: return -22;
    }
    return hipGetLastError() == hipSuccess && hipStreamSynchronize(s) == hipSuccess ? 0 : -5;
}

template <class T, int N>
int launch(int kind, int forward, const void* x, void* y, const void* H, int batch,
           const float2* tw, int* guard, hipStream_t s) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    if (batch <= 0 || batch % BPB) return -22;
    const unsigned grid = batch / BPB;
    auto* in = static_cast<const vec2_t<T>*>(x);
    auto* out = static_cast<vec2_t<T>*>(y);
    if (kind == 0) {
        if (forward) device_fft<T, N, true><<<grid, 256, 0, s>>>(in, out, tw, guard);
        else device_fft<T, N, false><<<grid, 256, 0, s>>>(in, out, tw, guard);
    } else if (kind == 1) {
        if (forward) device_fft_reg<T, N, true><<<grid, 256, 0, s>>>(in, out, tw);
        else device_fft_reg<T, N, false><<<grid, 256, 0, s>>>(in, out, tw);
    } else if (kind == 2) {
        fused_filter<T, N><<<grid, 256, 0, s>>>(in, out, static_cast<const float2*>(H), tw);
    } else if (kind == 5) {
        if (forward) device_fft<T, N, true, true><<<grid, 256, 0, s>>>(in, out, tw, guard);
        else device_fft<T, N, false, true><<<grid, 256, 0, s>>>(in, out, tw, guard);
    } else if (kind == 3) {
        if (forward) device_fft_w<T, N, true><<<grid, 256, 0, s>>>(in, out, tw);
        else device_fft_w<T, N, false><<<grid, 256, 0, s>>>(in, out, tw);
    } else {
        fused_filter_w<T, N><<<grid, 256, 0, s>>>(in, out, static_cast<const float2*>(H), tw);
    }
    return hipGetLastError() == hipSuccess && hipStreamSynchronize(s) == hipSuccess ? 0 : -5;
}

template <class T>
int dispatch(int n, int kind, int forward, const void* x, void* y, const void* H, int batch,
             const float2* tw, int* guard, hipStream_t s) {
    switch (n) {
    case 64: return launch<T, 64>(kind, forward, x, y, H, batch, tw, guard, s);
    case 128: return launch<T, 128>(kind, forward, x, y, H, batch, tw, guard, s);
    case 256: return launch<T, 256>(kind, forward, x, y, H, batch, tw, guard, s);
    case 512: return launch<T, 512>(kind, forward, x, y, H, batch, tw, guard, s);
    case 1024: return launch<T, 1024>(kind, forward, x, y, H, batch, tw, guard, s);
    case 2048: return launch<T, 2048>(kind, forward, x, y, H, batch, tw, guard, s);
    case 4096: return launch<T, 4096>(kind, forward, x, y, H, batch, tw, guard, s);
    default: return -22;
    }
}

int run(int precision, int n, int kind, int forward, const void* x, void* y, const void* H,
        int batch, int* guard, void* stream) {
    if (!x || !y || x == y || ((kind == 0 || kind == 5) && !guard) ||
        ((kind == 2 || kind == 4) && !H))
        return -22;
    const void* table = nullptr;
    int tn = 0;
    if (thff_twiddle_info(precision, &table, &tn) != 0 || tn != n || !table) return -22;
    auto* tw = static_cast<const float2*>(table);
    auto s = static_cast<hipStream_t>(stream);
    return precision == THFF_FLOAT ? dispatch<float>(n, kind, forward, x, y, H, batch, tw, guard, s)
                                   : dispatch<half>(n, kind, forward, x, y, H, batch, tw, guard, s);
}

}  // namespace

extern "C" {
// 2 * 256 * 16 ints: the fragment order of (precision, n) for one block.
int thffx_fragment_map(int precision, int n, int* d_map, void* stream) {
    if (!d_map) return -22;
    auto s = static_cast<hipStream_t>(stream);
    return precision == THFF_FLOAT ? launch_map<float>(n, d_map, s) : launch_map<half>(n, d_map, s);
}

int thffx_device_fft(int precision, int n, int forward, const void* x, void* y, int batch,
                     int* d_guard_changes, void* stream) {
    return run(precision, n, 0, forward, x, y, nullptr, batch, d_guard_changes, stream);
}
int thffx_device_fft_reg(int precision, int n, int forward, const void* x, void* y, int batch,
                         void* stream) {
    return run(precision, n, 1, forward, x, y, nullptr, batch, nullptr, stream);
}
int thffx_fused_filter(int precision, int n, const void* x, void* y, const void* d_filter,
                       int batch, void* stream) {
    return run(precision, n, 2, 1, x, y, d_filter, batch, nullptr, stream);
}
int thffx_device_fft_reversed_in(int precision, int n, int forward, const void* x, void* y,
                                 int batch, int* d_guard_changes, void* stream) {
    return run(precision, n, 5, forward, x, y, nullptr, batch, d_guard_changes, stream);
}
int thffx_device_fft_w(int precision, int n, int forward, const void* x, void* y, int batch,
                       void* stream) {
    return run(precision, n, 3, forward, x, y, nullptr, batch, nullptr, stream);
}
int thffx_fused_filter_w(int precision, int n, const void* x, void* y, const void* d_filter,
                         int batch, void* stream) {
    return run(precision, n, 4, 1, x, y, d_filter, batch, nullptr, stream);
}
}
