// thff_paper_fft -- the reference's paper timing adapter
// (sample/bench/paper_fft.cu) on MI355X, with the same command line, CSV
// columns and exit codes:
//
//   thff_paper_fft N fp16|tf32|fp32 register|shared [repeats=1000] [trials=3] [batch=65536]
//
// Kernels are written against the device-side API (<thunderfft/thunderfft.cuh>)
// the way the reference's ThunderFFT_benchmark_reg / _smem kernels
// (sample/bench/baseline/thunderfft_bench.h:7-56,134-178) are:
//   register: HBM -> LDS -> fragment, `repeats` forward ThunderFFT_kernel_reg
//             calls on the fragment, fragment -> LDS -> HBM;
//   shared:   HBM -> LDS, `repeats` x (LDS -> fragment, ThunderFFT_kernel_reg,
//             fragment -> LDS), LDS -> HBM.
// compute_us = (t_2R - t_R) / R, the differential compute time of the
// reference's Table 3 (paper_fft.cu:150-160); e2e_out_of_place_us = the mean
// of 10 single-transform launches.  Before timing, one 64-transform batch of
// seeded complex inputs is checked against hipFFT Z2Z (fp64) of the values
// the storage type holds, gate relative L2 <= 5e-3 (paper_fft.cu:101-127).
// "tf32" selects float storage as in the reference; this build computes it
// in fp32 (CDNA4 has no tf32), and the precision column echoes the argument.
// Exit codes: 0 success, 1 error (bad arguments, HIP/hipFFT failure, gate),
// 2 usage.
#include <hipfft/hipfft.h>
#include <thunderfft/thunderfft.cuh>

#include <type_traits>

#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
void fft_ok(hipfftResult e, const char* what) {
    if (e != HIPFFT_SUCCESS) throw std::runtime_error(std::string(what) + ": hipFFT " +
                                                      std::to_string(static_cast<int>(e)));
}

template <class T>
__device__ vec2_t<T> store_as(float re, float im) {
    if constexpr (std::is_same_v<T, float>)
        return make_float2(re, im);
    else
        return __floats2half2_rn(re, im);
}
template <class T>
__host__ __device__ double2 widen(vec2_t<T> v) {
    if constexpr (std::is_same_v<T, float>)
        return make_double2(v.x, v.y);
    else
        return make_double2(__low2float(v), __high2float(v));
}

// The adapter's inputs (paper_fft.cu:27-45).  With `reference` set: a
// linear-congruential complex value per element, scaled by 1/sqrt(n), and its
// stored value widened into `reference`; without: the timed input, a real
// sinusoid sin(2 pi (i mod n) / n) / sqrt(n).
template <class T>
__global__ void initialize(vec2_t<T>* input, double2* reference, size_t count, int n) {
    const float scale = 1.0f / sqrtf(static_cast<float>(n));
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        float re, im;
        if (reference) {
            unsigned z = static_cast<unsigned>(i) * 1664525u + 1013904223u;
            re = (static_cast<float>(static_cast<int>(z & 65535u)) - 32768.0f) / 32768.0f * scale;
            z = z * 1664525u + 1013904223u;
            im = (static_cast<float>(static_cast<int>(z & 65535u)) - 32768.0f) / 32768.0f * scale;
        } else {
            re = sinf(static_cast<float>(6.2831853071795864769 * static_cast<double>(i % n) / n)) *
                 scale;
            im = 0.0f;
        }
        const vec2_t<T> v = store_as<T>(re, im);
        input[i] = v;
        if (reference) reference[i] = widen<T>(v);
    }
}

// Natural-order staging layout with the library's padding (one slot of
// N + N/16 values per transform).

template <class T, int N, bool kShared>
__global__ __launch_bounds__(256) void repeat_kernel(const vec2_t<T>* __restrict__ in,
                                                     vec2_t<T>* __restrict__ out,
                                                     const float2* __restrict__ table,
                                                     unsigned repeats) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    using L = thunderfft::fragment_layout<T, N>;
    __shared__ __align__(16) unsigned char work[thunderfft::workspace_bytes<N, BPB>];
    auto* staged = reinterpret_cast<vec2_t<T>*>(work);
    // float: the lane's twiddle factors from the table; half: the per-lane
    // coefficients of unit_fp16::make_reg_b_precompute, built once here as
    // in the reference's fused samples (sample/README.md:406-409).
    thunderfft::lane_twiddles<N> tw_lane;
    vec2_t<T> coeffs[std::is_same_v<T, half> ? (N <= 128 ? 28 : 36) : 1];  // the reference's sizes
    if constexpr (std::is_same_v<T, half>)
        thunderfft::unit_fp16::make_reg_b_precompute<N, true>(coeffs);
    else
        thunderfft::ThunderFFT_load_twiddles<N>(tw_lane, table);
    auto fft = [&](vec2_t<T>* reg) {
        if constexpr (std::is_same_v<T, half>)
            thunderfft::ThunderFFT_kernel_reg<T, N, thunderfft::batch_per_block<N>, true>(reg, coeffs,
                                                                                      work);
        else
            thunderfft::ThunderFFT_kernel_reg<T, N, thunderfft::batch_per_block<N>, true>(reg, tw_lane,
                                                                                      work);
    };
    vec2_t<T> reg[thunderfft::elements_per_thread];

    thunderfft::ThunderFFT_gmem2smem<T, L>(staged, in + static_cast<size_t>(blockIdx.x) * BPB * N);
    __syncthreads();
    if constexpr (kShared) {
        for (unsigned r = 0; r < repeats; ++r) {
            thunderfft::ThunderFFT_smem2reg<T, L>(reg, staged);
            __syncthreads();
            fft(reg);
            __syncthreads();
            thunderfft::ThunderFFT_reg2smem<T, L>(staged, reg);
            __syncthreads();
        }
    } else {
        thunderfft::ThunderFFT_smem2reg<T, L>(reg, staged);
        __syncthreads();
        for (unsigned r = 0; r < repeats; ++r) {
            fft(reg);
            __syncthreads();
        }
        thunderfft::ThunderFFT_reg2smem<T, L>(staged, reg);
        __syncthreads();
    }
    thunderfft::ThunderFFT_smem2gmem<T, L>(out + static_cast<size_t>(blockIdx.x) * BPB * N, staged);
}

template <class Launch>
double elapsed_us(Launch launch, int runs) {
    hipEvent_t begin, end;
    hip_ok(hipEventCreate(&begin), "hipEventCreate");
    hip_ok(hipEventCreate(&end), "hipEventCreate");
    hip_ok(hipEventRecord(begin), "hipEventRecord");
    for (int i = 0; i < runs; ++i) launch();
    hip_ok(hipEventRecord(end), "hipEventRecord");
    hip_ok(hipEventSynchronize(end), "hipEventSynchronize");
    float ms = 0.f;
    hip_ok(hipEventElapsedTime(&ms, begin, end), "hipEventElapsedTime");
    (void)hipEventDestroy(begin);
    (void)hipEventDestroy(end);
    return static_cast<double>(ms) * 1000.0 / runs;
}

template <class V>
struct Device {
    V* p = nullptr;
    explicit Device(size_t count) { hip_ok(hipMalloc(&p, count * sizeof(V)), "hipMalloc"); }
    ~Device() { (void)hipFree(p); }
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
};

template <class T, int N, bool kShared>
void run(const std::string& label, int batch, int repeats, int trials) {
    using V = vec2_t<T>;
    constexpr int BPB = thunderfft::batch_per_block<N>;
    constexpr size_t kWorkspace = thunderfft::workspace_bytes<N, BPB>;
    if (batch <= 0 || batch % BPB) throw std::runtime_error("batch must be a positive BPB multiple");
    thunderfft::ThunderFFTInitialize<T>(N);
    const float2* table = thunderfft::ThunderFFT_twiddle_table<T>();
    auto launch = [&](const V* in, V* out, int count, unsigned r) {
        repeat_kernel<T, N, kShared><<<count / BPB, 256>>>(in, out, table, r);
        hip_ok(hipGetLastError(), "repeat_kernel launch");
    };

    // Single-transform gate on a separate, unmutated input (paper_fft.cu:101-127).
    constexpr int kValidationBatch = 64;
    constexpr size_t kValidationCount = static_cast<size_t>(N) * kValidationBatch;
    double rel = 0.0;
    {
        Device<V> vi(kValidationCount), vo(kValidationCount);
        Device<double2> vr(kValidationCount);
        initialize<T><<<128, 256>>>(vi.p, vr.p, kValidationCount, N);
        hip_ok(hipGetLastError(), "initialize");
        hipfftHandle plan;
        fft_ok(hipfftPlan1d(&plan, N, HIPFFT_Z2Z, kValidationBatch), "hipfftPlan1d");
        const hipfftResult fr =
            hipfftExecZ2Z(plan, reinterpret_cast<hipfftDoubleComplex*>(vr.p),
                          reinterpret_cast<hipfftDoubleComplex*>(vr.p), HIPFFT_FORWARD);
        (void)hipfftDestroy(plan);
        fft_ok(fr, "hipfftExecZ2Z");
        launch(vi.p, vo.p, kValidationBatch, 1);
        hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
        std::vector<V> actual(kValidationCount);
        std::vector<double2> reference(kValidationCount);
        hip_ok(hipMemcpy(actual.data(), vo.p, kValidationCount * sizeof(V), hipMemcpyDeviceToHost),
               "hipMemcpy");
        hip_ok(hipMemcpy(reference.data(), vr.p, kValidationCount * sizeof(double2),
                         hipMemcpyDeviceToHost),
               "hipMemcpy");
        double se = 0.0, sr = 0.0;
        bool finite = true;
        for (size_t i = 0; i < kValidationCount; ++i) {
            const double2 a = widen<T>(actual[i]);
            finite = finite && std::isfinite(a.x) && std::isfinite(a.y);
            const double dx = a.x - reference[i].x, dy = a.y - reference[i].y;
            se += dx * dx + dy * dy;
            sr += reference[i].x * reference[i].x + reference[i].y * reference[i].y;
        }
        rel = std::sqrt(se / sr);
        if (!finite || !std::isfinite(rel) || rel > 5e-3)
            throw std::runtime_error("single-FFT correctness gate failed relL2=" +
                                     std::to_string(rel));
    }

    const size_t count = static_cast<size_t>(N) * batch;
    Device<V> input(count), output(count);
    initialize<T><<<1024, 256>>>(input.p, nullptr, count, N);
    hip_ok(hipGetLastError(), "initialize");
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
    // Clock warm-up outside every reported interval (paper_fft.cu:136-138).
    for (int w = 0; w < 3; ++w) {
        launch(input.p, output.p, batch, repeats);
        hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
    }
    for (int t = 0; t < trials; ++t) {
        auto repeated = [&](unsigned r) { return [&, r] { launch(input.p, output.p, batch, r); }; };
        repeated(repeats)();
        hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
        const double t_r = elapsed_us(repeated(repeats), 1);
        repeated(2 * repeats)();
        hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
        const double t_2r = elapsed_us(repeated(2 * repeats), 1);
        if (!(std::isfinite(t_r) && std::isfinite(t_2r) && t_2r > t_r))
            throw std::runtime_error("nonpositive/nonfinite differential timing");
        auto once = [&] { launch(input.p, output.p, batch, 1); };
        once();
        hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
        const double e2e = elapsed_us(once, 10);
        std::printf("%d,%s,%s,%d,%d,%d,%.9g,%.9g,%.9g,%.9g,%.12g,%zu\n", N, label.c_str(),
                    kShared ? "shared" : "register", batch, repeats, t, t_r, t_2r,
                    (t_2r - t_r) / repeats, e2e, rel, kWorkspace);
        std::fflush(stdout);
    }
    thunderfft::ThunderFFTFinalize<T>();
}

template <int N>
void choose(const std::string& precision, bool shared, int batch, int repeats, int trials) {
    if (precision == "fp16") {
        if (shared)
            run<half, N, true>(precision, batch, repeats, trials);
        else
            run<half, N, false>(precision, batch, repeats, trials);
    } else {
        if (shared)
            run<float, N, true>(precision, batch, repeats, trials);
        else
            run<float, N, false>(precision, batch, repeats, trials);
    }
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc < 4 || argc > 7) {
            std::fprintf(stderr,
                         "usage: %s N fp16|tf32|fp32 register|shared [repeats=1000] [trials=3] "
                         "[batch=65536]\n",
                         argv[0]);
            return 2;
        }
        const int n = std::stoi(argv[1]);
        const int repeats = argc > 4 ? std::stoi(argv[4]) : 1000;
        const int trials = argc > 5 ? std::stoi(argv[5]) : 3;
        const int batch = argc > 6 ? std::stoi(argv[6]) : 65536;
        const std::string precision = argv[2], placement = argv[3];
        if ((precision != "fp16" && precision != "tf32" && precision != "fp32") ||
            (placement != "register" && placement != "shared") || repeats <= 0 || trials <= 0)
            throw std::runtime_error("invalid arguments");
        if (n != 64 && n != 128 && n != 256 && n != 512 && n != 1024 && n != 2048 && n != 4096)
            throw std::runtime_error("unsupported N");

        hipDeviceProp_t prop;
        hip_ok(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties");
        int driver = 0, runtime = 0, fft_version = 0;
        hip_ok(hipDriverGetVersion(&driver), "hipDriverGetVersion");
        hip_ok(hipRuntimeGetVersion(&runtime), "hipRuntimeGetVersion");
        fft_ok(hipfftGetVersion(&fft_version), "hipfftGetVersion");
        std::fprintf(stderr, "compiled_HIP=%d runtime=%d driver=%d hipFFT=%d extra_R_warmups=3\n",
                     HIP_VERSION, runtime, driver, fft_version);
        std::fprintf(stderr,
                     "GPU=%s arch=%s batch=%d R=%d trials=%d single_fft_relL2_limit=0.005 "
                     "float_arithmetic=fp32\n",
                     prop.name, prop.gcnArchName, batch, repeats, trials);
        std::puts("N,precision,placement,batch,inside_repeats,trial,t_R_us,t_2R_us,compute_us,"
                  "e2e_out_of_place_us,single_fft_relL2,shared_bytes");
        const bool shared = placement == "shared";
        switch (n) {
        case 64: choose<64>(precision, shared, batch, repeats, trials); break;
        case 128: choose<128>(precision, shared, batch, repeats, trials); break;
        case 256: choose<256>(precision, shared, batch, repeats, trials); break;
        case 512: choose<512>(precision, shared, batch, repeats, trials); break;
        case 1024: choose<1024>(precision, shared, batch, repeats, trials); break;
        case 2048: choose<2048>(precision, shared, batch, repeats, trials); break;
        default: choose<4096>(precision, shared, batch, repeats, trials); break;
        }
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ERROR: %s\n", e.what());
        return 1;
    }
}
