// thff_validate -- the correctness matrix of the reference's validation
// program (sample/validation/fft_validation.cu) on MI355X:
//
//   thff_validate [--device N] [--batch N] [--csv PATH] [--quick] [--host-only]
//
// * --host-only: the 18 host API checks (fft_validation.cu:320-352), decided
//   before any HIP call, so they pass on a machine without a GPU.
// * Otherwise, for T in {float, half}, N in {64, ..., 4096}, both directions
//   and the four input kinds (Gaussian RMS 1, offset impulse, complex tone,
//   constant; fft_validation.cu:130-163): the "direct" path (a kernel built on
//   the device-side API, <thunderfft/thunderfft_device.hpp>, with 64 LDS
//   sentinels after its workspace) and the "public" path (ThunderFFT_global)
//   at --batch (default 64; --quick: 16, Gaussian only), plus public tail
//   batches {1, BPB-1, BPB+1}; then Finalize, re-Initialize(64) and one more
//   N=64 pair.  The reference is hipFFT Z2Z (fp64) of the values the storage
//   type actually represents; outputs are NaN-prefilled and followed by 16
//   sentinels.  Pass: finite, relative L2 <= 5e-3, sentinels unchanged.
// * One CSV line per case on stdout (and --csv PATH), with the reference's
//   columns.  Exit codes: 0 pass, 1 numerical/guard failure, 2 usage or
//   HIP/hipFFT error.
#include <hipfft/hipfft.h>
#include <thunderfft/thunderfft.cuh>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr double kGate = 5e-3;               // fft_validation.cu:26
constexpr int kOutGuard = 16;                // fft_validation.cu:25
constexpr float kOutGuardRe = -271.f, kOutGuardIm = 137.f;
constexpr int kLdsGuard = 64;                // fft_validation.cu:24
constexpr float kLdsGuardRe = 299.f, kLdsGuardIm = -299.f;
constexpr const char* kKindNames[4] = {"gaussian_rms1", "offset_impulse", "complex_tone",
                                       "constant"};

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
void fft_ok(hipfftResult e, const char* what) {
    if (e != HIPFFT_SUCCESS) throw std::runtime_error(std::string(what) + ": hipFFT error " +
                                                      std::to_string(static_cast<int>(e)));
}

template <class V>
struct Device {
    V* p = nullptr;
    explicit Device(size_t count) { hip_ok(hipMalloc(&p, count * sizeof(V)), "hipMalloc"); }
    ~Device() { (void)hipFree(p); }
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
};

template <class T>
__host__ __device__ vec2_t<T> store_as(float re, float im) {
    if constexpr (std::is_same_v<T, float>)
        return make_float2(re, im);
    else
        return __floats2half2_rn(re, im);
}
template <class T>
__host__ __device__ float2 load_as(vec2_t<T> v) {
    if constexpr (std::is_same_v<T, float>)
        return v;
    else
        return __half22float2(v);
}

// The four input kinds, each signal b of n values.
std::vector<float2> kind_input(int n, int batch, int kind) {
    std::vector<float2> x(static_cast<size_t>(n) * batch, make_float2(0.f, 0.f));
    std::mt19937 random(1234 + n);
    std::normal_distribution<float> normal(0.f, 1.f);
    const double tau = 6.283185307179586476925286766559;
    for (int b = 0; b < batch; ++b) {
        float2* s = x.data() + static_cast<size_t>(b) * n;
        switch (kind) {
        case 0: {  // complex Gaussian scaled to RMS 1
            double energy = 0;
            for (int i = 0; i < n; ++i) {
                const float re = normal(random);
                const float im = normal(random);
                s[i] = make_float2(re, im);
                energy += double(re) * re + double(im) * im;
            }
            const double scale = std::sqrt(n / energy);
            for (int i = 0; i < n; ++i) s[i] = make_float2(s[i].x * scale, s[i].y * scale);
            break;
        }
        case 1:  // one nonzero sample, position varying with b
            s[(13 * b + 7) % n] = make_float2(.75f, .25f);
            break;
        case 2: {  // complex exponential, frequency and phase varying with b
            const int f = 1 + (7 * b) % (n - 1);
            for (int i = 0; i < n; ++i) {
                const double ph = tau * f * i / n + .13 * b;
                s[i] = make_float2(.5 * std::cos(ph), .5 * std::sin(ph));
            }
            break;
        }
        default:
            for (int i = 0; i < n; ++i) s[i] = make_float2(.25f, -.125f);
        }
    }
    return x;
}

// The direct path: a kernel built on the device-side API.  Partial last
// block: missing transforms are zero-filled and not stored.
template <class T, int N, bool FWD>
__global__ __launch_bounds__(256) void direct_core(const vec2_t<T>* in, vec2_t<T>* out, int batch,
                                                   const float2* tw, int* lds_guard_changes) {
    constexpr int BPB = thunderfft::batch_per_block<N>;
    using L = thunderfft::layout_t<N, BPB, 1, N + thunderfft::pad_h(N), 16, 1, false>;
    constexpr int kStage = (L::at(N - 1, BPB - 1) + 1) * static_cast<int>(sizeof(vec2_t<T>));
    constexpr int kWork = thunderfft::workspace_bytes<N, BPB>;
    constexpr int kBytes = kStage > kWork ? kStage : kWork;
    __shared__ __align__(16) unsigned char raw[kBytes + kLdsGuard * sizeof(float2)];
    auto* stage = reinterpret_cast<vec2_t<T>*>(raw);
    auto* guard = reinterpret_cast<float2*>(raw + kBytes);
    const int tid = threadIdx.x;
    if (tid < kLdsGuard) guard[tid] = make_float2(kLdsGuardRe, kLdsGuardIm);
    const long long first = static_cast<long long>(blockIdx.x) * BPB;
    const int valid = batch - first < BPB ? static_cast<int>(batch - first) : BPB;
    for (int e = tid; e < N * BPB; e += 256) {
        const vec2_t<T> zero = store_as<T>(0.f, 0.f);
        stage[L::at(e % N, e / N)] = e / N < valid ? in[first * N + e] : zero;
    }
    __syncthreads();
    vec2_t<T> reg[thunderfft::elements_per_thread];
    thunderfft::ThunderFFT_smem2reg<T, L>(reg, stage);
    __syncthreads();
    thunderfft::ThunderFFT_kernel_reg<T, N, BPB, FWD>(reg, tw, raw);
    __syncthreads();
    thunderfft::ThunderFFT_reg2smem<T, L>(stage, reg);
    __syncthreads();
    for (int e = tid; e < N * valid; e += 256) out[first * N + e] = stage[L::at(e % N, e / N)];
    if (tid < kLdsGuard) {
        const float2 g = guard[tid];
        if (g.x != kLdsGuardRe || g.y != kLdsGuardIm) atomicAdd(lds_guard_changes, 1);
    }
}

struct Report {
    std::ofstream file;
    int cases = 0, failures = 0;
    explicit Report(const std::string& path) {
        if (!path.empty()) {
            file.open(path);
            if (!file) throw std::runtime_error("Cannot open CSV output: " + path);
        }
        line("path,precision,N,direction,input,batch,relative_l2,max_abs,relative_linf,"
             "nonfinite_outputs,shared_guard_changed_max,output_guard_changed,pass");
    }
    void line(const std::string& s) {
        std::cout << s << '\n' << std::flush;
        if (file.is_open()) file << s << '\n' << std::flush;
    }
};

template <class T, int N, bool FWD>
void run_case(Report& rep, bool direct, int batch, int kind) {
    const size_t count = static_cast<size_t>(N) * batch;
    // input as the storage type holds it, and its exact fp64 value
    const std::vector<float2> base = kind_input(N, batch, kind);
    std::vector<vec2_t<T>> x(count);
    std::vector<double2> ref(count);
    for (size_t i = 0; i < count; ++i) {
        x[i] = store_as<T>(base[i].x, base[i].y);
        const float2 r = load_as<T>(x[i]);
        ref[i] = make_double2(r.x, r.y);
    }
    Device<vec2_t<T>> d_in(count), d_out(count + kOutGuard);
    Device<double2> d_ref(count);
    Device<int> d_guard(1);
    hip_ok(hipMemcpy(d_in.p, x.data(), count * sizeof(vec2_t<T>), hipMemcpyHostToDevice), "copy in");
    std::vector<vec2_t<T>> y(count + kOutGuard, store_as<T>(NAN, NAN));
    for (int g = 0; g < kOutGuard; ++g) y[count + g] = store_as<T>(kOutGuardRe, kOutGuardIm);
    hip_ok(hipMemcpy(d_out.p, y.data(), y.size() * sizeof(vec2_t<T>), hipMemcpyHostToDevice), "prefill");
    hip_ok(hipMemset(d_guard.p, 0, sizeof(int)), "guard reset");

    // reference: fp64 Z2Z, unnormalized both ways
    hip_ok(hipMemcpy(d_ref.p, ref.data(), count * sizeof(double2), hipMemcpyHostToDevice), "copy ref");
    hipfftHandle plan;
    fft_ok(hipfftPlan1d(&plan, N, HIPFFT_Z2Z, batch), "hipfftPlan1d");
    const hipfftResult fr = hipfftExecZ2Z(plan, reinterpret_cast<hipfftDoubleComplex*>(d_ref.p),
                                          reinterpret_cast<hipfftDoubleComplex*>(d_ref.p),
                                          FWD ? HIPFFT_FORWARD : HIPFFT_BACKWARD);
    (void)hipfftDestroy(plan);
    fft_ok(fr, "hipfftExecZ2Z");

    if (direct) {
        constexpr int BPB = thunderfft::batch_per_block<N>;
        direct_core<T, N, FWD><<<(batch + BPB - 1) / BPB, 256>>>(
            d_in.p, d_out.p, batch, thunderfft::ThunderFFT_twiddle_table<T>(), d_guard.p);
        hip_ok(hipGetLastError(), "direct_core launch");
        hip_ok(hipDeviceSynchronize(), "direct_core");
    } else {
        thunderfft::ThunderFFT_global<T, N, FWD>(d_in.p, d_out.p, batch);
    }
    hip_ok(hipMemcpy(y.data(), d_out.p, y.size() * sizeof(vec2_t<T>), hipMemcpyDeviceToHost), "copy out");
    hip_ok(hipMemcpy(ref.data(), d_ref.p, count * sizeof(double2), hipMemcpyDeviceToHost), "copy ref out");
    int lds_guard = 0;
    hip_ok(hipMemcpy(&lds_guard, d_guard.p, sizeof(int), hipMemcpyDeviceToHost), "copy guard");

    double err2 = 0, ref2 = 0, max_abs = 0, ref_max = 0;
    long nonfinite = 0;
    for (size_t i = 0; i < count; ++i) {
        const float2 v = load_as<T>(y[i]);
        if (!std::isfinite(v.x) || !std::isfinite(v.y)) ++nonfinite;
        const double dx = v.x - ref[i].x, dy = v.y - ref[i].y;
        err2 += dx * dx + dy * dy;
        ref2 += ref[i].x * ref[i].x + ref[i].y * ref[i].y;
        max_abs = std::fmax(max_abs, std::hypot(dx, dy));
        ref_max = std::fmax(ref_max, std::hypot(ref[i].x, ref[i].y));
    }
    int out_guard = 0;
    for (int g = 0; g < kOutGuard; ++g) {
        const float2 v = load_as<T>(y[count + g]);
        out_guard += v.x != kOutGuardRe || v.y != kOutGuardIm;
    }
    const double rel_l2 = ref2 > 0 ? std::sqrt(err2 / ref2) : std::sqrt(err2);
    const double rel_linf = ref_max > 0 ? max_abs / ref_max : max_abs;
    const bool pass = nonfinite == 0 && std::isfinite(rel_l2) && rel_l2 <= kGate && lds_guard == 0 &&
                      out_guard == 0;
    ++rep.cases;
    rep.failures += pass ? 0 : 1;
    std::ostringstream s;
    s.precision(6);
    s << std::scientific << (direct ? "direct" : "public") << ','
      << (std::is_same_v<T, float> ? "fp32" : "fp16") << ',' << N << ','
      << (FWD ? "forward" : "inverse") << ',' << kKindNames[kind] << ',' << batch << ',' << rel_l2
      << ',' << max_abs << ',' << rel_linf << ',' << nonfinite << ',' << lds_guard << ','
      << out_guard << ',' << (pass ? 1 : 0);
    rep.line(s.str());
}

struct Options {
    int device = 0, batch = 64;
    bool quick = false, host_only = false, batch_set = false;
    std::string csv;
};

template <class T, int N>
void run_size(Report& rep, const Options& o) {
    thunderfft::ThunderFFTInitialize<T>(N);
    constexpr int BPB = thunderfft::batch_per_block<N>;
    std::vector<int> tails = o.quick ? std::vector<int>{1} : std::vector<int>{1, BPB - 1, BPB + 1};
    for (int kind = 0; kind < (o.quick ? 1 : 4); ++kind) {
        run_case<T, N, true>(rep, true, o.batch, kind);
        run_case<T, N, false>(rep, true, o.batch, kind);
        run_case<T, N, true>(rep, false, o.batch, kind);
        run_case<T, N, false>(rep, false, o.batch, kind);
        int previous = -1;
        for (int b : tails) {
            if (b <= 0 || b == o.batch || b == previous) continue;
            previous = b;
            run_case<T, N, true>(rep, false, b, kind);
            run_case<T, N, false>(rep, false, b, kind);
        }
    }
    thunderfft::ThunderFFTFinalize<T>();
}

template <class T>
void run_type(Report& rep, const Options& o) {
    run_size<T, 64>(rep, o);
    run_size<T, 128>(rep, o);
    run_size<T, 256>(rep, o);
    run_size<T, 512>(rep, o);
    run_size<T, 1024>(rep, o);
    run_size<T, 2048>(rep, o);
    run_size<T, 4096>(rep, o);
    // the cache must come back cleanly after teardown (fft_validation.cu:306-310)
    thunderfft::ThunderFFTInitialize<T>(64);
    run_case<T, 64, true>(rep, false, 1, 0);
    run_case<T, 64, false>(rep, false, 1, 0);
    thunderfft::ThunderFFTFinalize<T>();
}

// ---------------------------------------------------------------- host checks
int g_checks = 0;

template <class Operation>
void expect_invalid_argument(Operation operation, const char* description) {
    try {
        operation();
    } catch (const std::invalid_argument&) {
        ++g_checks;
        return;
    }
    throw std::runtime_error(std::string("Host API check did not reject ") + description);
}

template <class T>
void host_checks() {
    // Host pointers appear only in calls that must reject them for nullness
    // or aliasing; none of these calls may reach the device.
    vec2_t<T> value{};
    expect_invalid_argument([] { thunderfft::ThunderFFT_global<T, 64>(nullptr, nullptr, -1); },
                            "negative batch");
    expect_invalid_argument([&] { thunderfft::ThunderFFT_global<T, 64>(nullptr, &value, 1); },
                            "null input");
    expect_invalid_argument([&] { thunderfft::ThunderFFT_global<T, 64>(&value, nullptr, 1); },
                            "null output");
    expect_invalid_argument([&] { thunderfft::ThunderFFT_global<T, 64>(&value, &value, 1); },
                            "aliased input/output");
    thunderfft::ThunderFFT_global<T, 64>(nullptr, nullptr, 0);
    ++g_checks;
    for (int n : {-1, 0, 32, 8192})
        expect_invalid_argument([n] { thunderfft::ThunderFFTInitialize<T>(n); },
                                "unsupported initialization length");
}

int parse_int(const char* text, const char* what) {
    char* end = nullptr;
    const long v = std::strtol(text, &end, 10);
    if (!*text || *end || v < -2147483647L || v > 2147483647L)
        throw std::runtime_error(std::string("Invalid ") + what + ": " + text);
    return static_cast<int>(v);
}

void usage(const char* exe) {
    std::cout << "Usage: " << exe << " [--device N] [--batch N] [--csv PATH] [--quick] [--host-only]\n"
              << "All seven lengths, fp32/fp16, forward/inverse, direct (device API) and public\n"
              << "(ThunderFFT_global) paths against hipFFT Z2Z (fp64) of the represented input.\n"
              << "Default batch 64 (1..65536); --quick: batch 16, Gaussian input, public tail 1.\n"
              << "Pass: finite output, relative L2 <= 0.005, unchanged LDS and output sentinels.\n"
              << "--host-only: the 18 API argument checks, without any HIP call.\n"
              << "CSV goes to stdout; --csv also writes a file. Exit: 0 pass, 1 failure, 2 error.\n";
}

}  // namespace

int main(int argc, char** argv) {
    try {
        Options o;
        for (int i = 1; i < argc; ++i) {
            const std::string a = argv[i];
            if (a == "--help" || a == "-h") {
                usage(argv[0]);
                return 0;
            }
            if (a == "--quick") { o.quick = true; continue; }
            if (a == "--host-only") { o.host_only = true; continue; }
            if (a != "--device" && a != "--batch" && a != "--csv")
                throw std::runtime_error("Unknown option: " + a);
            if (++i >= argc) throw std::runtime_error("Missing value for " + a);
            if (a == "--device") {
                o.device = parse_int(argv[i], "device");
            } else if (a == "--batch") {
                o.batch = parse_int(argv[i], "batch");
                o.batch_set = true;
            } else {
                o.csv = argv[i];
            }
        }
        if (o.quick && !o.batch_set) o.batch = 16;
        if (o.device < 0) throw std::runtime_error("Device must be nonnegative");
        if (o.batch <= 0 || o.batch > 65536) throw std::runtime_error("Batch must be in 1..65536");
        if (o.host_only && !o.csv.empty())
            throw std::runtime_error("--csv requires GPU validation; omit it with --host-only");
        host_checks<float>();
        host_checks<half>();
        std::cerr << "Host API validation: " << g_checks << " checks passed before any HIP calls\n";
        if (g_checks != 18) return 2;
        if (o.host_only) return 0;
        hip_ok(hipSetDevice(o.device), "hipSetDevice");
        Report rep(o.csv);
        run_type<float>(rep, o);
        run_type<half>(rep, o);
        std::cerr << "Validation: " << rep.cases << " cases, " << rep.failures
                  << " failures; relative L2 limit " << kGate << '\n';
        return rep.failures == 0 ? 0 : 1;
    } catch (const std::exception& e) {
        std::cerr << "Validation error: " << e.what() << '\n';
        return 2;
    }
}
