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
#include <thunderfft/thunderfft.cuh>

#include "cli_common.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
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

using thff_cli::DeviceArray;
using thff_cli::hip_check;

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
    // output: NaN-prefilled, then kOutGuard sentinels that must survive
    std::vector<vec2_t<T>> y(count + kOutGuard, store_as<T>(NAN, NAN));
    for (int g = 0; g < kOutGuard; ++g) y[count + g] = store_as<T>(kOutGuardRe, kOutGuardIm);
    DeviceArray<vec2_t<T>> d_in(count), d_out(y.size());
    DeviceArray<double2> d_ref(count);
    DeviceArray<int> d_guard(1);
    d_in.upload(x, "copy in");
    d_out.upload(y, "prefill");
    d_ref.upload(ref, "copy ref");
    d_guard.upload(std::vector<int>{0}, "guard reset");

    // reference: fp64 Z2Z in place, unnormalized both ways
    {
        const thff_cli::FftPlan plan(N, HIPFFT_Z2Z, batch);
        auto* z = reinterpret_cast<hipfftDoubleComplex*>(d_ref.get());
        thff_cli::fft_check(hipfftExecZ2Z(plan.get(), z, z, FWD ? HIPFFT_FORWARD : HIPFFT_BACKWARD),
                            "hipfftExecZ2Z");
    }
    if (direct) {
        constexpr int BPB = thunderfft::batch_per_block<N>;
        direct_core<T, N, FWD><<<(batch + BPB - 1) / BPB, 256>>>(
            d_in.get(), d_out.get(), batch, thunderfft::ThunderFFT_twiddle_table<T>(),
            d_guard.get());
        hip_check(hipGetLastError(), "direct_core launch");
        hip_check(hipDeviceSynchronize(), "direct_core");
    } else {
        thunderfft::ThunderFFT_global<T, N, FWD>(d_in.get(), d_out.get(), batch);
    }
    y = d_out.download("copy out");
    ref = d_ref.download("copy ref out");
    const int lds_guard = d_guard.download("copy guard")[0];

    thff_cli::ErrorStats stats;
    for (size_t i = 0; i < count; ++i) {
        const float2 v = load_as<T>(y[i]);
        stats.add(v.x, v.y, ref[i].x, ref[i].y);
    }
    int out_guard = 0;
    for (int g = 0; g < kOutGuard; ++g) {
        const float2 v = load_as<T>(y[count + g]);
        out_guard += v.x != kOutGuardRe || v.y != kOutGuardIm;
    }
    const double rel_l2 = stats.rel_l2();
    const bool pass = stats.nonfinite == 0 && std::isfinite(rel_l2) && rel_l2 <= kGate &&
                      lds_guard == 0 && out_guard == 0;
    ++rep.cases;
    rep.failures += pass ? 0 : 1;
    std::ostringstream s;
    s.precision(6);
    s << std::scientific << (direct ? "direct" : "public") << ','
      << (std::is_same_v<T, float> ? "fp32" : "fp16") << ',' << N << ','
      << (FWD ? "forward" : "inverse") << ',' << kKindNames[kind] << ',' << batch << ',' << rel_l2
      << ',' << stats.max_err << ',' << stats.rel_linf() << ',' << stats.nonfinite << ','
      << lds_guard << ',' << out_guard << ',' << (pass ? 1 : 0);
    rep.line(s.str());
}

struct Options {
    int device = 0, batch = 64;
    bool quick = false, host_only = false, batch_set = false, help = false;
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
// The public API's argument contract (fft_validation.cu:331-352): each entry
// is a call and whether it must be rejected with std::invalid_argument (or
// return normally).  Every one is decided before the library makes a HIP
// call, so the list runs on a machine without a GPU; the host addresses used
// appear only where they must be rejected.
struct HostCheck {
    std::string what;
    bool rejected;
    std::function<void()> call;
};

template <class T>
std::vector<HostCheck> host_checks() {
    static vec2_t<T> host_value{};
    vec2_t<T>* const p = &host_value;
    const std::string t = std::is_same_v<T, float> ? "float: " : "half: ";
    std::vector<HostCheck> list = {
        {t + "negative batch", true,
         [] { thunderfft::ThunderFFT_global<T, 64>(nullptr, nullptr, -1); }},
        {t + "null input", true, [p] { thunderfft::ThunderFFT_global<T, 64>(nullptr, p, 1); }},
        {t + "null output", true, [p] { thunderfft::ThunderFFT_global<T, 64>(p, nullptr, 1); }},
        {t + "aliased input/output", true, [p] { thunderfft::ThunderFFT_global<T, 64>(p, p, 1); }},
        {t + "zero batch returns before touching pointers", false,
         [] { thunderfft::ThunderFFT_global<T, 64>(nullptr, nullptr, 0); }},
    };
    for (int n : {-1, 0, 32, 8192})
        list.push_back({t + "Initialize(" + std::to_string(n) + ")", true,
                        [n] { thunderfft::ThunderFFTInitialize<T>(n); }});
    return list;
}

int run_host_checks() {
    std::vector<HostCheck> all = host_checks<float>();
    for (HostCheck& c : host_checks<half>()) all.push_back(std::move(c));
    int passed = 0;
    for (const HostCheck& c : all) {
        bool rejected = false;
        try {
            c.call();
        } catch (const std::invalid_argument&) {
            rejected = true;
        }
        if (rejected != c.rejected)
            throw std::runtime_error(std::string("Host API check ") +
                                     (c.rejected ? "did not reject " : "rejected ") + c.what);
        ++passed;
    }
    return passed;
}

// ---------------------------------------------------------------- options
int int_option(const std::string& text, const char* what) {
    int v = 0;
    if (!thff_cli::parse_decimal(text, INT32_MIN + 1LL, INT32_MAX, v))
        throw std::runtime_error(std::string("Invalid ") + what + ": " + text);
    return v;
}

Options read_options(int argc, char** argv) {
    Options o;
    const auto flag = [](bool& b) { return [&b](const std::string&) { b = true; }; };
    thff_cli::parse_options(
        argc, argv,
        {{"--help", false, flag(o.help)},
         {"-h", false, flag(o.help)},
         {"--quick", false, flag(o.quick)},
         {"--host-only", false, flag(o.host_only)},
         {"--device", true, [&o](const std::string& v) { o.device = int_option(v, "device"); }},
         {"--batch", true,
          [&o](const std::string& v) {
              o.batch = int_option(v, "batch");
              o.batch_set = true;
          }},
         {"--csv", true, [&o](const std::string& v) { o.csv = v; }}});
    if (o.help) return o;
    if (o.quick && !o.batch_set) o.batch = 16;
    if (o.device < 0) throw std::runtime_error("Device must be nonnegative");
    if (o.batch <= 0 || o.batch > 65536) throw std::runtime_error("Batch must be in 1..65536");
    if (o.host_only && !o.csv.empty())
        throw std::runtime_error("--csv requires GPU validation; omit it with --host-only");
    return o;
}

const char* const kUsage =
    " [--device N] [--batch N] [--csv PATH] [--quick] [--host-only]\n"
    "All seven lengths, fp32/fp16, forward/inverse, direct (device API) and public\n"
    "(ThunderFFT_global) paths against hipFFT Z2Z (fp64) of the represented input.\n"
    "Default batch 64 (1..65536); --quick: batch 16, Gaussian input, public tail 1.\n"
    "Pass: finite output, relative L2 <= 0.005, unchanged LDS and output sentinels.\n"
    "--host-only: the 18 API argument checks, without any HIP call.\n"
    "CSV goes to stdout; --csv also writes a file. Exit: 0 pass, 1 failure, 2 error.\n";

}  // namespace

int main(int argc, char** argv) {
    try {
        const Options o = read_options(argc, argv);
        if (o.help) {
            std::cout << "Usage: " << argv[0] << kUsage;
            return 0;
        }
        const int checks = run_host_checks();
        std::cerr << "Host API validation: " << checks << " checks passed before any HIP calls\n";
        if (o.host_only) return 0;
        hip_check(hipSetDevice(o.device), "hipSetDevice");
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
