// thff_fft -- the quick-start check of the reference's sample/fft1d/main.cu
// (`thff_fft`) on MI355X:
//
//   thff_fft [batch] [device]
//
// One unscaled, out-of-place, complex float forward transform of N=64 over
// `batch` signals (a positive multiple of 16, default 16) on HIP device
// `device` (default 0), through ThunderFFTInitialize<float>(64) and
// ThunderFFT_global<float, 64, true>, compared with hipFFT's single-precision
// C2C transform of the same input (the reference compares with cuFFT C2C).
//
// The input is the reference's deterministic one (main.cu:63-77): signal b
// holds a bin-aligned tone of frequency 1 + b % 13 and amplitude
// 0.5 + 0.1 * (b % 8), plus a tone of amplitude 0.1 at bin 7.
//
// Output and exit status follow main.cu:153-193: the configuration line,
// "Relative L2", "Relative Linf" and "Tolerance" in scientific notation,
// then PASS or FAIL.  PASS needs finite outputs and both relative errors
// <= 5e-3.  Invalid arguments, HIP/hipFFT errors, nonfinite values and a
// failed comparison all exit 1 ("FAIL: <reason>" on stderr for the first
// three); --help / -h prints the usage and exits 0.  Arguments are checked
// before any HIP call.
#include <hipfft/hipfft.h>
#include <thunderfft/thunderfft.cuh>

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <iomanip>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr int kN = 64;                // main.cu:21
constexpr int kSignalsPerTile = 16;   // main.cu:22: the batch granularity the sample accepts
constexpr double kGate = 5e-3;        // main.cu:24

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void fft_ok(hipfftResult e, const char* what) {
    if (e != HIPFFT_SUCCESS)
        throw std::runtime_error(std::string(what) + ": hipFFT status " +
                                 std::to_string(static_cast<int>(e)));
}

void usage(std::ostream& os, const char* prog) {
    os << "Usage: " << prog << " [batch] [device]\n"
       << "  batch   Positive multiple of 16 (default: 16).\n"
       << "  device  Nonnegative HIP device ordinal (default: 0).\n"
       << "Checks an unscaled, out-of-place, complex float forward FFT (N=64) against hipFFT.\n"
       << "PASS requires finite outputs and relative L2/Linf <= 5e-3 for this example input.\n";
}

int parse_count(const char* text, const char* name) {
    int v = 0;
    const char* end = text + std::strlen(text);
    const auto r = std::from_chars(text, end, v);
    if (r.ec != std::errc{} || r.ptr != end || v < 0)
        throw std::invalid_argument(std::string(name) + " must be a nonnegative integer in int range");
    return v;
}

// Signal b: a * e^{i f theta} + 0.1 * e^{i 7 theta}, theta = 2 pi n / N,
// f = 1 + b % 13, a = 0.5 + 0.1 * (b % 8); evaluated in double, stored as float.
std::vector<float2> tones(int batch) {
    std::vector<float2> x(static_cast<size_t>(batch) * kN);
    for (int b = 0; b < batch; ++b) {
        const double f = 1 + b % 13, a = 0.5 + 0.1 * (b % 8);
        for (int n = 0; n < kN; ++n) {
            const double theta = 2.0 * M_PI * n / kN;
            x[static_cast<size_t>(b) * kN + n] =
                make_float2(static_cast<float>(a * std::cos(f * theta) + 0.1 * std::cos(7.0 * theta)),
                            static_cast<float>(a * std::sin(f * theta) + 0.1 * std::sin(7.0 * theta)));
        }
    }
    return x;
}

// Owns every device resource so that an exception on any step releases them.
struct Session {
    float2* in = nullptr;
    float2* out = nullptr;
    float2* ref = nullptr;
    hipfftHandle plan = 0;
    bool plan_made = false;
    bool initialized = false;
    ~Session() {
        if (plan_made) (void)hipfftDestroy(plan);
        if (initialized) thunderfft::ThunderFFTFinalize<float>();
        if (ref) (void)hipFree(ref);
        if (out) (void)hipFree(out);
        if (in) (void)hipFree(in);
    }
};

bool run(int batch, int device) {
    hip_ok(hipSetDevice(device), "hipSetDevice");
    const size_t count = static_cast<size_t>(kN) * batch, bytes = count * sizeof(float2);
    const std::vector<float2> x = tones(batch);
    std::vector<float2> y(count), r(count);

    Session s;
    hip_ok(hipMalloc(&s.in, bytes), "hipMalloc(input)");
    hip_ok(hipMalloc(&s.out, bytes), "hipMalloc(output)");
    hip_ok(hipMalloc(&s.ref, bytes), "hipMalloc(reference)");
    hip_ok(hipMemcpy(s.in, x.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy(input)");

    s.initialized = true;
    thunderfft::ThunderFFTInitialize<float>(kN);
    hip_ok(hipGetLastError(), "ThunderFFTInitialize");
    hip_ok(hipDeviceSynchronize(), "ThunderFFTInitialize synchronization");

    thunderfft::ThunderFFT_global<float, kN, true>(s.in, s.out, batch, /*stream=*/0);
    hip_ok(hipGetLastError(), "ThunderFFT launch");
    hip_ok(hipDeviceSynchronize(), "ThunderFFT synchronization");

    fft_ok(hipfftPlan1d(&s.plan, kN, HIPFFT_C2C, batch), "hipfftPlan1d");
    s.plan_made = true;
    fft_ok(hipfftExecC2C(s.plan, reinterpret_cast<hipfftComplex*>(s.in),
                         reinterpret_cast<hipfftComplex*>(s.ref), HIPFFT_FORWARD),
           "hipfftExecC2C");
    hip_ok(hipGetLastError(), "hipFFT launch");
    hip_ok(hipDeviceSynchronize(), "hipFFT synchronization");
    hip_ok(hipMemcpy(y.data(), s.out, bytes, hipMemcpyDeviceToHost), "hipMemcpy(output)");
    hip_ok(hipMemcpy(r.data(), s.ref, bytes, hipMemcpyDeviceToHost), "hipMemcpy(reference)");

    double err2 = 0.0, ref2 = 0.0, err_max = 0.0, ref_max = 0.0;
    for (size_t i = 0; i < count; ++i) {
        if (!std::isfinite(y[i].x) || !std::isfinite(y[i].y) || !std::isfinite(r[i].x) ||
            !std::isfinite(r[i].y))
            throw std::runtime_error("nonfinite output at complex element " + std::to_string(i));
        const double e = std::hypot(double(y[i].x) - r[i].x, double(y[i].y) - r[i].y);
        const double m = std::hypot(double(r[i].x), double(r[i].y));
        err2 += e * e;
        ref2 += m * m;
        err_max = std::max(err_max, e);
        ref_max = std::max(ref_max, m);
    }
    const double l2 = ref2 > 0.0 ? std::sqrt(err2 / ref2) : std::sqrt(err2);
    const double linf = ref_max > 0.0 ? err_max / ref_max : err_max;
    const bool pass = std::isfinite(l2) && std::isfinite(linf) && l2 <= kGate && linf <= kGate;
    std::cout << "ThunderFFT vs hipFFT: float2, N=" << kN << ", forward (unscaled), batch=" << batch
              << ", device=" << device << '\n'
              << std::scientific << std::setprecision(6) << "Relative L2:   " << l2 << '\n'
              << "Relative Linf: " << linf << '\n'
              << "Tolerance:     " << kGate << " (this example input)\n"
              << (pass ? "PASS" : "FAIL") << '\n';
    return pass;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc == 2 && (std::strcmp(argv[1], "--help") == 0 || std::strcmp(argv[1], "-h") == 0)) {
        usage(std::cout, argv[0]);
        return EXIT_SUCCESS;
    }
    try {
        if (argc > 3) throw std::invalid_argument("too many arguments");
        const int batch = argc > 1 ? parse_count(argv[1], "batch") : kSignalsPerTile;
        const int device = argc > 2 ? parse_count(argv[2], "device") : 0;
        if (batch <= 0 || batch % kSignalsPerTile != 0)
            throw std::invalid_argument("batch must be a positive multiple of 16");
        if (static_cast<size_t>(batch) > std::numeric_limits<size_t>::max() / (kN * sizeof(float2)))
            throw std::invalid_argument("batch allocation size overflows size_t");
        return run(batch, device) ? EXIT_SUCCESS : EXIT_FAILURE;
    } catch (const std::exception& e) {
        std::cerr << "FAIL: " << e.what() << '\n';
        return EXIT_FAILURE;
    }
}
