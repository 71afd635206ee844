// thff_fft -- quick-start check of the public API on MI355X:
//
//   thff_fft [batch] [device]
//
// Transforms `batch` example signals of N = 64 (batch a positive multiple of
// 16, default 16) forward, unscaled and out of place with
// ThunderFFT_global<float, 64, true> on HIP device `device` (default 0), and
// compares the result with hipFFT's single-precision C2C transform of the
// same input.
//
// Command-line contract of the reference's quick start (sample/fft1d/main.cu:
// arguments :170-193, example input :63-77, report :153-160): the same
// arguments, report lines and exit codes.  PASS needs finite values and both
// relative L2 and relative Linf <= 5e-3; a failed comparison, invalid
// arguments (checked before any HIP call), HIP/hipFFT errors and nonfinite
// values exit 1, the last three with "FAIL: <reason>" on stderr; --help or
// -h prints the usage and exits 0.
#include <thunderfft/thunderfft.cuh>

#include "cli_common.hpp"

#include <climits>
#include <complex>
#include <cstring>
#include <iomanip>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

using thff_cli::DeviceArray;
using thff_cli::ErrorStats;

constexpr int kLength = 64;
constexpr int kBatchGranule = 16;  // the example accepts whole 16-signal groups
constexpr double kGate = 5e-3;

struct Request {
    int batch = kBatchGranule;
    int device = 0;
};

const char* const kUsage =
    " [batch] [device]\n"
    "  batch   Positive multiple of 16 (default: 16).\n"
    "  device  Nonnegative HIP device ordinal (default: 0).\n"
    "Checks an unscaled, out-of-place, complex float forward FFT (N=64) against hipFFT.\n"
    "PASS requires finite outputs and relative L2/Linf <= 5e-3 for this example input.\n";

int nonnegative(const char* text, const char* what) {
    int value = 0;
    if (!thff_cli::parse_decimal(text, 0, INT_MAX, value) || text[0] == '+')
        throw std::invalid_argument(std::string(what) +
                                    " must be a nonnegative integer in int range");
    return value;
}

// Positional arguments -> request; every rule is checked before any HIP call.
Request read_request(int argc, char** argv) {
    if (argc > 3) throw std::invalid_argument("too many arguments");
    Request r;
    if (argc >= 2) r.batch = nonnegative(argv[1], "batch");
    if (argc >= 3) r.device = nonnegative(argv[2], "device");
    if (r.batch == 0 || r.batch % kBatchGranule != 0)
        throw std::invalid_argument("batch must be a positive multiple of 16");
    return r;
}

// Signal b: a tone of amplitude 0.5 + 0.1 (b mod 8) on bin 1 + (b mod 13)
// plus a tone of amplitude 0.1 on bin 7, evaluated in double and stored as
// float (the reference's example input).
std::vector<float2> example_signals(int batch) {
    std::vector<float2> signals;
    signals.reserve(static_cast<size_t>(batch) * kLength);
    for (int b = 0; b < batch; ++b) {
        const double amplitude = 0.5 + 0.1 * (b % 8);
        const int bin = 1 + b % 13;
        for (int n = 0; n < kLength; ++n) {
            const double theta = 2.0 * M_PI * n / kLength;
            const std::complex<double> v =
                std::polar(amplitude, bin * theta) + std::polar(0.1, 7.0 * theta);
            signals.push_back(make_float2(static_cast<float>(v.real()),
                                          static_cast<float>(v.imag())));
        }
    }
    return signals;
}

// Makes the twiddle table live for the scope and releases it on every exit.
struct LiveTable {
    LiveTable() { thunderfft::ThunderFFTInitialize<float>(kLength); }
    ~LiveTable() {
        try {
            thunderfft::ThunderFFTFinalize<float>();
        } catch (...) {
        }
    }
};

// Both transforms of the example input; returns {ours, hipFFT's}.
std::pair<std::vector<float2>, std::vector<float2>> transform_both(const Request& r) {
    thff_cli::hip_check(hipSetDevice(r.device), "hipSetDevice");
    const std::vector<float2> input = example_signals(r.batch);
    DeviceArray<float2> in(input.size(), "hipMalloc(input)");
    DeviceArray<float2> ours(input.size(), "hipMalloc(output)");
    DeviceArray<float2> theirs(input.size(), "hipMalloc(reference)");
    in.upload(input, "hipMemcpy(input)");
    {
        const LiveTable table;
        // synchronous: returns once the transform has finished, throws on failure
        thunderfft::ThunderFFT_global<float, kLength, true>(in.get(), ours.get(), r.batch);
    }
    const thff_cli::FftPlan plan(kLength, HIPFFT_C2C, r.batch);
    thff_cli::fft_check(hipfftExecC2C(plan.get(), reinterpret_cast<hipfftComplex*>(in.get()),
                                      reinterpret_cast<hipfftComplex*>(theirs.get()),
                                      HIPFFT_FORWARD),
                        "hipfftExecC2C");
    thff_cli::hip_check(hipDeviceSynchronize(), "hipFFT synchronization");
    return {ours.download("hipMemcpy(output)"), theirs.download("hipMemcpy(reference)")};
}

ErrorStats compare(const std::vector<float2>& ours, const std::vector<float2>& theirs) {
    ErrorStats stats, reference_finite;
    for (size_t i = 0; i < ours.size(); ++i) {
        stats.add(ours[i].x, ours[i].y, theirs[i].x, theirs[i].y);
        reference_finite.add(theirs[i].x, theirs[i].y, 0, 0);
    }
    if (stats.nonfinite || reference_finite.nonfinite)
        throw std::runtime_error("nonfinite output (" + std::to_string(stats.nonfinite) +
                                 " ThunderFFT, " + std::to_string(reference_finite.nonfinite) +
                                 " hipFFT values)");
    return stats;
}

bool report(const Request& r, const ErrorStats& stats) {
    const double l2 = stats.rel_l2(), linf = stats.rel_linf();
    const bool pass = std::isfinite(l2) && std::isfinite(linf) && l2 <= kGate && linf <= kGate;
    std::cout << "ThunderFFT vs hipFFT: float2, N=" << kLength << ", forward (unscaled), batch="
              << r.batch << ", device=" << r.device << '\n'
              << std::scientific << std::setprecision(6)
              << "Relative L2:   " << l2 << '\n'
              << "Relative Linf: " << linf << '\n'
              << "Tolerance:     " << kGate << " (this example input)\n"
              << (pass ? "PASS" : "FAIL") << '\n';
    return pass;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc == 2 && (!std::strcmp(argv[1], "--help") || !std::strcmp(argv[1], "-h"))) {
        std::cout << "Usage: " << argv[0] << kUsage;
        return 0;
    }
    try {
        const Request request = read_request(argc, argv);
        const auto [ours, theirs] = transform_both(request);
        return report(request, compare(ours, theirs)) ? 0 : 1;
    } catch (const std::exception& e) {
        std::cerr << "FAIL: " << e.what() << '\n';
        return 1;
    }
}
