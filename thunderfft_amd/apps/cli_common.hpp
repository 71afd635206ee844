// cli_common.hpp -- pieces shared by the command-line programs in this
// directory: HIP/hipFFT status checks that throw, owning device arrays and
// FFT plans, the relative-error accumulator every validation reports, and a
// small table-driven option parser.
#pragma once

#include <hip/hip_runtime.h>
#include <hipfft/hipfft.h>

#include <cmath>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

namespace thff_cli {

inline void hip_check(hipError_t status, const std::string& context) {
    if (status != hipSuccess)
        throw std::runtime_error(context + ": " + hipGetErrorString(status));
}

inline void fft_check(hipfftResult status, const std::string& context) {
    if (status != HIPFFT_SUCCESS)
        throw std::runtime_error(context + ": hipFFT status " +
                                 std::to_string(static_cast<int>(status)));
}

// An owning device allocation of `count` values of V.
template <class V>
class DeviceArray {
public:
    explicit DeviceArray(size_t count, const char* what = "hipMalloc") : count_(count) {
        hip_check(hipMalloc(reinterpret_cast<void**>(&ptr_), count * sizeof(V)), what);
    }
    ~DeviceArray() {
        if (ptr_) (void)hipFree(ptr_);
    }
    DeviceArray(const DeviceArray&) = delete;
    DeviceArray& operator=(const DeviceArray&) = delete;

    V* get() const { return ptr_; }
    size_t bytes() const { return count_ * sizeof(V); }
    void upload(const std::vector<V>& host, const char* what = "hipMemcpy (to device)") {
        hip_check(hipMemcpy(ptr_, host.data(), host.size() * sizeof(V), hipMemcpyHostToDevice),
                  what);
    }
    std::vector<V> download(const char* what = "hipMemcpy (to host)") const {
        std::vector<V> host(count_);
        hip_check(hipMemcpy(host.data(), ptr_, bytes(), hipMemcpyDeviceToHost), what);
        return host;
    }

private:
    V* ptr_ = nullptr;
    size_t count_ = 0;
};

// A batched 1-D hipFFT plan, destroyed with its owner.
class FftPlan {
public:
    FftPlan(int n, hipfftType type, int batch) {
        fft_check(hipfftPlan1d(&plan_, n, type, batch), "hipfftPlan1d");
    }
    ~FftPlan() { (void)hipfftDestroy(plan_); }
    FftPlan(const FftPlan&) = delete;
    FftPlan& operator=(const FftPlan&) = delete;
    hipfftHandle get() const { return plan_; }

private:
    hipfftHandle plan_{};
};

// Accumulates |got - want| over complex values, in double: relative L2
// (sqrt(sum err^2 / sum |want|^2)), the largest absolute error, relative
// Linf (largest error / largest |want|) and the count of nonfinite `got`
// values.  With an all-zero reference the relative figures fall back to the
// absolute ones.
struct ErrorStats {
    double err2 = 0, ref2 = 0, max_err = 0, max_ref = 0;
    long long nonfinite = 0;

    void add(double got_re, double got_im, double want_re, double want_im) {
        if (!std::isfinite(got_re) || !std::isfinite(got_im)) ++nonfinite;
        const double e = std::hypot(got_re - want_re, got_im - want_im);
        const double m = std::hypot(want_re, want_im);
        err2 += e * e;
        ref2 += m * m;
        if (e > max_err) max_err = e;
        if (m > max_ref) max_ref = m;
    }
    double rel_l2() const { return ref2 > 0 ? std::sqrt(err2 / ref2) : std::sqrt(err2); }
    double rel_linf() const { return max_ref > 0 ? max_err / max_ref : max_err; }
};

// Table-driven option parsing: each option is a name, whether it takes a
// value, and what to do with it.  parse() walks argv once; an unknown option
// or a missing value throws std::runtime_error.
struct Option {
    std::string name;
    bool takes_value;
    std::function<void(const std::string&)> apply;
};

inline void parse_options(int argc, char** argv, const std::vector<Option>& table) {
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        const Option* match = nullptr;
        for (const Option& o : table)
            if (o.name == arg) match = &o;
        if (!match) throw std::runtime_error("Unknown option: " + arg);
        if (!match->takes_value) {
            match->apply(arg);
            continue;
        }
        if (i + 1 >= argc) throw std::runtime_error("Missing value for " + arg);
        match->apply(argv[++i]);
    }
}

// A decimal int that fills the whole text, or nothing.
inline bool parse_decimal(const std::string& text, long long lo, long long hi, int& out) {
    if (text.empty()) return false;
    size_t i = text[0] == '-' || text[0] == '+' ? 1 : 0;
    if (i == text.size()) return false;
    long long v = 0;
    for (; i < text.size(); ++i) {
        if (text[i] < '0' || text[i] > '9') return false;
        v = v * 10 + (text[i] - '0');
        if (v > (1LL << 40)) return false;
    }
    if (text[0] == '-') v = -v;
    if (v < lo || v > hi) return false;
    out = static_cast<int>(v);
    return true;
}

}  // namespace thff_cli
