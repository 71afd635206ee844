// thff_validate_cache -- twiddle-cache lifecycle and device ownership on
// every visible GPU, with no kernel launched.
//
// Command-line contract of the reference's cache check
// (sample/validation/cache_validation.cu): no arguments (--help / -h prints
// the usage and exits 0, anything else exits 2), one CSV row
// "precision,device,stage,N,pointer,pass" per checked stage with the same
// stage names, exit 0 when every check holds and 2 on the first failure.
// The float precision is labelled "fp32": this build's float path computes in
// fp32 (the reference labels its TF32 path "tf32").
//
// The checks are scripted: a lifecycle is a table of steps, each an action
// on the current device's cache (Initialize(N), Finalize, or none) and the
// state it must leave -- live with length N, or released -- optionally with
// the table pointer an earlier stage recorded.  One runner executes every
// script for both precisions.  A live table (thff_twiddle_info) must be
// device memory of the current device, have the current length, and hold
// W[0] = 1 + 0i exactly and W[1] = (cos, sin)(2 pi / N) within 1e-6; the
// table is fp32 for both precisions here.
#include <thunderfft/thunderfft.hpp>

#include "cli_common.hpp"

#include <cmath>
#include <cstring>
#include <iostream>
#include <map>
#include <stdexcept>
#include <string>
#include <tuple>
#include <type_traits>
#include <utility>
#include <vector>

namespace {

enum class Action { kInitialize, kFinalize, kNone };
enum class Expect { kLive, kReleased };

struct Step {
    const char* stage;  // CSV stage name; null: checked but not reported
    Action action;
    int n;              // the length to initialize and then expect live
    Expect expect;
    const char* keeps;  // earlier stage whose table pointer must be kept
};

// One device on its own: cache hit, length replacement, double Finalize and
// re-initialization (cache_validation.cu:105-121).
const std::vector<Step> kSingleDevice = {
    {"initialize", Action::kInitialize, 64, Expect::kLive, nullptr},
    {"same_length_cache_hit", Action::kInitialize, 64, Expect::kLive, "initialize"},
    {"replace_length", Action::kInitialize, 128, Expect::kLive, nullptr},
    {"finalize", Action::kFinalize, 0, Expect::kReleased, nullptr},
    {"repeated_finalize", Action::kFinalize, 0, Expect::kReleased, nullptr},
    {"reinitialize_after_finalize", Action::kInitialize, 64, Expect::kLive, nullptr},
    {"final_cleanup", Action::kFinalize, 0, Expect::kReleased, nullptr},
};

// Every device live at once with its own length; the three phases run over
// all devices in turn (cache_validation.cu:123-148).
std::vector<std::vector<Step>> cross_device_phases(int n) {
    return {
        {{"cross_device_initialize", Action::kInitialize, n, Expect::kLive, nullptr}},
        {{"return_to_device", Action::kNone, n, Expect::kLive, "cross_device_initialize"},
         {nullptr, Action::kInitialize, n, Expect::kLive, "cross_device_initialize"}},
        {{"cross_device_cleanup", Action::kFinalize, 0, Expect::kReleased, nullptr}},
    };
}

class Audit {
public:
    int checks() const { return checks_; }

    template <class T>
    void run(int device, const Step& step) {
        thff_cli::hip_check(hipSetDevice(device), "hipSetDevice");
        if (step.action == Action::kInitialize) thunderfft::ThunderFFTInitialize<T>(step.n);
        if (step.action == Action::kFinalize) thunderfft::ThunderFFTFinalize<T>();
        const void* table = nullptr;
        int n = 0;
        thunderfft::detail::check(
            thff_twiddle_info(thunderfft::detail::precision_code<T>(), &table, &n));
        if (step.expect == Expect::kLive)
            verify_live(device, step.n, table, n);
        else
            verify_released(table, n);
        if (step.keeps) {
            const auto earlier = pointers_.find(std::make_tuple(device, label<T>(), step.keeps));
            expect(earlier != pointers_.end() && earlier->second == table,
                   std::string(step.stage ? step.stage : "re-initialization") +
                       " must keep the allocation recorded at " + step.keeps);
        }
        if (!step.stage) return;
        pointers_[std::make_tuple(device, label<T>(), step.stage)] = table;
        std::cout << label<T>() << ',' << device << ',' << step.stage << ',' << n << ',';
        if (table)
            std::cout << table;
        else
            std::cout << '0';
        std::cout << ",1\n";
    }

    template <class T>
    void run_type(const std::vector<int>& devices) {
        for (int device : devices)
            for (const Step& step : kSingleDevice) run<T>(device, step);
        for (size_t phase = 0; phase < 3; ++phase)
            for (size_t i = 0; i < devices.size(); ++i) {
                const std::vector<std::vector<Step>> script = cross_device_phases(i % 2 ? 128 : 64);
                for (const Step& step : script[phase]) run<T>(devices[i], step);
            }
    }

private:
    template <class T>
    static const char* label() {
        return std::is_same_v<T, half> ? "fp16" : "fp32";
    }

    void expect(bool holds, const std::string& what) {
        if (!holds) throw std::runtime_error("Cache check failed: " + what);
        ++checks_;
    }

    void verify_live(int device, int n_expected, const void* table, int n) {
        expect(table != nullptr, "a live table pointer must be non-null");
        expect(n == n_expected, "the table length must match the last initialization");
        hipPointerAttribute_t attributes{};
        thff_cli::hip_check(hipPointerGetAttributes(&attributes, table), "hipPointerGetAttributes");
        expect(attributes.type == hipMemoryTypeDevice, "the table must be device memory");
        expect(attributes.device == device, "the table must belong to the current device");
        float2 w[2];
        thff_cli::hip_check(hipMemcpy(w, table, sizeof(w), hipMemcpyDeviceToHost), "hipMemcpy");
        const double angle = 2.0 * M_PI / n;
        expect(w[0].x == 1.f && w[0].y == 0.f, "W[0] must be exactly 1 + 0i");
        expect(std::fabs(w[1].x - std::cos(angle)) <= 1e-6 &&
                   std::fabs(w[1].y - std::sin(angle)) <= 1e-6,
               "W[1] must be e^(2 pi i / N) for the current length");
    }

    void verify_released(const void* table, int n) {
        expect(table == nullptr && n == 0, "Finalize must release the table and its length");
    }

    int checks_ = 0;
    std::map<std::tuple<int, std::string, std::string>, const void*> pointers_;
};

// Leaves no table behind on any device, whatever failed.
void release_all(const std::vector<int>& devices, int original) noexcept {
    for (int device : devices) {
        if (hipSetDevice(device) != hipSuccess) continue;
        (void)thff_finalize(THFF_FLOAT);
        (void)thff_finalize(THFF_HALF);
    }
    if (!devices.empty()) (void)hipSetDevice(original);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc == 2 && (!std::strcmp(argv[1], "--help") || !std::strcmp(argv[1], "-h"))) {
        std::cout << "Usage: " << argv[0] << "\n"
                  << "Validate twiddle lifecycle and device ownership on every visible GPU.\n"
                  << "No FFT or other GPU kernels are launched.\n";
        return 0;
    }
    std::vector<int> devices;
    int original = 0;
    try {
        if (argc != 1) throw std::runtime_error("This program accepts only --help");
        int count = 0;
        thff_cli::hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        thff_cli::hip_check(hipGetDevice(&original), "hipGetDevice");
        for (int d = 0; d < count; ++d) devices.push_back(d);
        if (devices.empty()) throw std::runtime_error("No visible GPU");
        std::cout << "precision,device,stage,N,pointer,pass\n";
        Audit audit;
        audit.run_type<float>(devices);
        audit.run_type<half>(devices);
        release_all(devices, original);
        std::cerr << "Cache validation: " << audit.checks() << " checks passed across "
                  << devices.size() << " visible GPUs; no GPU kernels launched\n";
        if (devices.size() < 2)
            std::cerr << "Cross-device isolation needs at least two visible GPUs.\n";
        return 0;
    } catch (const std::exception& e) {
        release_all(devices, original);
        std::cerr << "Cache validation error: " << e.what() << '\n';
        return 2;
    }
}
