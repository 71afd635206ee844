// thff_validate.cpp -- host API checks of the reference's correctness program.
//
// Restates check_host_arguments<T>() of sample/validation/fft_validation.cu:
// 320-352 (9 checks per type, 18 in total) against the C++ API of
// <thunderfft/thunderfft.cuh>.  Every check must be decided before any HIP
// call, so `thff_validate --host-only` passes on a machine without a GPU.
// Exit codes as the reference (:401-407): 0 pass, 2 error.
#include <thunderfft/thunderfft.cuh>

#include <cstring>
#include <iostream>
#include <stdexcept>
#include <string>

namespace {

int checks = 0;

template <class Operation>
void expect_invalid_argument(Operation operation, const char* description) {
    try {
        operation();
    } catch (const std::invalid_argument&) {
        ++checks;
        return;
    }
    throw std::runtime_error(std::string("Host API check did not reject ") + description);
}

template <class T>
void check_host_arguments() {
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
    ++checks;
    for (int n : {-1, 0, 32, 8192})
        expect_invalid_argument([n] { thunderfft::ThunderFFTInitialize<T>(n); },
                                "unsupported initialization length");
}

}  // namespace

int main(int argc, char** argv) {
    bool host_only = false;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--host-only") == 0) {
            host_only = true;
        } else if (std::strcmp(argv[i], "--help") == 0 || std::strcmp(argv[i], "-h") == 0) {
            std::cout << "Usage: " << argv[0] << " --host-only\n"
                      << "Checks invalid public API arguments and zero-batch handling without a GPU.\n";
            return 0;
        } else {
            std::cerr << "Validation error: Unknown option: " << argv[i] << '\n';
            return 2;
        }
    }
    if (!host_only) {
        std::cerr << "Validation error: only --host-only is available in this program; the GPU "
                     "matrix runs under pytest -m gpu\n";
        return 2;
    }
    try {
        check_host_arguments<float>();
        check_host_arguments<half>();
        std::cerr << "Host API validation: " << checks << " checks passed before any HIP calls\n";
        return checks == 18 ? 0 : 2;
    } catch (const std::exception& error) {
        std::cerr << "Validation error: " << error.what() << '\n';
        return 2;
    }
}
