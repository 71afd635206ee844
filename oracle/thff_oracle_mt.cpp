// thff_oracle_mt.cpp -- input kind 0 of the reference validation matrix.
//
// TEST INFRASTRUCTURE ONLY (see thff_oracle.c).  Restates
// sample/validation/fft_validation.cu:130-147: complex Gaussian signals from
// std::mt19937(1234 + n) and std::normal_distribution<float>(0, 1), drawn
// real-then-imaginary for every element of every signal in order, each
// signal then scaled to RMS 1 (scale = sqrt(n / sum |x|^2) accumulated in
// double, applied in float).  The generator and distribution are the C++
// standard library's.  The reference draws both parts inside one call,
// make_float2(normal(random), normal(random)), whose argument evaluation
// order C++ leaves unspecified; this restatement fixes real-then-imaginary.
// The kind only has to be a reproducible RMS-1 Gaussian: every check
// compares against the fp64 DFT of the exact values handed to the FFT.
#include <cmath>
#include <cstddef>
#include <random>

extern "C" int thff_make_input_gaussian(int n, long batch, float* out) {
    if (n <= 0 || batch < 0) return -1;
    std::mt19937 random(1234 + n);
    std::normal_distribution<float> normal(0.f, 1.f);
    for (long b = 0; b < batch; ++b) {
        float* x = out + 2 * static_cast<size_t>(b) * n;
        double squared_norm = 0;
        for (int i = 0; i < n; ++i) {
            // Two separate statements fix the draw order (real, then imaginary).
            const float re = normal(random);
            const float im = normal(random);
            x[2 * i] = re;
            x[2 * i + 1] = im;
            squared_norm += double(re) * re + double(im) * im;
        }
        const double scale = std::sqrt(n / squared_norm);
        for (int i = 0; i < n; ++i) {
            x[2 * i] *= scale;
            x[2 * i + 1] *= scale;
        }
    }
    return 0;
}
