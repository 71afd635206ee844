/*
 * thff_oracle.c -- CPU oracle for the batched C2C FFT hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (thunderfft_amd/, include/)
 * links, loads or calls this file.  It is used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, always as the
 * checker and never as the thing measured or shipped.
 *
 * What it restates (paths relative to the reference tree):
 *   - the mathematical target of the reference's numeric oracle, an
 *     unnormalized fp64 C2C transform (cuFFT Z2Z in
 *     sample/validation/fft_validation.cu:55-61,219-222): forward uses
 *     exp(-2*pi*i*n*k/N), inverse exp(+2*pi*i*n*k/N), no 1/N scaling
 *     (include/thunderfft/thunderfft.cuh:129-141);
 *       thff_dft_f64   -- closed-form O(N^2) DFT, exact index reduction
 *       thff_fft_f64   -- iterative radix-2 fp64 FFT, pinned to thff_dft_f64
 *   - the reference's algorithm class in fp32 (radix-4 stages with the
 *     per-size four-step split of include/thunderfft/detail/kernel/
 *     shared_kernel_n*.cuh, e.g. 1024 = 64 x 16 in shared_kernel_n1024_b1.cuh:12-54):
 *       thff_fft_f32_fourstep -- the CPU baseline ("port"), threaded
 *   - the validation metrics of fft_validation.cu:247-272 (relative L2,
 *     max abs, relative Linf, nonfinite count)   -> thff_metrics
 *   - the encode->decode rounding of half storage (fft_validation.cu:63-74,
 *     203-208: __floats2half2_rn / __half22float2)  -> thff_f32_to_f16 ...
 *   - input kinds 1..3 of fft_validation.cu:130-163 -> thff_make_input_kind
 *     (kind 0, mt19937 + normal_distribution, lives in thff_oracle_mt.cpp)
 *   - the counter-based U[-1,1) generator used for the benchmark workloads
 *     -> thff_uniform_fill (identical to the library's device generator)
 *   - direct circular convolution for the fused-convolution checks
 *     (conv1d_fullfft_l4096_thunder.cu:499-545) -> thff_circconv1d_f64,
 *     thff_circconv2d_f64, and its real per-channel form
 *     thff_circconv1d_channels_f64
 *   - the real convolution sample's seeded inputs (srand/rand,
 *     conv1d_fullfft_l4096_thunder.cu:389-401) -> thff_conv_real_inputs
 *   - the tiled valid correlation of sample/conv1d/main.cu:156-174 and that
 *     sample's seeded inputs -> thff_conv1d_valid_f64, thff_conv1d_valid_inputs
 *
 * Pinning: every function here is checked in tests/test_oracle.py against
 * closed forms (impulse/constant/tone spectra), invariants (Parseval,
 * linearity, inverse(forward(x)) = N x), brute force (direct DFT on tiny N),
 * and an independent library routine (numpy.fft / numpy.float16).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define THFF_TAU 6.283185307179586476925286766559

/* ------------------------------------------------------------------------ */
/* fp64 twiddle table: tw[m] = exp(sign * 2*pi*i*m/N), m in [0, N).          */
/* Built from one octant so that every entry is the correctly rounded value  */
/* of cos/sin at an exactly reduced angle.                                   */
/* ------------------------------------------------------------------------ */
static void twiddle_table_f64(int n, int sign, double* re, double* im) {
    for (int m = 0; m < n; ++m) {
        double a = THFF_TAU * (double)m / (double)n;
        re[m] = cos(a);
        im[m] = (double)sign * sin(a);
    }
    /* exact values at the quarter points keep symmetric inputs symmetric */
    re[0] = 1.0; im[0] = 0.0;
    if (n % 4 == 0) {
        re[n / 4] = 0.0; im[n / 4] = (double)sign;
        re[n / 2] = -1.0; im[n / 2] = 0.0;
        re[3 * n / 4] = 0.0; im[3 * n / 4] = -(double)sign;
    }
}

/* Closed-form DFT, X[k] = sum_n x[n] * exp(sign*2*pi*i*((n*k) mod N)/N).
 * in/out: interleaved (re, im) doubles, batch contiguous signals of n.
 * sign = -1 forward, +1 inverse. */
int thff_dft_f64(int n, long batch, int sign, const double* in, double* out) {
    if (n <= 0 || batch < 0 || (sign != 1 && sign != -1)) return -1;
    double* re = (double*)malloc(sizeof(double) * n);
    double* im = (double*)malloc(sizeof(double) * n);
    if (!re || !im) { free(re); free(im); return -2; }
    twiddle_table_f64(n, sign, re, im);
    for (long b = 0; b < batch; ++b) {
        const double* x = in + 2 * (size_t)b * n;
        double* y = out + 2 * (size_t)b * n;
        for (int k = 0; k < n; ++k) {
            double sr = 0.0, si = 0.0;
            long idx = 0;
            for (int j = 0; j < n; ++j) {
                double xr = x[2 * j], xi = x[2 * j + 1];
                sr += xr * re[idx] - xi * im[idx];
                si += xr * im[idx] + xi * re[idx];
                idx += k;
                if (idx >= n) idx -= n;
            }
            y[2 * k] = sr;
            y[2 * k + 1] = si;
        }
    }
    free(re); free(im);
    return 0;
}

/* Iterative radix-2 decimation-in-time FFT in fp64 (bit-reversed load,
 * natural-order output).  n must be a power of two. */
int thff_fft_f64(int n, long batch, int sign, const double* in, double* out) {
    if (n <= 0 || (n & (n - 1)) || batch < 0 || (sign != 1 && sign != -1)) return -1;
    int logn = 0;
    while ((1 << logn) < n) ++logn;
    double* re = (double*)malloc(sizeof(double) * n);
    double* im = (double*)malloc(sizeof(double) * n);
    if (!re || !im) { free(re); free(im); return -2; }
    twiddle_table_f64(n, sign, re, im);
    for (long b = 0; b < batch; ++b) {
        const double* x = in + 2 * (size_t)b * n;
        double* y = out + 2 * (size_t)b * n;
        for (int i = 0; i < n; ++i) {
            int r = 0;
            for (int bit = 0; bit < logn; ++bit) r |= ((i >> bit) & 1) << (logn - 1 - bit);
            y[2 * r] = x[2 * i];
            y[2 * r + 1] = x[2 * i + 1];
        }
        for (int len = 2; len <= n; len <<= 1) {
            int half = len >> 1, step = n / len;
            for (int s = 0; s < n; s += len) {
                for (int j = 0; j < half; ++j) {
                    double wr = re[j * step], wi = im[j * step];
                    double* u = y + 2 * (s + j);
                    double* v = y + 2 * (s + j + half);
                    double tr = v[0] * wr - v[1] * wi;
                    double ti = v[0] * wi + v[1] * wr;
                    v[0] = u[0] - tr; v[1] = u[1] - ti;
                    u[0] += tr; u[1] += ti;
                }
            }
        }
    }
    free(re); free(im);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* fp32 restatement of the reference's algorithm class (CPU baseline).       */
/* Sub-transforms of length 4^k are radix-4 DIT stages; lengths 2*4^k add a  */
/* radix-2 stage; longer lengths use the reference's four-step split         */
/* N = N1 x N2 (first N2 FFTs of length N1 over stride-N2 columns, then the  */
/* W_N^(n2*k1) twiddle, then N1 FFTs of length N2), with N1/N2 taken from     */
/* shared_kernel_n*.cuh: 128=64x2, 256=64x4, 512=64x8, 1024=64x16,           */
/* 2048=32x64, 4096=64x64.  Twiddles come from an fp32 table of W_N rounded  */
/* once from fp64, as in thunderfft_impl_twiddle.cuh:76-91.                  */
/* ------------------------------------------------------------------------ */
typedef struct { float re, im; } cf32;

static void small_fft_f32(int n, const float* twr, const float* twi, int tw_stride,
                          cf32* x, cf32* tmp) {
    /* Stockham-style radix-4 / radix-2 passes on a length-n vector (n <= 64),
     * twiddles W_n^m = tw[m * tw_stride] from the caller's table. */
    int L = 1;
    cf32* src = x;
    cf32* dst = tmp;
    while (L < n) {
        int R = ((n / L) % 4 == 0) ? 4 : 2;
        int m = n / R; /* butterflies */
        for (int b = 0; b < m; ++b) {
            int k = b % L;
            cf32 u[4];
            for (int j = 0; j < R; ++j) {
                cf32 v = src[b + j * m];
                int e = (j * k * (n / (L * R))) % n;
                float wr = twr[e * tw_stride], wi = twi[e * tw_stride];
                u[j].re = v.re * wr - v.im * wi;
                u[j].im = v.re * wi + v.im * wr;
            }
            cf32 o[4];
            if (R == 2) {
                o[0].re = u[0].re + u[1].re; o[0].im = u[0].im + u[1].im;
                o[1].re = u[0].re - u[1].re; o[1].im = u[0].im - u[1].im;
            } else {
                /* sign of the quarter turn follows the table direction */
                float s = twi[(n / 4) * tw_stride]; /* -1 forward, +1 inverse */
                cf32 a = u[0], bb = u[1], c = u[2], d = u[3];
                cf32 t0 = {a.re + c.re, a.im + c.im}, t1 = {a.re - c.re, a.im - c.im};
                cf32 t2 = {bb.re + d.re, bb.im + d.im}, t3 = {bb.re - d.re, bb.im - d.im};
                /* t3 * (s*i) */
                cf32 r3 = {-s * t3.im, s * t3.re};
                o[0].re = t0.re + t2.re; o[0].im = t0.im + t2.im;
                o[2].re = t0.re - t2.re; o[2].im = t0.im - t2.im;
                o[1].re = t1.re + r3.re; o[1].im = t1.im + r3.im;
                o[3].re = t1.re - r3.re; o[3].im = t1.im - r3.im;
            }
            int base = (b - k) * R + k;
            for (int j = 0; j < R; ++j) dst[base + j * L] = o[j];
        }
        cf32* t = src; src = dst; dst = t;
        L *= R;
    }
    if (src != x) memcpy(x, src, sizeof(cf32) * n);
}

static int split_n1(int n) {
    switch (n) {
    case 128: return 64;
    case 256: return 64;
    case 512: return 64;
    case 1024: return 64;
    case 2048: return 32;
    case 4096: return 64;
    default: return n; /* n <= 64: one small transform */
    }
}

typedef struct {
    int n, sign;
    long b0, b1;
    const float* in;
    float* out;
    const float* twr;
    const float* twi;
} f32_job;

static void fft_one_f32(int n, const float* twr, const float* twi, const cf32* x, cf32* y,
                        cf32* work, cf32* col, cf32* tmp) {
    int n1 = split_n1(n);
    if (n1 == n) {
        memcpy(work, x, sizeof(cf32) * n);
        small_fft_f32(n, twr, twi, 1, work, tmp);
        memcpy(y, work, sizeof(cf32) * n);
        return;
    }
    int n2 = n / n1;
    /* step 1: for each n2, FFT of length n1 over x[n2 + N2*n1] */
    for (int c = 0; c < n2; ++c) {
        for (int r = 0; r < n1; ++r) col[r] = x[c + n2 * r];
        small_fft_f32(n1, twr, twi, n2, col, tmp);
        /* step 2: twiddle W_N^(c*k1) */
        for (int k1 = 0; k1 < n1; ++k1) {
            int e = (c * k1) % n;
            float wr = twr[e], wi = twi[e];
            cf32 v = col[k1];
            work[k1 * n2 + c].re = v.re * wr - v.im * wi;
            work[k1 * n2 + c].im = v.re * wi + v.im * wr;
        }
    }
    /* step 3: for each k1, FFT of length n2 over c; X[k1 + n1*k2] */
    for (int k1 = 0; k1 < n1; ++k1) {
        cf32* row = work + (size_t)k1 * n2;
        small_fft_f32(n2, twr, twi, n1, row, tmp);
        for (int k2 = 0; k2 < n2; ++k2) y[k1 + n1 * k2] = row[k2];
    }
}

static void* f32_worker(void* arg) {
    f32_job* job = (f32_job*)arg;
    int n = job->n;
    cf32* work = (cf32*)malloc(sizeof(cf32) * n * 3);
    if (!work) return (void*)1;
    cf32* col = work + n;
    cf32* tmp = work + 2 * n;
    for (long b = job->b0; b < job->b1; ++b) {
        const cf32* x = (const cf32*)(job->in + 2 * (size_t)b * n);
        cf32* y = (cf32*)(job->out + 2 * (size_t)b * n);
        fft_one_f32(n, job->twr, job->twi, x, y, work, col, tmp);
    }
    free(work);
    return NULL;
}

/* fp32 four-step FFT over `batch` signals using `threads` POSIX threads. */
int thff_fft_f32_fourstep(int n, long batch, int sign, const float* in, float* out,
                          int threads) {
    if (n < 4 || (n & (n - 1)) || n > 4096 || batch < 0 || (sign != 1 && sign != -1))
        return -1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    double* dre = (double*)malloc(sizeof(double) * n);
    double* dim = (double*)malloc(sizeof(double) * n);
    float* twr = (float*)malloc(sizeof(float) * n);
    float* twi = (float*)malloc(sizeof(float) * n);
    if (!dre || !dim || !twr || !twi) { free(dre); free(dim); free(twr); free(twi); return -2; }
    twiddle_table_f64(n, sign, dre, dim);
    for (int m = 0; m < n; ++m) { twr[m] = (float)dre[m]; twi[m] = (float)dim[m]; }
    free(dre); free(dim);
    pthread_t tid[256];
    f32_job jobs[256];
    long per = (batch + threads - 1) / threads;
    int launched = 0, rc = 0;
    for (int t = 0; t < threads; ++t) {
        long b0 = (long)t * per, b1 = b0 + per;
        if (b1 > batch) b1 = batch;
        if (b0 >= b1) break;
        jobs[t] = (f32_job){n, sign, b0, b1, in, out, twr, twi};
        if (threads == 1) { if (f32_worker(&jobs[t])) rc = -2; continue; }
        if (pthread_create(&tid[t], NULL, f32_worker, &jobs[t]) != 0) { rc = -3; break; }
        ++launched;
    }
    for (int t = 0; t < launched; ++t) {
        void* r = NULL;
        pthread_join(tid[t], &r);
        if (r) rc = -2;
    }
    free(twr); free(twi);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Metrics (fft_validation.cu:247-272).  y is float interleaved, ref double. */
/* out[0]=rel_l2 out[1]=max_abs out[2]=rel_linf out[3]=nonfinite count       */
/* ------------------------------------------------------------------------ */
void thff_metrics(long count, const float* y, const double* ref, double* out) {
    double se = 0, sr = 0, maxe = 0, maxr = 0;
    long nonfinite = 0;
    for (long i = 0; i < count; ++i) {
        double yx = y[2 * i], yy = y[2 * i + 1];
        if (!isfinite(yx) || !isfinite(yy)) ++nonfinite;
        double dx = yx - ref[2 * i], dy = yy - ref[2 * i + 1];
        se += dx * dx + dy * dy;
        sr += ref[2 * i] * ref[2 * i] + ref[2 * i + 1] * ref[2 * i + 1];
        double e = hypot(dx, dy), r = hypot(ref[2 * i], ref[2 * i + 1]);
        if (e > maxe) maxe = e;
        if (r > maxr) maxr = r;
    }
    out[0] = sqrt(se / sr);
    out[1] = maxe;
    out[2] = maxr > 0 ? maxe / maxr : maxe;
    out[3] = (double)nonfinite;
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 round-to-nearest-even conversion (== __float2half_rn) and    */
/* exact widening (== __half2float).                                          */
/* ------------------------------------------------------------------------ */
uint16_t thff_f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u | ((absx >> 13) & 0x3FFu) : 0));
    if (absx >= 0x477FF000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00u);
    if (absx < 0x38800000u) { /* result is subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t mant = (absx & 0x7FFFFFu) | 0x800000u;
        int exp = (int)(absx >> 23); /* 102..112 */
        int shift = 126 - exp;       /* value = mant * 2^(exp-150); half ulp 2^-24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t mant = absx & 0x7FFFFFu;
    uint32_t q = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

float thff_f16_bits_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t x;
    if (e == 0x1F) x = sign | 0x7F800000u | (m << 13);
    else if (e == 0) {
        if (m == 0) x = sign;
        else {
            float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else x = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void thff_f32_to_f16_array(long count, const float* in, uint16_t* out) {
    for (long i = 0; i < count; ++i) out[i] = thff_f32_to_f16_bits(in[i]);
}
void thff_f16_to_f32_array(long count, const uint16_t* in, float* out) {
    for (long i = 0; i < count; ++i) out[i] = thff_f16_bits_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Counter-based U[-1,1) generator: component c (real of element e is        */
/* c = 2e, imaginary c = 2e+1) gets 2*(splitmix64(seed ^ c) >> 40)*2^-24 - 1, */
/* exact in fp32.  The library's device fill uses the same formula.          */
/* ------------------------------------------------------------------------ */
static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void thff_uniform_fill(uint64_t seed, uint64_t first_component, long count, float* out) {
    for (long i = 0; i < count; ++i) {
        uint64_t r = splitmix64(seed ^ (first_component + (uint64_t)i)) >> 40;
        out[i] = (float)((double)r * (1.0 / 8388608.0) - 1.0);
    }
}

/* Input kinds 1..3 of fft_validation.cu:130-163 (kind 0 is in the C++ file):
 *   1 offset impulse (.75,.25) at (13b+7) mod n
 *   2 complex tone .5*exp(i(2*pi*f*i/n + .13b)), f = 1 + (7b) mod (n-1)
 *   3 constant (.25, -.125)                                                  */
int thff_make_input_kind(int n, long batch, int kind, float* out) {
    if (n <= 1 || batch < 0 || kind < 1 || kind > 3) return -1;
    memset(out, 0, sizeof(float) * 2 * (size_t)n * batch);
    for (long b = 0; b < batch; ++b) {
        float* x = out + 2 * (size_t)b * n;
        if (kind == 1) {
            long i = (13 * b + 7) % n;
            x[2 * i] = 0.75f;
            x[2 * i + 1] = 0.25f;
        } else if (kind == 2) {
            long f = 1 + (7 * b) % (n - 1);
            for (int i = 0; i < n; ++i) {
                double phase = THFF_TAU * (double)f * i / n + 0.13 * (double)b;
                x[2 * i] = (float)(0.5 * cos(phase));
                x[2 * i + 1] = (float)(0.5 * sin(phase));
            }
        } else {
            for (int i = 0; i < n; ++i) { x[2 * i] = 0.25f; x[2 * i + 1] = -0.125f; }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Direct circular convolution in fp64 (conv1d_fullfft_l4096_thunder.cu:     */
/* 499-545 compares against this quantity).  1D: y[b][n] = sum_m x[b][m] *   */
/* h[hb][(n-m) mod N] with hb = b (per-signal filters) or 0 (shared filter). */
/* 2D: y[b][r][c] = sum x[b][r'][c'] * h[(r-r') mod H][(c-c') mod W].        */
/* All arrays interleaved complex doubles.                                   */
/* ------------------------------------------------------------------------ */
int thff_circconv1d_f64(int n, long batch, int per_signal_filter, const double* x,
                        const double* h, double* y) {
    if (n <= 0 || batch < 0) return -1;
    for (long b = 0; b < batch; ++b) {
        const double* xs = x + 2 * (size_t)b * n;
        const double* hs = h + (per_signal_filter ? 2 * (size_t)b * n : 0);
        double* ys = y + 2 * (size_t)b * n;
        for (int k = 0; k < n; ++k) {
            double sr = 0, si = 0;
            for (int m = 0; m < n; ++m) {
                int d = k - m;
                if (d < 0) d += n;
                double ar = xs[2 * m], ai = xs[2 * m + 1];
                double br = hs[2 * d], bi = hs[2 * d + 1];
                sr += ar * br - ai * bi;
                si += ar * bi + ai * br;
            }
            ys[2 * k] = sr;
            ys[2 * k + 1] = si;
        }
    }
    return 0;
}

/* Direct 2-D circular convolution, y[r][c] = sum_{dr,dc} h[dr][dc] *
 * x[(r - dr) mod rows][(c - dc) mod cols], accumulated one filter tap at a
 * time so that zero taps cost nothing: O(rows cols nnz(h)) per image, which
 * keeps a 1024 x 1024 image with a 7 x 7 filter (the reference sample's
 * shape, sample/conv2d/thunder.cu:556-565, with its small f x f filters)
 * within a second. */
int thff_circconv2d_f64(int rows, int cols, long batch, const double* x, const double* h,
                        double* y) {
    if (rows <= 0 || cols <= 0 || batch < 0) return -1;
    size_t img = (size_t)rows * cols;
    for (long b = 0; b < batch; ++b) {
        const double* xs = x + 2 * img * b;
        double* ys = y + 2 * img * b;
        memset(ys, 0, 2 * img * sizeof(double));
        for (int dr = 0; dr < rows; ++dr)
            for (int dc = 0; dc < cols; ++dc) {
                const double wr = h[2 * ((size_t)dr * cols + dc)];
                const double wi = h[2 * ((size_t)dr * cols + dc) + 1];
                if (wr == 0.0 && wi == 0.0) continue;
                for (int r = 0; r < rows; ++r) {
                    int r2 = r - dr;
                    if (r2 < 0) r2 += rows;
                    const double* xrow = xs + 2 * (size_t)r2 * cols;
                    double* yrow = ys + 2 * (size_t)r * cols;
                    for (int c = 0; c < cols; ++c) {
                        int c2 = c - dc;
                        if (c2 < 0) c2 += cols;
                        const double ar = xrow[2 * c2], ai = xrow[2 * c2 + 1];
                        yrow[2 * c] += ar * wr - ai * wi;
                        yrow[2 * c + 1] += ar * wi + ai * wr;
                    }
                }
            }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Real-input convolution with one real filter per channel, as the real     */
/* fused-convolution sample validates it (conv1d_fullfft_l4096_thunder.cu:  */
/* 499-520): signals x[s][n], s = b*channels + d, filter d = s mod channels */
/* with `taps` leading taps h[d][k], k < taps (the rest of its n are zero): */
/*   y[s][n] = sum_{k < taps} x[s][(n - k) mod n] * h[d][k].                */
/* ------------------------------------------------------------------------ */
int thff_circconv1d_channels_f64(int n, long signals, int channels, int taps, const double* x,
                                 const double* h, double* y) {
    if (n <= 0 || signals < 0 || channels <= 0 || taps < 0 || taps > n) return -1;
    for (long s = 0; s < signals; ++s) {
        const double* xs = x + (size_t)s * n;
        const double* hs = h + (size_t)(s % channels) * n;
        double* ys = y + (size_t)s * n;
        for (int k = 0; k < n; ++k) {
            double acc = 0;
            for (int j = 0; j < taps; ++j) {
                int m = k - j;
                if (m < 0) m += n;
                acc += xs[m] * hs[j];
            }
            ys[k] = acc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* The real fused-convolution sample's inputs (conv1d_fullfft_l4096_thunder */
/* .cu:389-401, seeded by std::srand(seed) at :617): after srand(seed),     */
/* signals*n values rand()/RAND_MAX in signal order, then for each channel  */
/* d its first `taps` taps (rand()/RAND_MAX)/n (the sample draws no         */
/* imaginary part for its real filters).  Taps k >= taps are zero.  Uses    */
/* the C library's own srand/rand, i.e. the same sequence as the sample on  */
/* the same C library.                                                      */
/* ------------------------------------------------------------------------ */
int thff_conv_real_inputs(int n, int taps, long signals, int channels, unsigned seed, float* x,
                          float* h) {
    if (n <= 0 || signals < 0 || channels <= 0 || taps < 0 || taps > n) return -1;
    srand(seed);
    for (size_t i = 0; i < (size_t)signals * n; ++i) x[i] = (float)rand() / (float)RAND_MAX;
    memset(h, 0, sizeof(float) * (size_t)channels * n);
    for (int d = 0; d < channels; ++d)
        for (int k = 0; k < taps; ++k)
            h[(size_t)d * n + k] = ((float)rand() / (float)RAND_MAX) / (float)n;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Valid complex correlation, the tiled-conv sample's definition            */
/* (sample/conv1d/main.cu:156-174, no conjugation), per signal b:           */
/*   y[b][i] = sum_{k < ntaps} x[b][i + k] * f[k],  i < len - ntaps + 1.    */
/* Interleaved complex doubles.                                             */
/* ------------------------------------------------------------------------ */
int thff_conv1d_valid_f64(long len, int ntaps, long batch, const double* x, const double* f,
                          double* y) {
    if (ntaps < 1 || len < ntaps || batch < 0) return -1;
    const long out = len - ntaps + 1;
    for (long b = 0; b < batch; ++b) {
        const double* xs = x + 2 * (size_t)b * len;
        double* ys = y + 2 * (size_t)b * out;
        for (long i = 0; i < out; ++i) {
            double sr = 0, si = 0;
            for (int k = 0; k < ntaps; ++k) {
                const double ar = xs[2 * (i + k)], ai = xs[2 * (i + k) + 1];
                sr += ar * f[2 * k] - ai * f[2 * k + 1];
                si += ar * f[2 * k + 1] + ai * f[2 * k];
            }
            ys[2 * i] = sr;
            ys[2 * i + 1] = si;
        }
    }
    return 0;
}

/* The tiled-conv sample's inputs (sample/conv1d/main.cu:233,130-135,260-262): */
/* after srand(seed), len complex inputs then ntaps complex taps, each value  */
/* (rand()/RAND_MAX, rand()/RAND_MAX) as fp32 (real drawn first).             */
int thff_conv1d_valid_inputs(long len, int ntaps, unsigned seed, float* x, float* f) {
    if (len < 0 || ntaps < 0) return -1;
    srand(seed);
    for (size_t i = 0; i < 2 * (size_t)len; ++i) x[i] = (float)rand() / (float)RAND_MAX;
    for (int i = 0; i < 2 * ntaps; ++i) f[i] = (float)rand() / (float)RAND_MAX;
    return 0;
}
