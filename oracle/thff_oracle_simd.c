/*
 * thff_oracle_simd.c -- the CPU baseline's batched fp32 FFT, vectorised
 * across signals.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (thunderfft_amd/, include/)
 * links, loads or calls this file.  bench.py's cpu_baseline leg times it (and
 * tests/ check it); it is never the thing measured on the GPU or shipped.
 *
 * What it restates: the same unnormalized C2C transform as thff_fft_f32_fourstep
 * (forward exp(-2*pi*i*n*k/N), inverse exp(+...), no scaling; the reference's
 * include/thunderfft/thunderfft.cuh:129-141), in the reference's algorithm
 * class -- radix-4 stages, a radix-2 stage for N = 2 * 4^k
 * (include/thunderfft/detail/kernel/unit_kernel_fp32.cuh:138-210 runs radix-4
 * stages) -- written for a CPU: V = 16 signals are transformed in lockstep,
 * each complex value of the transform held as 16 real and 16 imaginary parts
 * (one per signal), so every butterfly is a few vector instructions over the
 * 16 signals (the compiler vectorises the loops over them); Stockham passes
 * between two buffers of N such values (128 KiB at N = 1024, in L2); the
 * twiddles of every pass precomputed once per call from fp64 (one fp32
 * rounding, as the four-step's table).  Groups of 16 signals are split over
 * POSIX threads; a last partial group is padded with zeros.
 *
 * Pinning: tests/test_oracle.py checks it against the fp64 FFT (itself pinned
 * to the direct DFT) at every N in both directions, on batches that are not
 * multiples of 16, and for thread-count independence.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define THFF_TAU_D 6.283185307179586476925286766559
#define V 16

typedef struct {
    float re[V], im[V];
} vcf;

typedef struct {
    int n, sign, passes;
    int radix[8];     /* radix of each pass */
    int L[8];         /* product of the previous radices */
    int tw_off[8];    /* offset of the pass's twiddles in twr / twi */
    float* twr;       /* pass p: [k][j - 1], k < L, j < radix */
    float* twi;
} plan_t;

static int plan_make(int n, int sign, plan_t* p) {
    p->n = n;
    p->sign = sign;
    p->passes = 0;
    int total = 0, L = 1;
    while (L < n) {
        int R = ((n / L) % 4 == 0) ? 4 : 2;
        p->radix[p->passes] = R;
        p->L[p->passes] = L;
        p->tw_off[p->passes] = total;
        total += L * (R - 1);
        L *= R;
        p->passes++;
    }
    p->twr = (float*)malloc(sizeof(float) * (total > 0 ? total : 1));
    p->twi = (float*)malloc(sizeof(float) * (total > 0 ? total : 1));
    if (!p->twr || !p->twi) return -1;
    for (int s = 0; s < p->passes; ++s) {
        const int R = p->radix[s], Ls = p->L[s];
        for (int k = 0; k < Ls; ++k)
            for (int j = 1; j < R; ++j) {
                /* W_n^(j k n / (L R)), the exponent reduced exactly */
                const long e = ((long)j * k * (n / (Ls * R))) % n;
                const double a = THFF_TAU_D * (double)e / (double)n;
                p->twr[p->tw_off[s] + k * (R - 1) + (j - 1)] = (float)cos(a);
                p->twi[p->tw_off[s] + k * (R - 1) + (j - 1)] = (float)(sign * sin(a));
            }
    }
    return 0;
}

static void plan_free(plan_t* p) {
    free(p->twr);
    free(p->twi);
}

/* One transform of V signals: x (n values) -> result in x; y is scratch. */
static void fft_group(const plan_t* p, vcf* x, vcf* y) {
    const int n = p->n;
    const float s = (float)p->sign; /* -1 forward, +1 inverse: the quarter turn */
    vcf* src = x;
    vcf* dst = y;
    for (int pass = 0; pass < p->passes; ++pass) {
        const int R = p->radix[pass], L = p->L[pass], m = n / R;
        const float* wr = p->twr + p->tw_off[pass];
        const float* wi = p->twi + p->tw_off[pass];
        for (int q = 0; q < m / L; ++q) {
            for (int k = 0; k < L; ++k) {
                const int b = q * L + k;
                vcf* o = dst + q * L * R + k;
                if (R == 4) {
                    const vcf* a0 = src + b;
                    const vcf* a1 = src + b + m;
                    const vcf* a2 = src + b + 2 * m;
                    const vcf* a3 = src + b + 3 * m;
                    const float w1r = wr[3 * k], w1i = wi[3 * k];
                    const float w2r = wr[3 * k + 1], w2i = wi[3 * k + 1];
                    const float w3r = wr[3 * k + 2], w3i = wi[3 * k + 2];
                    for (int v = 0; v < V; ++v) {
                        const float u0r = a0->re[v], u0i = a0->im[v];
                        const float u1r = a1->re[v] * w1r - a1->im[v] * w1i;
                        const float u1i = a1->re[v] * w1i + a1->im[v] * w1r;
                        const float u2r = a2->re[v] * w2r - a2->im[v] * w2i;
                        const float u2i = a2->re[v] * w2i + a2->im[v] * w2r;
                        const float u3r = a3->re[v] * w3r - a3->im[v] * w3i;
                        const float u3i = a3->re[v] * w3i + a3->im[v] * w3r;
                        const float t0r = u0r + u2r, t0i = u0i + u2i;
                        const float t1r = u0r - u2r, t1i = u0i - u2i;
                        const float t2r = u1r + u3r, t2i = u1i + u3i;
                        const float t3r = u1r - u3r, t3i = u1i - u3i;
                        /* t3 * (s i) */
                        const float r3r = -s * t3i, r3i = s * t3r;
                        o[0].re[v] = t0r + t2r;
                        o[0].im[v] = t0i + t2i;
                        o[2 * L].re[v] = t0r - t2r;
                        o[2 * L].im[v] = t0i - t2i;
                        o[L].re[v] = t1r + r3r;
                        o[L].im[v] = t1i + r3i;
                        o[3 * L].re[v] = t1r - r3r;
                        o[3 * L].im[v] = t1i - r3i;
                    }
                } else {
                    const vcf* a0 = src + b;
                    const vcf* a1 = src + b + m;
                    const float w1r = wr[k], w1i = wi[k];
                    for (int v = 0; v < V; ++v) {
                        const float u1r = a1->re[v] * w1r - a1->im[v] * w1i;
                        const float u1i = a1->re[v] * w1i + a1->im[v] * w1r;
                        o[0].re[v] = a0->re[v] + u1r;
                        o[0].im[v] = a0->im[v] + u1i;
                        o[L].re[v] = a0->re[v] - u1r;
                        o[L].im[v] = a0->im[v] - u1i;
                    }
                }
            }
        }
        vcf* t = src;
        src = dst;
        dst = t;
    }
    if (src != x) memcpy(x, src, sizeof(vcf) * (size_t)n);
}

typedef struct {
    const plan_t* p;
    long g0, g1, batch;
    const float* in;
    float* out;
} job_t;

static void* worker(void* arg) {
    const job_t* j = (const job_t*)arg;
    const int n = j->p->n;
    vcf* x = (vcf*)aligned_alloc(64, sizeof(vcf) * (size_t)n);
    vcf* y = (vcf*)aligned_alloc(64, sizeof(vcf) * (size_t)n);
    if (!x || !y) {
        free(x);
        free(y);
        return (void*)1;
    }
    for (long g = j->g0; g < j->g1; ++g) {
        const long b0 = g * V;
        for (int v = 0; v < V; ++v) {
            const long b = b0 + v;
            if (b < j->batch) {
                const float* src = j->in + 2 * (size_t)b * n;
                for (int t = 0; t < n; ++t) {
                    x[t].re[v] = src[2 * t];
                    x[t].im[v] = src[2 * t + 1];
                }
            } else {
                for (int t = 0; t < n; ++t) x[t].re[v] = x[t].im[v] = 0.0f;
            }
        }
        fft_group(j->p, x, y);
        for (int v = 0; v < V; ++v) {
            const long b = b0 + v;
            if (b >= j->batch) break;
            float* dst = j->out + 2 * (size_t)b * n;
            for (int t = 0; t < n; ++t) {
                dst[2 * t] = x[t].re[v];
                dst[2 * t + 1] = x[t].im[v];
            }
        }
    }
    free(x);
    free(y);
    return NULL;
}

/* Batched fp32 FFT, 16 signals per vector group, over `threads` threads. */
int thff_fft_f32_batched(int n, long batch, int sign, const float* in, float* out, int threads) {
    if (n < 4 || (n & (n - 1)) || n > 4096 || batch < 0 || (sign != 1 && sign != -1)) return -1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    plan_t p;
    if (plan_make(n, sign, &p) != 0) {
        plan_free(&p);
        return -2;
    }
    const long groups = (batch + V - 1) / V;
    const long per = (groups + threads - 1) / threads;
    pthread_t tid[256];
    job_t jobs[256];
    int launched = 0, rc = 0;
    for (int t = 0; t < threads; ++t) {
        const long g0 = (long)t * per;
        const long g1 = g0 + per < groups ? g0 + per : groups;
        if (g0 >= g1) break;
        jobs[t] = (job_t){&p, g0, g1, batch, in, out};
        if (threads == 1) {
            if (worker(&jobs[t])) rc = -2;
            continue;
        }
        if (pthread_create(&tid[t], NULL, worker, &jobs[t]) != 0) {
            rc = -3;
            break;
        }
        ++launched;
    }
    for (int t = 0; t < launched; ++t) {
        void* r = NULL;
        pthread_join(tid[t], &r);
        if (r) rc = -2;
    }
    plan_free(&p);
    return rc;
}
