/*
 * butterfly_oracle.c -- CPU restatement of the reference's radix-2 butterfly
 * path, used ONLY as test infrastructure (the parity checker, the smoke check
 * and bench.py's cpu_baseline leg).  Nothing in the shipped library links or
 * calls this file.
 *
 * What it restates (reference files under TruNcat3/kunlunxin-fft):
 *   include/butterfly/bit_reverse.hpp:15-22   bit_reverse(x, bits)
 *   include/butterfly/twiddle.hpp:18-36       twiddle(idx, n), twiddle_table(n),
 *                                             twiddle_stride(n, n_stage)
 *   include/butterfly/fft.hpp:28-40           dit_stage  (a + w*b, a - w*b)
 *   include/butterfly/fft.hpp:43-55           dif_stage  (a + b, (a - b)*w)
 *   include/butterfly/fft.hpp:58-67           bit_reverse_permute (out of place)
 *   include/butterfly/fft.hpp:70-80           fft_dit: permute, then stages 1,2,..,N/2
 *   include/butterfly/fft.hpp:84-96           fft_dif: stages N/2,..,1, then permute
 *
 * Data are interleaved complex<double> (re, im, re, im, ...), the memory
 * layout of numpy complex128 and of std::complex<double> arrays.  Like the
 * reference, every stage rebuilds the N/2-entry twiddle table (N/2 cos/sin
 * calls per stage): that cost is part of the CPU baseline being timed.
 *
 * Arithmetic follows the reference's operation order in double precision
 * (complex product (ac - bd, ad + bc)); build with -ffp-contract=off so no
 * fused multiply-add changes the rounding.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>
#include <time.h>

static const double kPi = 3.14159265358979323846;

/* bit_reverse.hpp:15-22 */
uint32_t oracle_bit_reverse(uint32_t x, int bits) {
    uint32_t rev = 0;
    for (int i = 0; i < bits; ++i) {
        rev = (rev << 1) | (x & 1u);
        x >>= 1;
    }
    return rev;
}

/* bit_reverse.hpp:25-36: returns -1 when n is not a power of two. */
int oracle_log2_exact(int64_t n) {
    if (n <= 0 || (n & (n - 1)) != 0) return -1;
    int b = 0;
    while (((int64_t)1 << b) != n) ++b;
    return b;
}

/* twiddle.hpp:25-31: w[idx] = exp(-2*pi*i*idx/n), idx in [0, n/2). */
void oracle_twiddle_table(int64_t n, double* w) {
    for (int64_t idx = 0; idx < n / 2; ++idx) {
        const double ang = -2.0 * kPi * (double)idx / (double)n;
        w[2 * idx] = cos(ang);
        w[2 * idx + 1] = sin(ang);
    }
}

/* fft.hpp:28-40 -- one radix-2 DIT stage in place, half-span n_stage. */
void oracle_dit_stage(double* a, int64_t n, int64_t n_stage) {
    const int64_t M = n / (2 * n_stage); /* twiddle.hpp:34-36 */
    double* w = (double*)malloc(sizeof(double) * (size_t)(n > 1 ? n : 2));
    oracle_twiddle_table(n, w);
    for (int64_t k = 0; k < n / 2; ++k) {
        const int64_t j = k % n_stage;
        const int64_t i = (k / n_stage) * 2 * n_stage + j;
        const double xr = a[2 * i], xi = a[2 * i + 1];
        const double br = a[2 * (i + n_stage)], bi = a[2 * (i + n_stage) + 1];
        const double wr = w[2 * (j * M)], wi = w[2 * (j * M) + 1];
        const double yr = br * wr - bi * wi;
        const double yi = br * wi + bi * wr;
        a[2 * i] = xr + yr;
        a[2 * i + 1] = xi + yi;
        a[2 * (i + n_stage)] = xr - yr;
        a[2 * (i + n_stage) + 1] = xi - yi;
    }
    free(w);
}

/* fft.hpp:43-55 -- one radix-2 DIF stage in place. */
void oracle_dif_stage(double* a, int64_t n, int64_t n_stage) {
    const int64_t M = n / (2 * n_stage);
    double* w = (double*)malloc(sizeof(double) * (size_t)(n > 1 ? n : 2));
    oracle_twiddle_table(n, w);
    for (int64_t k = 0; k < n / 2; ++k) {
        const int64_t j = k % n_stage;
        const int64_t i = (k / n_stage) * 2 * n_stage + j;
        const double xr = a[2 * i], xi = a[2 * i + 1];
        const double yr = a[2 * (i + n_stage)], yi = a[2 * (i + n_stage) + 1];
        const double dr = xr - yr, di = xi - yi;
        const double wr = w[2 * (j * M)], wi = w[2 * (j * M) + 1];
        a[2 * i] = xr + yr;
        a[2 * i + 1] = xi + yi;
        a[2 * (i + n_stage)] = dr * wr - di * wi;
        a[2 * (i + n_stage) + 1] = dr * wi + di * wr;
    }
    free(w);
}

/* fft.hpp:58-67: out[bit_reverse(i)] = a[i]. */
void oracle_bit_reverse_permute(const double* a, double* out, int64_t n) {
    const int bits = oracle_log2_exact(n);
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t r = oracle_bit_reverse((uint32_t)i, bits);
        out[2 * (int64_t)r] = a[2 * i];
        out[2 * (int64_t)r + 1] = a[2 * i + 1];
    }
}

/* fft.hpp:70-80: forward FFT in place; returns -1 for a non power of two. */
int oracle_fft_dit(double* a, int64_t n) {
    if (oracle_log2_exact(n) < 0) return -1;
    double* t = (double*)malloc(sizeof(double) * 2 * (size_t)n);
    oracle_bit_reverse_permute(a, t, n);
    memcpy(a, t, sizeof(double) * 2 * (size_t)n);
    free(t);
    for (int64_t s = 1; s < n; s *= 2) oracle_dit_stage(a, n, s);
    return 0;
}

/* fft.hpp:84-96: DIF stages N/2 .. 1, then the bit-reversal permutation. */
int oracle_fft_dif(double* a, int64_t n) {
    if (oracle_log2_exact(n) < 0) return -1;
    for (int64_t s = n / 2; s >= 1; s /= 2) oracle_dif_stage(a, n, s);
    double* t = (double*)malloc(sizeof(double) * 2 * (size_t)n);
    oracle_bit_reverse_permute(a, t, n);
    memcpy(a, t, sizeof(double) * 2 * (size_t)n);
    free(t);
    return 0;
}

/* ---- batch drivers (rows are independent: the reference loops over rows) */

typedef struct {
    double* a;
    int64_t n, r0, r1;
    int dif;
} row_job;

static void* row_worker(void* p) {
    row_job* j = (row_job*)p;
    for (int64_t r = j->r0; r < j->r1; ++r) {
        if (j->dif) oracle_fft_dif(j->a + 2 * r * j->n, j->n);
        else oracle_fft_dit(j->a + 2 * r * j->n, j->n);
    }
    return NULL;
}

/* Forward FFT of `batch` contiguous rows of length n, rows split over
 * `threads` POSIX threads (threads <= 1 runs on the calling thread). */
int oracle_fft_batch(double* a, int64_t n, int64_t batch, int dif, int threads) {
    if (oracle_log2_exact(n) < 0 || batch < 0) return -1;
    if (threads <= 1 || batch <= 1) {
        row_job j = {a, n, 0, batch, dif};
        row_worker(&j);
        return 0;
    }
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    row_job jobs[256];
    int64_t per = (batch + threads - 1) / threads;
    int used = 0;
    for (int t = 0; t < threads; ++t) {
        int64_t r0 = t * per, r1 = r0 + per < batch ? r0 + per : batch;
        if (r0 >= r1) break;
        jobs[t] = (row_job){a, n, r0, r1, dif};
        pthread_create(&tid[t], NULL, row_worker, &jobs[t]);
        ++used;
    }
    for (int t = 0; t < used; ++t) pthread_join(tid[t], NULL);
    return 0;
}

/* Median wall time (seconds, CLOCK_MONOTONIC) of `reps` runs of
 * oracle_fft_batch over a private copy of `a` refreshed before each run. */
double oracle_time_fft_batch(const double* a, int64_t n, int64_t batch, int dif,
                             int threads, int reps) {
    if (reps < 1) reps = 1;
    if (reps > 64) reps = 64;
    size_t bytes = sizeof(double) * 2 * (size_t)n * (size_t)batch;
    double* work = (double*)malloc(bytes);
    double t[64];
    for (int r = 0; r < reps; ++r) {
        memcpy(work, a, bytes);
        struct timespec s0, s1;
        clock_gettime(CLOCK_MONOTONIC, &s0);
        oracle_fft_batch(work, n, batch, dif, threads);
        clock_gettime(CLOCK_MONOTONIC, &s1);
        t[r] = (double)(s1.tv_sec - s0.tv_sec) + 1e-9 * (double)(s1.tv_nsec - s0.tv_nsec);
    }
    free(work);
    for (int i = 1; i < reps; ++i) { /* insertion sort */
        double v = t[i];
        int k = i - 1;
        while (k >= 0 && t[k] > v) { t[k + 1] = t[k]; --k; }
        t[k + 1] = v;
    }
    return t[reps / 2];
}

/* Naive O(N^2) DFT in double (src/host/fft_check.cpp:20-34 restated), the
 * brute-force truth the radix-2 restatement is pinned against. */
void oracle_naive_dft(const double* a, double* out, int64_t n, int inverse) {
    const double sgn = inverse ? 2.0 : -2.0;
    for (int64_t k = 0; k < n; ++k) {
        double sr = 0.0, si = 0.0;
        for (int64_t m = 0; m < n; ++m) {
            const double ang = sgn * kPi * (double)k * (double)m / (double)n;
            const double c = cos(ang), s = sin(ang);
            sr += a[2 * m] * c - a[2 * m + 1] * s;
            si += a[2 * m] * s + a[2 * m + 1] * c;
        }
        out[2 * k] = sr;
        out[2 * k + 1] = si;
    }
}
