/* A plain C caller of the C ABI in include/mfft.h: no Python and no torch,
 * only the HIP runtime for device memory and a stream.  Built by
 * __graft_entry__.build() into tests/_build/c_abi_caller and run by
 * tests/test_gpu_c_abi.py on a GPU.
 *
 * 1. c2c forward, automatic flow, backward norm, on the NULL stream;
 * 2. c2c inverse, ortho norm, the radix-2 stage flow, with a plan created
 *    with MFFT_PLAN_CALLER_WORKSPACE and executed through mfft_execute_ws
 *    on a stream of its own (mfft_execute must refuse that plan);
 * 3. r2c forward then c2r inverse (automatic flows), a round trip;
 * 4. the same two transforms by hand around an N/2-point c2c plan: the
 *    packed reals through the core and mfft_r2c_stitch, then mfft_c2r_pre,
 *    the core again and mfft_c2r_unpack with scale 2/N.
 * Each result is compared with a direct O(n^2) DFT in double precision
 * (relative L2 error, the library's 1e-5 gate).  Exit status 0 = all pass.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "mfft.h"

#define N 1024
#define B 3
#define TOL 1e-5

static void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        exit(2);
    }
}

static void mfft_ok(int rc, const char* what) {
    if (rc != MFFT_OK) {
        fprintf(stderr, "%s: rc=%d %s\n", what, rc, mfft_last_error());
        exit(2);
    }
}

/* out[r][k] = scale * sum_j in[r][j] exp(sign 2 pi i j k / n), interleaved doubles */
static void dft(const double* in, double* out, int n, int rows, int sign, double scale) {
    for (int r = 0; r < rows; ++r) {
        const double* x = in + 2 * (size_t)r * n;
        double* y = out + 2 * (size_t)r * n;
        for (int k = 0; k < n; ++k) {
            double re = 0.0, im = 0.0;
            for (int j = 0; j < n; ++j) {
                const double a = sign * 2.0 * M_PI * (double)(((long long)j * k) % n) / n;
                const double c = cos(a), s = sin(a);
                re += x[2 * j] * c - x[2 * j + 1] * s;
                im += x[2 * j] * s + x[2 * j + 1] * c;
            }
            y[2 * k] = scale * re;
            y[2 * k + 1] = scale * im;
        }
    }
}

static double rel_l2(const float* got, const double* ref, size_t count) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < count; ++i) {
        const double d = (double)got[i] - ref[i];
        num += d * d;
        den += ref[i] * ref[i];
    }
    return sqrt(num / den);
}

int main(void) {
    const size_t cplx = (size_t)N * B;  /* complex elements of one c2c buffer */
    float* h_in = malloc(cplx * 2 * sizeof(float));
    float* h_out = malloc(cplx * 2 * sizeof(float));
    double* d_in = malloc(cplx * 2 * sizeof(double));
    double* d_ref = malloc(cplx * 2 * sizeof(double));
    if (!h_in || !h_out || !d_in || !d_ref) return 2;
    unsigned long long s = 20261202ULL;
    for (size_t i = 0; i < cplx * 2; ++i) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;  /* LCG, top 24 bits -> [-1, 1) */
        h_in[i] = (float)((double)(s >> 40) / (double)(1ULL << 23) - 1.0);
        d_in[i] = h_in[i];
    }
    void *din = NULL, *dout = NULL, *ws = NULL, *dreal = NULL;
    hip_ok(hipMalloc(&din, cplx * 8), "hipMalloc in");
    hip_ok(hipMalloc(&dout, cplx * 8), "hipMalloc out");
    hip_ok(hipMemcpy(din, h_in, cplx * 8, hipMemcpyHostToDevice), "copy in");
    int fails = 0;

    /* 1. c2c forward, automatic flow */
    mfft_plan* p = NULL;
    mfft_ok(mfft_plan_create(&p, N, B, MFFT_C2C, MFFT_FORWARD, MFFT_NORM_BACKWARD, MFFT_FLOW_AUTO, NULL, 0),
            "plan c2c");
    mfft_ok(mfft_execute(p, din, dout, NULL), "execute c2c");
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(h_out, dout, cplx * 8, hipMemcpyDeviceToHost), "copy out");
    dft(d_in, d_ref, N, B, -1, 1.0);
    double e = rel_l2(h_out, d_ref, cplx * 2);
    printf("c2c forward (auto flow): rel L2 %.3e\n", e);
    fails += !(e <= TOL);
    mfft_ok(mfft_plan_destroy(p), "destroy");

    /* 2. c2c inverse, ortho, stage flow with the caller's workspace on a stream */
    hipStream_t st;
    hip_ok(hipStreamCreate(&st), "stream");
    mfft_plan* q = NULL;
    mfft_ok(mfft_plan_create_ex(&q, N, B, MFFT_C2C, MFFT_INVERSE, MFFT_NORM_ORTHO, MFFT_FLOW_RADIX2_DIT, NULL, 0,
                                MFFT_PLAN_CALLER_WORKSPACE),
            "plan c2c caller workspace");
    int64_t wsb = 0;
    mfft_ok(mfft_plan_workspace_size(q, &wsb), "workspace size");
    if (wsb != (int64_t)(cplx * 8)) {
        printf("workspace size %lld, expected %lld\n", (long long)wsb, (long long)(cplx * 8));
        fails++;
    }
    if (mfft_execute(q, din, dout, st) != MFFT_ERR_VALUE) {
        printf("mfft_execute accepted a caller-workspace plan\n");
        fails++;
    }
    hip_ok(hipMalloc(&ws, (size_t)wsb), "hipMalloc workspace");
    mfft_ok(mfft_execute_ws(q, din, dout, ws, wsb, st), "execute_ws");
    hip_ok(hipStreamSynchronize(st), "stream sync");
    hip_ok(hipMemcpy(h_out, dout, cplx * 8, hipMemcpyDeviceToHost), "copy out");
    dft(d_in, d_ref, N, B, 1, 1.0 / sqrt((double)N));
    e = rel_l2(h_out, d_ref, cplx * 2);
    printf("c2c inverse ortho (radix-2, caller workspace, own stream): rel L2 %.3e\n", e);
    fails += !(e <= TOL);
    mfft_ok(mfft_plan_destroy(q), "destroy");
    hip_ok(hipStreamDestroy(st), "stream destroy");

    /* 3. r2c then c2r: the real parts of h_in as B rows of N reals */
    float* h_real = malloc((size_t)N * B * sizeof(float));
    float* h_back = malloc((size_t)N * B * sizeof(float));
    if (!h_real || !h_back) return 2;
    for (size_t i = 0; i < (size_t)N * B; ++i) h_real[i] = h_in[2 * i];
    hip_ok(hipMalloc(&dreal, (size_t)N * B * 4), "hipMalloc real");
    hip_ok(hipMemcpy(dreal, h_real, (size_t)N * B * 4, hipMemcpyHostToDevice), "copy real");
    mfft_plan *pr = NULL, *pc = NULL;
    mfft_ok(mfft_plan_create(&pr, N, B, MFFT_R2C, MFFT_FORWARD, MFFT_NORM_BACKWARD, MFFT_FLOW_AUTO, NULL, 0),
            "plan r2c");
    mfft_ok(mfft_plan_create(&pc, N, B, MFFT_C2R, MFFT_INVERSE, MFFT_NORM_BACKWARD, MFFT_FLOW_AUTO, NULL, 0),
            "plan c2r");
    mfft_ok(mfft_execute(pr, dreal, dout, NULL), "execute r2c");           /* dout: B x (N/2+1) bins */
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(h_out, dout, (size_t)B * (N / 2 + 1) * 8, hipMemcpyDeviceToHost), "copy bins");
    for (size_t i = 0; i < (size_t)N * B; ++i) {
        d_in[2 * i] = h_real[i];
        d_in[2 * i + 1] = 0.0;
    }
    dft(d_in, d_ref, N, B, -1, 1.0);
    double num = 0.0, den = 0.0;
    for (int r = 0; r < B; ++r)
        for (int k = 0; k <= N / 2; ++k)
            for (int c = 0; c < 2; ++c) {
                const double ref = d_ref[2 * ((size_t)r * N + k) + c];
                const double d = h_out[2 * ((size_t)r * (N / 2 + 1) + k) + c] - ref;
                num += d * d;
                den += ref * ref;
            }
    e = sqrt(num / den);
    printf("r2c forward (auto flow): rel L2 %.3e\n", e);
    fails += !(e <= TOL);
    mfft_ok(mfft_execute(pc, dout, din, NULL), "execute c2r");             /* din: B x N reals */
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(h_back, din, (size_t)N * B * 4, hipMemcpyDeviceToHost), "copy back");
    num = den = 0.0;
    for (size_t i = 0; i < (size_t)N * B; ++i) {
        const double d = (double)h_back[i] - h_real[i];
        num += d * d;
        den += (double)h_real[i] * h_real[i];
    }
    e = sqrt(num / den);
    printf("c2r(r2c(x)) round trip: rel L2 %.3e\n", e);
    fails += !(e <= TOL);
    mfft_ok(mfft_plan_destroy(pr), "destroy");
    mfft_ok(mfft_plan_destroy(pc), "destroy");

    /* 4. the standalone real epilogues around an N/2-point c2c core (d_ref
     * still holds the DFT of the real rows) */
    void *dz = NULL, *dbins = NULL, *du = NULL;
    hip_ok(hipMalloc(&dz, (size_t)B * (N / 2) * 8), "hipMalloc z");
    hip_ok(hipMalloc(&dbins, (size_t)B * (N / 2 + 1) * 8), "hipMalloc bins");
    hip_ok(hipMalloc(&du, (size_t)B * (N / 2) * 8), "hipMalloc u");
    mfft_plan* ph = NULL;
    mfft_ok(mfft_plan_create(&ph, N / 2, B, MFFT_C2C, MFFT_FORWARD, MFFT_NORM_NONE, MFFT_FLOW_AUTO, NULL, 0),
            "plan half core");
    mfft_ok(mfft_execute(ph, dreal, dz, NULL), "core of the packed reals");
    mfft_ok(mfft_r2c_stitch(dz, dbins, N, B, 1.0f, NULL), "r2c stitch");
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(h_out, dbins, (size_t)B * (N / 2 + 1) * 8, hipMemcpyDeviceToHost), "copy stitched bins");
    num = den = 0.0;
    for (int r = 0; r < B; ++r)
        for (int k = 0; k <= N / 2; ++k)
            for (int c = 0; c < 2; ++c) {
                const double ref = d_ref[2 * ((size_t)r * N + k) + c];
                const double d = h_out[2 * ((size_t)r * (N / 2 + 1) + k) + c] - ref;
                num += d * d;
                den += ref * ref;
            }
    e = sqrt(num / den);
    printf("core + mfft_r2c_stitch: rel L2 %.3e\n", e);
    fails += !(e <= TOL);
    mfft_ok(mfft_c2r_pre(dbins, dz, N, B, NULL), "c2r pre");
    mfft_ok(mfft_execute(ph, dz, du, NULL), "core of the pre-twiddled bins");
    mfft_ok(mfft_c2r_unpack(du, din, N, B, 2.0f / N, NULL), "c2r unpack");  /* din: B x N reals */
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(h_back, din, (size_t)N * B * 4, hipMemcpyDeviceToHost), "copy unpacked");
    num = den = 0.0;
    for (size_t i = 0; i < (size_t)N * B; ++i) {
        const double d = (double)h_back[i] - h_real[i];
        num += d * d;
        den += (double)h_real[i] * h_real[i];
    }
    e = sqrt(num / den);
    printf("mfft_c2r_pre + core + mfft_c2r_unpack round trip: rel L2 %.3e\n", e);
    fails += !(e <= TOL);
    if (mfft_r2c_stitch(dz, dz, N, B, 1.0f, NULL) != MFFT_ERR_VALUE) {
        printf("mfft_r2c_stitch accepted overlapping buffers\n");
        fails++;
    }
    mfft_ok(mfft_plan_destroy(ph), "destroy");
    hipFree(dz);
    hipFree(dbins);
    hipFree(du);

    hipFree(din);
    hipFree(dout);
    hipFree(ws);
    hipFree(dreal);
    free(h_in);
    free(h_out);
    free(d_in);
    free(d_ref);
    free(h_real);
    free(h_back);
    printf("%s\n", fails ? "FAIL" : "OK");
    return fails ? 1 : 0;
}
