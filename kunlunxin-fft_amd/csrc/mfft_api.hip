// mfft_api.hip -- the C ABI of include/mfft.h: plan creation (validation,
// twiddle tables, workspace), execution (kernel launches only) and queries.
//
// Validation mirrors the reference's contracts and happens before any device
// allocation: power-of-two lengths (validate.py:13-16 log2_exact), the
// direction lock of real transforms (entry.py:157-172), known enums
// (entry.py:136-156).  Twiddles are computed on the host in double and
// rounded once to float (the reference builds them per call in float32,
// runner.py:93-97; here they are built once per plan).
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "mfft_device.hpp"
#include "mfft_internal.hpp"

namespace mfft {
thread_local LaunchTimer* g_timer = nullptr;
}

// Scratch of mfft_execute_noalloc: one copy per device, held until the
// process ends.  Host code never uses this name as an address (on the host
// it is a stand-in, not device memory); it uses the per-device address that
// hipGetSymbolAddress returns (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[MFFT_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(MFFT_ERR_RUNTIME, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

int log2_exact(int64_t n) {
    if (n <= 0 || (n & (n - 1)) != 0) return -1;
    int b = 0;
    while (((int64_t)1 << b) != n) ++b;
    return b;
}

double norm_scale(int64_t n, int dir, int norm) {
    // entry.py:81-102
    if (norm == MFFT_NORM_ORTHO) return 1.0 / std::sqrt((double)n);
    if ((norm == MFFT_NORM_FORWARD && dir == MFFT_FORWARD) ||
        (norm == MFFT_NORM_BACKWARD && dir == MFFT_INVERSE))
        return 1.0 / (double)n;
    return 1.0;
}

// forward root exp(-2*pi*i*e/len), computed in long double and rounded once;
// exact values on the axes keep symmetric roots symmetric
float2 root(int64_t len, int64_t e) {
    e %= len;
    if (e == 0) return make_float2(1.0f, 0.0f);
    if (4 * e == len) return make_float2(0.0f, -1.0f);
    if (2 * e == len) return make_float2(-1.0f, 0.0f);
    if (4 * e == 3 * len) return make_float2(0.0f, 1.0f);
    const long double two_pi = 6.283185307179586476925286766559005768L;
    const long double a = -two_pi * (long double)e / (long double)len;
    return make_float2((float)cosl(a), (float)sinl(a));
}

// roots W_len^(m*step) for m in [0, count)
std::vector<float2> roots(int64_t len, int64_t count, int64_t step) {
    std::vector<float2> w((size_t)count);
    for (int64_t m = 0; m < count; ++m) w[m] = root(len, m * step);
    return w;
}

// Stockham pass table of a length-2^logl transform at 2^le elements per
// thread: pass p >= 1 (span NS, radix R) holds rows i < log2 R of
// W_{NS*R}^(2^i * k), k < NS, at offset sched_tw_off (mfft_device.hpp);
// rf: the remainder radix runs first.
std::vector<float2> pass_table(int logl, int le, bool rf = false) {
    const int passes = mfft::sched_passes(logl, le);
    const int size = mfft::sched_tw_size(logl, le, rf);
    std::vector<float2> t((size_t)(size > 0 ? size : 1), make_float2(0.0f, 0.0f));
    for (int p = 1; p < passes; ++p) {
        const int lr = mfft::sched_logr(logl, le, p, rf);
        const int64_t ns = (int64_t)1 << mfft::sched_lns_rf(logl, le, p, rf);
        const int64_t span = ns << lr;
        const int off = mfft::sched_tw_off(logl, le, p, rf);
        for (int i = 0; i < lr; ++i)
            for (int64_t k = 0; k < ns; ++k) t[(size_t)(off + i * ns + k)] = root(span, k << i);
    }
    return t;
}

// Plan uploads go through one private non-blocking stream per device, and
// plan creation waits for that stream alone: a plan created while other
// streams run kernels neither waits for them nor stalls them (a plain
// hipMemcpy would run on the legacy default stream and wait for every
// blocking stream's work).
constexpr int kMaxDevices = 64;
std::mutex g_upload_mu;
hipStream_t g_upload[kMaxDevices] = {};

int upload_stream(int dev, hipStream_t* out) {
    if (dev < 0 || dev >= kMaxDevices) return fail(MFFT_ERR_RUNTIME, "device %d beyond %d devices", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_upload_mu);
    if (!g_upload[dev]) {
        hipError_t e = hipStreamCreateWithFlags(&g_upload[dev], hipStreamNonBlocking);
        if (e != hipSuccess) {
            g_upload[dev] = nullptr;
            return hip_fail(e, "hipStreamCreateWithFlags(upload stream)");
        }
    }
    *out = g_upload[dev];
    return MFFT_OK;
}

// Allocates a device copy of `h` and enqueues the copy on `us`; the caller
// waits for `us` before the plan is handed out (`h` must live until then).
int upload(float2** dptr, const std::vector<float2>& h, int64_t* bytes, hipStream_t us) {
    const size_t nb = h.size() * sizeof(float2);
    hipError_t e = hipMalloc((void**)dptr, nb > 0 ? nb : sizeof(float2));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(twiddle table)");
    if (nb) {
        e = hipMemcpyAsync(*dptr, h.data(), nb, hipMemcpyHostToDevice, us);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(twiddle table)");
    }
    *bytes += (int64_t)nb;
    return MFFT_OK;
}

void release(mfft_plan* p) {
    float2** bufs[] = {&p->tw, &p->tw_n1, &p->tw_n2, &p->tw_lo,  &p->tw_hi,
                       &p->tw_real, &p->tw_ra, &p->tw_rb, &p->ws_a, &p->ws_b};
    for (float2** b : bufs) {
        if (*b) (void)hipFree(*b);
        *b = nullptr;
    }
    if (p->overrun) (void)hipFree(p->overrun);
    p->overrun = nullptr;
    if (p->ws_f) (void)hipFree(p->ws_f);
    p->ws_f = nullptr;
}

// Device address of `scratch` on device `dev` (current), looked up on the
// first call for that device and kept.
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

int noalloc_scratch(int dev, void** out) {
    if (dev < 0 || dev >= kMaxDevices) return fail(MFFT_ERR_RUNTIME, "device %d beyond %d devices", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(static scratch)");
        if (!ptr) return fail(MFFT_ERR_RUNTIME, "hipGetSymbolAddress(static scratch) returned NULL");
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return MFFT_OK;
}

bool is_stage_flow(int f) {
    return f == MFFT_FLOW_RADIX2_DIT || f == MFFT_FLOW_RADIX2_DIF || f == MFFT_FLOW_RADIX4_DIT ||
           f == MFFT_FLOW_RADIX4_DIF;
}

// Alignment of a caller workspace and of the ws_b offset inside it.
constexpr int64_t kWorkAlign = 256;

// The scratch of one execute: the plan's own, or carved out of a caller's
// workspace.
struct Work {
    float2* a;  // core-sized: the core output (r2c) or input (c2r) of a non-fused real flow
    float2* b;  // core-sized: stage-flow ping-pong
    char* f;    // the fused four-step schedule's counters and Z ring
};

// The three scratch regions of a workspace (or of the static noalloc buffer)
Work carve(const mfft_plan* p, char* w) {
    return Work{p->need_a ? (float2*)w : nullptr, p->need_b ? (float2*)(w + p->work_b_off) : nullptr,
                p->need_f ? w + p->work_f_off : nullptr};
}

// Enqueue the complex core of length p->core_n over `rows` rows.
int run_core(const mfft_plan* p, const float2* src, float2* dst, int dir, float scale, const Work& w,
             hipStream_t stream) {
    hipError_t e = hipSuccess;
    int launches = 0;
    switch (p->flow) {
        case MFFT_FLOW_RADIX2_DIT:
        case MFFT_FLOW_RADIX2_DIF:
            e = mfft::launch_radix2(p->flow == MFFT_FLOW_RADIX2_DIF, dir, src, dst, w.b, p->tw,
                                    p->core_n, p->batch, scale, p->block, stream, &launches);
            break;
        case MFFT_FLOW_RADIX4_DIT:
        case MFFT_FLOW_RADIX4_DIF:
            e = mfft::launch_radix4(p->flow == MFFT_FLOW_RADIX4_DIF, dir, src, dst, w.b, p->tw,
                                    p->core_n, p->batch, scale, p->block, stream, &launches);
            break;
        case MFFT_FLOW_LDS_FUSED:
            e = mfft::launch_lds(0, dir, mfft::ilog2((int)p->core_n), p->elems, src, dst, p->tw, nullptr,
                                 p->batch, scale, stream, p->num_cus, p->stagger, p->staged);
            break;
        case MFFT_FLOW_FOUR_STEP:
            e = mfft::launch_fourstep(dir, src, dst, w.f, p, p->batch, scale, stream, &launches);
            break;
        case MFFT_FLOW_DENSE_MFMA:
            e = mfft::launch_mfma(dir, mfft::ilog2((int)p->core_n), src, dst, p->tw, p->batch, scale, stream);
            break;
        default:
            return fail(MFFT_ERR_VALUE, "internal: unknown flow %d", p->flow);
    }
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return MFFT_OK;
}

// A real transform over a four-step core whose batch is split into chunks:
// its stitch or pre-twiddle runs chunk by chunk between the core's chunks.
bool real_chunked(const mfft_plan* p) {
    return p->flow == MFFT_FLOW_FOUR_STEP && p->schedule != 2 && p->chunk_rows > 0 && p->chunk_rows < p->batch;
}

// One execute with the scratch `w`; ws/ws_bytes: the caller's workspace
// (checked against in and out), or NULL for the plan's own.
int execute_impl(const mfft_plan* p, const void* in, void* out, const Work& w, void* stream_v,
                 const void* ws = nullptr, int64_t ws_bytes = 0) {
    if (!in || !out) return fail(MFFT_ERR_VALUE, "in and out must not be NULL");
    const size_t in_bytes = (size_t)p->batch *
        (p->transform_type == MFFT_R2C ? (size_t)p->n * 4
         : p->transform_type == MFFT_C2R ? (size_t)(p->n / 2 + 1) * 8 : (size_t)p->n * 8);
    const size_t out_bytes = (size_t)p->batch *
        (p->transform_type == MFFT_R2C ? (size_t)(p->n / 2 + 1) * 8
         : p->transform_type == MFFT_C2R ? (size_t)p->n * 4 : (size_t)p->n * 8);
    const char* ib = (const char*)in;
    const char* ob = (const char*)out;
    if (ib < ob + out_bytes && ob < ib + in_bytes)
        return fail(MFFT_ERR_VALUE, "in and out must not overlap");
    if (ws) {
        const char* wb = (const char*)ws;
        if ((wb < ib + in_bytes && ib < wb + ws_bytes) || (wb < ob + out_bytes && ob < wb + ws_bytes))
            return fail(MFFT_ERR_VALUE, "the workspace must not overlap in or out");
    }
    if ((((uintptr_t)in) & 7) && p->transform_type != MFFT_R2C)
        return fail(MFFT_ERR_VALUE, "complex input must be 8-byte aligned");
    if ((((uintptr_t)in) & 7) && p->transform_type == MFFT_R2C)
        return fail(MFFT_ERR_VALUE, "r2c input must be 8-byte aligned (pairs are read as complex)");
    if (((uintptr_t)out) & 7) return fail(MFFT_ERR_VALUE, "output must be 8-byte aligned");
    int dev = -1;
    hipError_t he = hipGetDevice(&dev);
    if (he != hipSuccess) return hip_fail(he, "hipGetDevice");
    if (dev != p->device)
        return fail(MFFT_ERR_RUNTIME, "plan was created on device %d but device %d is current", p->device, dev);
    hipStream_t stream = (hipStream_t)stream_v;
    const int dir = p->transform_direction == MFFT_FORWARD ? -1 : 1;

    if (p->transform_type == MFFT_C2C)
        return run_core(p, (const float2*)in, (float2*)out, dir, p->scale, w, stream);

    const int logc = mfft::ilog2((int)p->core_n);
    if (p->transform_type == MFFT_R2C) {
        if (p->r2c_fused) {
            he = mfft::launch_lds(1, -1, logc, p->elems, in, out, p->tw, p->tw_real, p->batch, p->scale, stream,
                                  p->num_cus, p->stagger, p->staged);
            return he == hipSuccess ? MFFT_OK : hip_fail(he, "kernel launch");
        }
        if (p->real4_fused) {
            he = mfft::launch_fourstep_real((const float2*)in, (float2*)out, w.a, p, p->scale, stream);
            return he == hipSuccess ? MFFT_OK : hip_fail(he, "kernel launch");
        }
        if (real_chunked(p)) {
            // chunk by chunk: the stitch reads the core output of its chunk
            // while that is still in the MALL
            const int64_t cn = p->core_n;
            for (int64_t r0 = 0; r0 < p->batch; r0 += p->chunk_rows) {
                const int64_t rc = p->batch - r0 < p->chunk_rows ? p->batch - r0 : p->chunk_rows;
                he = mfft::launch_fourstep(-1, (const float2*)in + r0 * cn, w.a + r0 * cn, nullptr, p, rc, 1.0f,
                                           stream, nullptr);
                if (he == hipSuccess)
                    he = mfft::launch_r2c_stitch(w.a + r0 * cn, (float2*)out + r0 * (cn + 1), p->tw_real, p->n, rc,
                                                 p->scale, stream);
                if (he != hipSuccess) return hip_fail(he, "kernel launch");
            }
            return MFFT_OK;
        }
        int rc = run_core(p, (const float2*)in, w.a, -1, 1.0f, w, stream);
        if (rc != MFFT_OK) return rc;
        he = mfft::launch_r2c_stitch(w.a, (float2*)out, p->tw_real, p->n, p->batch, p->scale, stream);
        return he == hipSuccess ? MFFT_OK : hip_fail(he, "kernel launch");
    }
    // c2r
    if (p->c2r_fused) {
        he = mfft::launch_lds(2, 1, logc, p->elems, in, out, p->tw, p->tw_real, p->batch, p->scale, stream,
                              p->num_cus, p->stagger, p->staged);
        return he == hipSuccess ? MFFT_OK : hip_fail(he, "kernel launch");
    }
    if (p->real4_fused) {
        he = mfft::launch_fourstep_real((const float2*)in, (float2*)out, nullptr, p, p->scale, stream);
        return he == hipSuccess ? MFFT_OK : hip_fail(he, "kernel launch");
    }
    if (real_chunked(p)) {
        // chunk by chunk: pass 1 reads the pre-twiddled chunk while that is
        // still in the MALL
        const int64_t cn = p->core_n;
        for (int64_t r0 = 0; r0 < p->batch; r0 += p->chunk_rows) {
            const int64_t rc = p->batch - r0 < p->chunk_rows ? p->batch - r0 : p->chunk_rows;
            he = mfft::launch_c2r_pre((const float2*)in + r0 * (cn + 1), w.a + r0 * cn, p->tw_real, p->n, rc, stream);
            if (he == hipSuccess)
                he = mfft::launch_fourstep(1, w.a + r0 * cn, (float2*)out + r0 * cn, nullptr, p, rc, p->scale,
                                           stream, nullptr);
            if (he != hipSuccess) return hip_fail(he, "kernel launch");
        }
        return MFFT_OK;
    }
    he = mfft::launch_c2r_pre((const float2*)in, w.a, p->tw_real, p->n, p->batch, stream);
    if (he != hipSuccess) return hip_fail(he, "kernel launch");
    return run_core(p, w.a, (float2*)out, 1, p->scale, w, stream);
}

}  // namespace

extern "C" {

int mfft_abi_version(void) { return MFFT_ABI_VERSION; }

const char* mfft_last_error(void) { return g_err.c_str(); }

int mfft_plan_create(mfft_plan** out, int64_t n, int64_t batch, int transform_type,
                     int transform_direction, int norm, int flow, const int32_t* params, int nparams) {
    return mfft_plan_create_ex(out, n, batch, transform_type, transform_direction, norm, flow, params, nparams, 0);
}

int mfft_plan_create_ex(mfft_plan** out, int64_t n, int64_t batch, int transform_type, int transform_direction,
                        int norm, int flow, const int32_t* params, int nparams, int flags) {
    g_err.clear();
    if (!out) return fail(MFFT_ERR_VALUE, "out must not be NULL");
    *out = nullptr;
    if (flags & ~MFFT_PLAN_CALLER_WORKSPACE) return fail(MFFT_ERR_VALUE, "unknown plan flags 0x%x", flags);
    if (transform_type < MFFT_C2C || transform_type > MFFT_C2R)
        return fail(MFFT_ERR_VALUE, "unsupported transform_type %d", transform_type);
    if (transform_direction != MFFT_FORWARD && transform_direction != MFFT_INVERSE)
        return fail(MFFT_ERR_VALUE, "unsupported transform_direction %d", transform_direction);
    if (norm < MFFT_NORM_NONE || norm > MFFT_NORM_ORTHO) return fail(MFFT_ERR_VALUE, "unsupported norm %d", norm);
    if (transform_type == MFFT_R2C && transform_direction != MFFT_FORWARD)
        return fail(MFFT_ERR_VALUE, "r2c is a forward transform");
    if (transform_type == MFFT_C2R && transform_direction != MFFT_INVERSE)
        return fail(MFFT_ERR_VALUE, "c2r is an inverse transform");
    const int logn = log2_exact(n);
    if (logn < 0) return fail(MFFT_ERR_VALUE, "size must be a positive power of two, got %lld", (long long)n);
    if (logn > mfft::kMaxLog2N)
        return fail(MFFT_ERR_VALUE, "n=%lld exceeds the supported maximum 2^%d", (long long)n, mfft::kMaxLog2N);
    if (transform_type != MFFT_C2C && n < 2)
        return fail(MFFT_ERR_VALUE, "real transforms need n >= 2, got %lld", (long long)n);
    if (batch < 1) return fail(MFFT_ERR_VALUE, "batch must be >= 1, got %lld", (long long)batch);
    // at most 2^40 bytes of complex64 rows (above any GPU's memory): keeps
    // every byte count in range and every grid below 2^31 blocks
    if (batch > ((int64_t)1 << 37) / n)
        return fail(MFFT_ERR_VALUE, "batch=%lld of n=%lld exceeds 2^40 bytes of complex64 rows", (long long)batch,
                    (long long)n);
    if (nparams < 0 || nparams > MFFT_MAX_PARAMS || (nparams > 0 && !params))
        return fail(MFFT_ERR_VALUE, "bad params (nparams=%d)", nparams);
    int32_t prm[MFFT_MAX_PARAMS] = {0, 0, 0, 0};
    for (int i = 0; i < nparams; ++i) prm[i] = params[i];
    for (int i = 0; i < MFFT_MAX_PARAMS; ++i)
        if (prm[i] < 0) return fail(MFFT_ERR_VALUE, "params[%d]=%d must be >= 0", i, prm[i]);

    const bool real = transform_type != MFFT_C2C;
    const int64_t core_n = real ? n / 2 : n;
    const int logc = log2_exact(core_n);
    const int dir = transform_direction == MFFT_FORWARD ? -1 : 1;

    // ---- resolve and check the flow
    if (flow == MFFT_FLOW_AUTO)
        flow = mfft::lds_supported(logc, 0) ? MFFT_FLOW_LDS_FUSED : MFFT_FLOW_FOUR_STEP;
    int block = 256, elems = 0, stagger = 0;
    bool staged = false;
    int64_t n1 = 0, n2 = 0, chunk = 0;
    int schedule = 0, pass2_rev = 0, fused_lag = 0, fused_take = 0, fused_ring = 0, fused_bpc = 0;
    switch (flow) {
        case MFFT_FLOW_RADIX2_DIT:
        case MFFT_FLOW_RADIX2_DIF:
        case MFFT_FLOW_RADIX4_DIT:
        case MFFT_FLOW_RADIX4_DIF: {
            const int min_log = (flow == MFFT_FLOW_RADIX4_DIT || flow == MFFT_FLOW_RADIX4_DIF) ? 2 : 1;
            if (logc < min_log)
                return fail(MFFT_ERR_UNSUPPORTED, "flow %d needs a core length >= %d, got %lld", flow,
                            1 << min_log, (long long)core_n);
            if (prm[0]) {
                const int lb = log2_exact(prm[0]);
                if (lb < 6 || lb > 10)
                    return fail(MFFT_ERR_VALUE, "threads per block %d must be a power of two in [64, 1024]", prm[0]);
                block = prm[0];
            }
            break;
        }
        case MFFT_FLOW_LDS_FUSED:
            if (!mfft::lds_supported(logc, prm[0]))
                return fail(MFFT_ERR_UNSUPPORTED,
                            "LDS_FUSED runs core lengths up to 2^%d with 4, 8, 16 or 32 "
                            "elements per thread (32 from 2^10; 2^13, 2^14: 16 or 32; 2^15: 32) "
                            "(got core length %lld, elements %d)",
                            mfft::kMaxLdsLog2, (long long)core_n, prm[0]);
            elems = prm[0] ? prm[0] : mfft::lds_default_elems(logc);
            block = mfft::lds_threads_per_block(logc, elems);
            if (prm[1] > mfft::kMaxStagger)
                return fail(MFFT_ERR_VALUE, "LDS_FUSED start stagger params[1]=%d exceeds %d", prm[1],
                            mfft::kMaxStagger);
            stagger = prm[1];
            if (prm[2] > 1)
                return fail(MFFT_ERR_VALUE, "LDS_FUSED staged form params[2] must be 0 or 1, got %d", prm[2]);
            if (prm[2] && !mfft::lds_staged_supported(logc, elems))
                return fail(MFFT_ERR_UNSUPPORTED,
                            "the staged LDS_FUSED form (params[2] = 1) runs transforms of fewer than 16 "
                            "threads (core length / elements per thread < 16; got core length %lld, "
                            "elements %d)",
                            (long long)core_n, elems);
            staged = prm[2] != 0;
            break;
        case MFFT_FLOW_FOUR_STEP: {
            int l1, l2;
            mfft::fourstep_default_split(logc, &l1, &l2);
            if (prm[0]) {
                l1 = log2_exact(prm[0]);
                if (l1 < 0) return fail(MFFT_ERR_VALUE, "n1=%d must be a power of two", prm[0]);
                l2 = logc - l1;
            }
            if (logc < mfft::kMinFourStepLog2 || !mfft::fourstep_supported(l1, l2))
                return fail(MFFT_ERR_UNSUPPORTED,
                            "FOUR_STEP needs core length 2^8..2^20 split into n1, n2 in [16, 1024] "
                            "(got core length %lld, n1=2^%d)",
                            (long long)core_n, l1);
            n1 = (int64_t)1 << l1;
            n2 = (int64_t)1 << l2;
            chunk = prm[1] > 0 ? prm[1] : 0;
            if (prm[2] < 0 || prm[2] > 3)
                return fail(MFFT_ERR_VALUE, "FOUR_STEP schedule must be 0, 1, 2 or 3, got %d", prm[2]);
            schedule = prm[2];
            if (schedule != 2 && (prm[3] < 0 || prm[3] > 1))
                return fail(MFFT_ERR_VALUE, "FOUR_STEP pass-2 row order must be 0 or 1, got %d", prm[3]);
            if (schedule == 2 && (prm[3] & 0xff) >= mfft::kFusedMaxRing)
                return fail(MFFT_ERR_VALUE, "FOUR_STEP fused queue lag (params[3] bits 0-7) must be in [0, %d], got %d",
                            mfft::kFusedMaxRing - 1, prm[3] & 0xff);
            if (schedule == 2 && ((prm[3] >> 8) & 0xff) > 64)
                return fail(MFFT_ERR_VALUE,
                            "FOUR_STEP fused items per dequeue (params[3] bits 8-15) must be in [0, 64], got %d",
                            (prm[3] >> 8) & 0xff);
            if (schedule == 2 && ((prm[3] >> 16) & 0xff) > mfft::kFusedMaxRing)
                return fail(MFFT_ERR_VALUE,
                            "FOUR_STEP fused Z slots per XCD (params[3] bits 16-23) must be in [0, %d], got %d",
                            mfft::kFusedMaxRing, (prm[3] >> 16) & 0xff);
            if (schedule == 2 && (prm[3] >> 24) > 16)
                return fail(MFFT_ERR_VALUE,
                            "FOUR_STEP fused blocks per CU (params[3] bits 24-30) must be in [0, 16], got %d",
                            prm[3] >> 24);
            pass2_rev = schedule == 2 ? 0 : prm[3];
            fused_lag = schedule == 2 ? (prm[3] & 0xff) : 0;
            fused_take = schedule == 2 ? ((prm[3] >> 8) & 0xff) : 0;
            fused_ring = schedule == 2 ? ((prm[3] >> 16) & 0xff) : 0;
            fused_bpc = schedule == 2 ? (prm[3] >> 24) : 0;
            if (schedule == 2 && !mfft::fourstep_fused_supported(l1, l2))
                return fail(MFFT_ERR_UNSUPPORTED,
                            "the fused FOUR_STEP schedule needs n1, n2 in [128, 512] within a factor 2 "
                            "(got 2^%d x 2^%d)",
                            l1, l2);
            if (schedule == 2 && !mfft::kFusedScheduleEnabled)
                return fail(MFFT_ERR_UNSUPPORTED,
                            "the fused FOUR_STEP schedule (params[2] = 2) is disabled in this build");
            break;
        }
        case MFFT_FLOW_DENSE_MFMA:
            if (!mfft::mfma_supported(logc))
                return fail(MFFT_ERR_UNSUPPORTED, "DENSE_MFMA runs core lengths 2..2^%d (got core length %lld)",
                            mfft::kMaxMfmaLog2, (long long)core_n);
            block = core_n > 4096 ? (int)(core_n / 16) : 256;  // threads per block of the kernel
            break;
        default:
            return fail(MFFT_ERR_VALUE, "unknown flow id %d", flow);
    }

    // ---- every launch of the plan must fit one dispatch: an upper bound on
    // the work-items of its largest launch, from each flow's threads per
    // transform (checked again at every launch)
    {
        int64_t items = 0;
        auto most = [&](int64_t v) { items = v > items ? v : items; };
        switch (flow) {
            case MFFT_FLOW_LDS_FUSED: {
                const int e = elems ? elems : mfft::lds_default_elems(logc);
                const int64_t t = core_n / e > 0 ? core_n / e : 1;  // threads per transform
                most(batch * t + 1024);
                break;
            }
            case MFFT_FLOW_FOUR_STEP: {
                const int e1 = 1 << mfft::fourstep_col_loge(mfft::ilog2((int)n1), schedule);
                const int e2 = 1 << mfft::fourstep_col_loge(mfft::ilog2((int)n2), schedule);
                most(batch * (core_n / (e1 < e2 ? e1 : e2)) + 1024);
                break;
            }
            case MFFT_FLOW_DENSE_MFMA:
                most((batch * core_n + 15) / 16 + 4096);  // L/16 threads per transform
                break;
            default:  // stage flows: radix-2 stages (also the radix-4 flows' odd tail)
                most(batch * (core_n >> 1) + block);
        }
        // a real transform whose core does not carry the stitch / pre-twiddle
        // runs it as its own launch: one thread per mirror pair, core/2 + 1
        // a row, over the flat batch
        const bool real_fused = flow == MFFT_FLOW_LDS_FUSED || (flow == MFFT_FLOW_FOUR_STEP && schedule == 0);
        if (real && !real_fused) most(batch * ((core_n >> 1) + 1) + 256);
        if (items > mfft::kMaxLaunchItems)
            return fail(MFFT_ERR_UNSUPPORTED,
                        "batch=%lld of n=%lld: a launch of this flow would run %lld work-items, above the "
                        "%lld one dispatch holds; split the batch",
                        (long long)batch, (long long)n, (long long)items, (long long)mfft::kMaxLaunchItems);
    }

    int dev = 0;
    hipError_t he = hipGetDevice(&dev);
    if (he != hipSuccess) return hip_fail(he, "hipGetDevice");
    int num_cus = 0;
    he = hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (he != hipSuccess) return hip_fail(he, "hipDeviceGetAttribute(MultiprocessorCount)");
    int clock_khz = 0;
    he = hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, dev);
    if (he != hipSuccess) return hip_fail(he, "hipDeviceGetAttribute(WallClockRate)");
    int num_xcc = 0;
    he = hipDeviceGetAttribute(&num_xcc, hipDeviceAttributeNumberOfXccs, dev);
    if (he != hipSuccess) return hip_fail(he, "hipDeviceGetAttribute(NumberOfXccs)");
    if (schedule == 2 && (num_xcc < 1 || num_xcc > mfft::kFusedSlots))
        return fail(MFFT_ERR_UNSUPPORTED, "the fused FOUR_STEP schedule needs 1..%d XCDs (device reports %d)",
                    mfft::kFusedSlots, num_xcc);
    int fused_grid = 0;
    if (schedule == 2) {
        // one resident wave of blocks (at most fused_bpc per CU), a multiple
        // of the XCD count: blocks go to the XCDs round-robin, so every XCD,
        // and every queue, gets blocks
        const int l1 = mfft::ilog2((int)n1), l2 = mfft::ilog2((int)n2);
        int per_cu = mfft::fourstep_fused_occupancy(l1, l2);
        if (per_cu < 1) return fail(MFFT_ERR_RUNTIME, "occupancy query of the fused four-step kernel failed");
        if (fused_bpc > 0 && fused_bpc < per_cu) per_cu = fused_bpc;
        const int nx = num_xcc, cus = num_cus > 0 ? num_cus : 1;
        fused_grid = (per_cu * cus) / nx * nx;
        if (fused_grid < nx) fused_grid = nx;
        // defaults, the fastest of the measured settings at 2^16..2^18: one
        // item per dequeue; pass 1 one transform more ahead of pass 2 than
        // the blocks of one XCD hold items (wt transforms of G1 + G2 items),
        // so pass 2 rarely waits for Z; and wt slots more than that, so pass 1
        // rarely waits for its slot
        if (fused_take == 0) fused_take = 1;
        const int items = (int)((n2 >> 4) + (n1 >> 4));
        const int wt = (fused_grid / nx * fused_take + items - 1) / items;
        if (fused_lag == 0) fused_lag = wt + 1;
        if (fused_lag >= mfft::kFusedMaxRing) fused_lag = mfft::kFusedMaxRing - 1;
        // a ring slot is rewritten by pass 1 of transform k + R only after
        // pass 2 of k has read it; R >= lag + 1 keeps that wait on a
        // transform the queue handed out earlier
        if (fused_ring == 0) fused_ring = fused_lag + 1 + wt;
        if (fused_ring > mfft::kFusedMaxRing) fused_ring = mfft::kFusedMaxRing;
        if (fused_ring < fused_lag + 1 || fused_ring > mfft::kFusedMaxRing)
            return fail(MFFT_ERR_VALUE, "FOUR_STEP fused Z slots per XCD (%d) must be in [lag + 1 = %d, %d]",
                        fused_ring, fused_lag + 1, mfft::kFusedMaxRing);
    }

    mfft_plan* p = new (std::nothrow) mfft_plan();
    if (!p) return fail(MFFT_ERR_RUNTIME, "out of host memory");
    p->n = n;
    p->batch = batch;
    p->core_n = core_n;
    p->transform_type = transform_type;
    p->transform_direction = transform_direction;
    p->norm = norm;
    p->flow = flow;
    p->device = dev;
    p->block = block;
    p->elems = elems;
    p->stagger = stagger;
    p->staged = staged;
    p->n1 = n1;
    p->n2 = n2;
    p->chunk_rows = chunk;
    p->schedule = schedule;
    p->pass2_rev = pass2_rev;
    p->fused_lag = fused_lag;
    p->fused_take = fused_take;
    p->fused_ring = fused_ring;
    p->fused_grid = fused_grid;
    p->num_cus = num_cus > 0 ? num_cus : 1;
    p->clock_khz = clock_khz > 0 ? clock_khz : 100000;
    p->num_xcc = num_xcc > 0 ? num_xcc : 1;
    p->r2c_fused = transform_type == MFFT_R2C && flow == MFFT_FLOW_LDS_FUSED;
    p->c2r_fused = transform_type == MFFT_C2R && flow == MFFT_FLOW_LDS_FUSED;
    // the stitch / pre-twiddle run inside the four-step passes (one column
    // group per workgroup); the persistent and fused schedules keep them as
    // a separate pass around the core
    p->real4_fused = real && flow == MFFT_FLOW_FOUR_STEP && schedule == 0;
    // c2r: the half-length inverse core carries a factor 2 (entry.py:583-587)
    const double sc = norm_scale(n, transform_direction, norm) * (transform_type == MFFT_C2R ? 2.0 : 1.0);
    p->scale = (float)sc;

    hipStream_t us = nullptr;
    int rc = upload_stream(dev, &us);
    // ---- twiddle tables (host copies live until the upload stream is drained)
    std::vector<std::vector<float2>> host;
    auto put = [&](float2** d, std::vector<float2>&& h) {
        host.push_back(std::move(h));
        return upload(d, host.back(), &p->table_bytes, us);
    };
    host.reserve(7);
    if (rc == MFFT_OK && flow == MFFT_FLOW_FOUR_STEP) {
        const int lc = logc;
        const int l1 = mfft::ilog2((int)n1), l2 = mfft::ilog2((int)n2);
        p->tw_h = (lc + 1) / 2;
        if (rc == MFFT_OK) rc = put(&p->tw_n1, pass_table(l1, mfft::fourstep_col_loge(l1, schedule)));
        if (rc == MFFT_OK) rc = put(&p->tw_n2, pass_table(l2, mfft::fourstep_col_loge(l2, schedule)));
        if (rc == MFFT_OK) rc = put(&p->tw_lo, roots(core_n, (int64_t)1 << p->tw_h, 1));
        if (rc == MFFT_OK) rc = put(&p->tw_hi, roots(core_n, core_n >> p->tw_h, (int64_t)1 << p->tw_h));
    } else if (rc == MFFT_OK && flow == MFFT_FLOW_LDS_FUSED) {
        const int le = mfft::sched_le(logc, mfft::ilog2(elems));
        rc = put(&p->tw, pass_table(logc, le, mfft::lds_remainder_first(logc, le, p->r2c_fused)));
    } else if (rc == MFFT_OK) {
        rc = put(&p->tw, roots(core_n, core_n, 1));
    }
    if (rc == MFFT_OK && real && !p->real4_fused) {
        // exp(-2*pi*i*k/n), k in [0, n/2]  (runner.py:1650-1658 range); the
        // fused real four-step takes its bin roots from the two small tables
        // below instead (this one would be 4 MiB at n = 2^20)
        rc = put(&p->tw_real, roots(n, n / 2 + 1, 1));
    }
    if (rc == MFFT_OK && p->real4_fused) {
        // bin roots exp(-2 pi i k / n) as the product of two small tables:
        // r2c k = k1 + n1 k2 (pass 2 grid), c2r k = n1 n2_len + n2 (pass 1 grid)
        if (transform_type == MFFT_R2C) {
            rc = put(&p->tw_ra, roots(n, n1, 1));
            if (rc == MFFT_OK) rc = put(&p->tw_rb, roots(n, n2 + 1, n1));
        } else {
            rc = put(&p->tw_ra, roots(n, n2, 1));
            if (rc == MFFT_OK) rc = put(&p->tw_rb, roots(n, n1, n2));
        }
    }

    // ---- workspace
    const size_t core_bytes = (size_t)batch * (size_t)core_n * sizeof(float2);
    // the core output (r2c) / input (c2r) of a real flow that does not fuse
    // both ends; the fused real four-step keeps only r2c's permuted Z there
    const bool need_a = real && !(p->r2c_fused || p->c2r_fused) && !(p->real4_fused && transform_type == MFFT_C2R);
    const bool need_b = is_stage_flow(flow);
    const bool need_f = flow == MFFT_FLOW_FOUR_STEP && schedule == 2;
    auto align = [](int64_t x) { return (x + kWorkAlign - 1) / kWorkAlign * kWorkAlign; };
    p->need_a = need_a;
    p->need_b = need_b;
    p->need_f = need_f;
    p->core_bytes = (int64_t)core_bytes;
    p->work_b_off = need_a ? align(p->core_bytes) : 0;
    const int64_t end_ab = need_b ? p->work_b_off + p->core_bytes : (need_a ? p->core_bytes : 0);
    if (need_f) {
        // counters of one launch (a chunk, or the batch), then num_xcc x
        // fused_ring Z slots of one transform each
        const int64_t rows = chunk > 0 && chunk < batch ? chunk : batch;
        p->fused_ring_off = align((int64_t)(mfft::kFusedHead + 2 * rows) * (int64_t)sizeof(int));
        p->fused_bytes = p->fused_ring_off + (int64_t)p->num_xcc * fused_ring * core_n * (int64_t)sizeof(float2);
        p->work_f_off = align(end_ab);
        p->work_bytes = p->work_f_off + p->fused_bytes;
    } else {
        p->work_bytes = end_ab;
    }
    p->caller_ws = (flags & MFFT_PLAN_CALLER_WORKSPACE) != 0;
    if (rc == MFFT_OK && need_a && !p->caller_ws) {
        he = hipMalloc((void**)&p->ws_a, core_bytes);
        if (he != hipSuccess) rc = hip_fail(he, "hipMalloc(workspace)");
        else p->ws_bytes += (int64_t)core_bytes;
    }
    if (rc == MFFT_OK && need_b && !p->caller_ws) {
        he = hipMalloc((void**)&p->ws_b, core_bytes);
        if (he != hipSuccess) rc = hip_fail(he, "hipMalloc(workspace)");
        else p->ws_bytes += (int64_t)core_bytes;
    }
    if (rc == MFFT_OK && need_f && !p->caller_ws) {
        he = hipMalloc((void**)&p->ws_f, (size_t)p->fused_bytes);
        if (he != hipSuccess) rc = hip_fail(he, "hipMalloc(four-step Z ring)");
        else p->ws_bytes += p->fused_bytes;
    }
    if (rc == MFFT_OK && need_f) {
        // the plan's count of fused-schedule waits that gave up (all launches)
        he = hipMalloc((void**)&p->overrun, sizeof(int));
        if (he == hipSuccess) he = hipMemsetAsync(p->overrun, 0, sizeof(int), us);
        if (he != hipSuccess) rc = hip_fail(he, "hipMalloc(four-step overrun count)");
        else p->ws_bytes += (int64_t)sizeof(int);
    }

    // ---- launch count (per execute)
    int core_launches = 0;
    switch (flow) {
        case MFFT_FLOW_RADIX2_DIT:
        case MFFT_FLOW_RADIX2_DIF: core_launches = logc; break;
        case MFFT_FLOW_RADIX4_DIT:
        case MFFT_FLOW_RADIX4_DIF: core_launches = logc / 2 + (logc & 1); break;
        case MFFT_FLOW_LDS_FUSED:
        case MFFT_FLOW_DENSE_MFMA: core_launches = 1; break;
        case MFFT_FLOW_FOUR_STEP: {
            const int64_t ch = chunk > 0 ? chunk : batch;
            const int64_t nc = (batch + ch - 1) / ch;
            core_launches = (int)(2 * nc);
            break;
        }
    }
    // the stitch / pre-twiddle of a non-fused real flow: once, or once per
    // chunk of a chunked four-step core
    const int64_t real_launches = (!need_a || p->real4_fused) ? 0 : real_chunked(p) ? (batch + chunk - 1) / chunk : 1;
    p->launches = core_launches + (int)real_launches;

    // the uploads are complete before the plan is handed out (and before the
    // host copies go); an error return still drains the stream first
    if (us) {
        he = hipStreamSynchronize(us);
        if (he != hipSuccess && rc == MFFT_OK) rc = hip_fail(he, "hipStreamSynchronize(upload stream)");
    }
    if (rc != MFFT_OK) {
        release(p);
        delete p;
        return rc;
    }
    (void)dir;
    *out = p;
    return MFFT_OK;
}

int mfft_execute(const mfft_plan* p, const void* in, void* out, void* stream_v) {
    g_err.clear();
    if (!p) return fail(MFFT_ERR_VALUE, "plan must not be NULL");
    if (p->caller_ws && p->work_bytes > 0)
        return fail(MFFT_ERR_VALUE,
                    "the plan was created with MFFT_PLAN_CALLER_WORKSPACE and needs %lld bytes of workspace: "
                    "use mfft_execute_ws",
                    (long long)p->work_bytes);
    return execute_impl(p, in, out, Work{p->ws_a, p->ws_b, p->ws_f}, stream_v);
}

int mfft_plan_workspace_size(const mfft_plan* p, int64_t* bytes) {
    g_err.clear();
    if (!p || !bytes) return fail(MFFT_ERR_VALUE, "plan and bytes must not be NULL");
    *bytes = p->work_bytes;
    return MFFT_OK;
}

int mfft_execute_ws(const mfft_plan* p, const void* in, void* out, void* workspace, int64_t workspace_bytes,
                    void* stream_v) {
    g_err.clear();
    if (!p) return fail(MFFT_ERR_VALUE, "plan must not be NULL");
    if (workspace_bytes < 0) return fail(MFFT_ERR_VALUE, "workspace_bytes must be >= 0");
    if (p->work_bytes == 0) return execute_impl(p, in, out, Work{nullptr, nullptr, nullptr}, stream_v);
    if (!workspace) return fail(MFFT_ERR_VALUE, "this plan needs %lld bytes of workspace", (long long)p->work_bytes);
    if (workspace_bytes < p->work_bytes)
        return fail(MFFT_ERR_VALUE, "workspace of %lld bytes is smaller than the plan's %lld",
                    (long long)workspace_bytes, (long long)p->work_bytes);
    if (((uintptr_t)workspace) % kWorkAlign)
        return fail(MFFT_ERR_VALUE, "workspace must be %d-byte aligned", (int)kWorkAlign);
    return execute_impl(p, in, out, carve(p, (char*)workspace), stream_v, workspace, p->work_bytes);
}

int mfft_execute_noalloc(const mfft_plan* p, const void* in, void* out, void* stream_v) {
    g_err.clear();
    if (!p) return fail(MFFT_ERR_VALUE, "plan must not be NULL");
    if (p->work_bytes > MFFT_NOALLOC_SCRATCH_BYTES)
        return fail(MFFT_ERR_VALUE,
                    "this plan needs %lld bytes of scratch, more than the %lld-byte static buffer of "
                    "mfft_execute_noalloc: use mfft_execute or mfft_execute_ws",
                    (long long)p->work_bytes, (long long)MFFT_NOALLOC_SCRATCH_BYTES);
    if (p->work_bytes == 0) return execute_impl(p, in, out, Work{nullptr, nullptr, nullptr}, stream_v);
    int dev = -1;
    const hipError_t he = hipGetDevice(&dev);
    if (he != hipSuccess) return hip_fail(he, "hipGetDevice");
    if (dev != p->device)
        return fail(MFFT_ERR_RUNTIME, "plan was created on device %d but device %d is current", p->device, dev);
    void* ws = nullptr;
    const int rc = noalloc_scratch(dev, &ws);
    if (rc != MFFT_OK) return rc;
    return execute_impl(p, in, out, carve(p, (char*)ws), stream_v, ws, p->work_bytes);
}

int mfft_execute_timed(const mfft_plan* p, const void* in, void* out, void* workspace, int64_t workspace_bytes,
                       void* stream_v, float* launch_ms, int cap, int* n_launches) {
    g_err.clear();
    if (!launch_ms || !n_launches || cap < 1 || cap > 4096)
        return fail(MFFT_ERR_VALUE, "launch_ms/n_launches must be valid and 1 <= cap <= 4096");
    *n_launches = 0;
    if (!p) return fail(MFFT_ERR_VALUE, "plan must not be NULL");
    std::vector<hipEvent_t> ev((size_t)cap + 1, nullptr);
    int rc = MFFT_OK;
    for (auto& e : ev) {
        hipError_t he = hipEventCreate(&e);
        if (he != hipSuccess) {
            rc = hip_fail(he, "hipEventCreate");
            break;
        }
    }
    hipStream_t stream = (hipStream_t)stream_v;
    mfft::LaunchTimer timer{ev.data(), cap, 0};
    if (rc == MFFT_OK) {
        hipError_t he = hipEventRecord(ev[0], stream);
        if (he != hipSuccess) rc = hip_fail(he, "hipEventRecord");
    }
    if (rc == MFFT_OK) {
        mfft::g_timer = &timer;
        rc = workspace ? mfft_execute_ws(p, in, out, workspace, workspace_bytes, stream_v)
                       : mfft_execute(p, in, out, stream_v);
        mfft::g_timer = nullptr;
    }
    if (rc == MFFT_OK && timer.count > 0) {
        hipError_t he = hipEventSynchronize(ev[timer.count]);
        if (he != hipSuccess) rc = hip_fail(he, "hipEventSynchronize");
        for (int i = 0; rc == MFFT_OK && i < timer.count; ++i) {
            float ms = 0.0f;
            he = hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
            if (he != hipSuccess) rc = hip_fail(he, "hipEventElapsedTime");
            launch_ms[i] = ms;
        }
        if (rc == MFFT_OK) *n_launches = timer.count;
    }
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    return rc;
}

int mfft_plan_destroy(mfft_plan* p) {
    g_err.clear();
    if (!p) return MFFT_OK;
    // no synchronisation here: the caller has made sure no execute of the
    // plan is still pending on any stream (include/mfft.h)
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (cur != p->device) (void)hipSetDevice(p->device);
    release(p);
    if (cur >= 0 && cur != p->device) (void)hipSetDevice(cur);
    delete p;
    return MFFT_OK;
}

int mfft_plan_query(const mfft_plan* p, mfft_plan_info* info) {
    g_err.clear();
    if (!p || !info) return fail(MFFT_ERR_VALUE, "plan and info must not be NULL");
    std::memset(info, 0, sizeof(*info));
    info->n = p->n;
    info->batch = p->batch;
    info->core_n = p->core_n;
    info->transform_type = p->transform_type;
    info->transform_direction = p->transform_direction;
    info->norm = p->norm;
    info->flow = p->flow;
    info->device = p->device;
    info->launches = p->launches;
    info->elems_per_thread = p->elems;
    info->threads_per_block = p->block;
    info->n1 = p->n1;
    info->n2 = p->n2;
    info->chunk_rows = p->chunk_rows;
    info->workspace_bytes = p->ws_bytes;
    info->table_bytes = p->table_bytes;
    info->scale = (double)p->scale;
    return MFFT_OK;
}

int mfft_plan_sync_overruns(const mfft_plan* p, int64_t* count) {
    g_err.clear();
    if (!p || !count) return fail(MFFT_ERR_VALUE, "plan and count must not be NULL");
    *count = 0;
    if (!p->overrun) return MFFT_OK;
    int v = 0;
    hipError_t he = hipMemcpy(&v, p->overrun, sizeof(int), hipMemcpyDeviceToHost);
    if (he != hipSuccess) return hip_fail(he, "hipMemcpy(four-step counters)");
    *count = v;
    return MFFT_OK;
}

int mfft_bit_reverse_permute(const void* in, void* out, int64_t n, int64_t batch, void* stream) {
    g_err.clear();
    if (!in || !out) return fail(MFFT_ERR_VALUE, "in and out must not be NULL");
    const int logn = log2_exact(n);
    if (logn < 0 || logn > mfft::kMaxLog2N)
        return fail(MFFT_ERR_VALUE, "size must be a power of two in [1, 2^%d], got %lld", mfft::kMaxLog2N, (long long)n);
    if (batch < 1) return fail(MFFT_ERR_VALUE, "batch must be >= 1");
    if (batch > ((int64_t)1 << 37) / n) return fail(MFFT_ERR_VALUE, "batch too large (over 2^40 bytes)");
    if (!mfft::launch_fits((n * batch + 255) / 256, 256))  // one thread per element
        return fail(MFFT_ERR_UNSUPPORTED, "batch=%lld of n=%lld needs a launch of 2^32 work-items or more; "
                    "split the batch", (long long)batch, (long long)n);
    const size_t bytes = (size_t)n * (size_t)batch * 8;
    if ((const char*)in < (const char*)out + bytes && (const char*)out < (const char*)in + bytes)
        return fail(MFFT_ERR_VALUE, "in and out must not overlap");
    hipError_t e = mfft::launch_bitrev((const float2*)in, (float2*)out, n, batch, (hipStream_t)stream);
    return e == hipSuccess ? MFFT_OK : hip_fail(e, "kernel launch");
}

int mfft_twiddle_transpose(const void* in, void* out, int64_t rows, int64_t cols, int64_t batch, int direction,
                           void* stream) {
    g_err.clear();
    if (!in || !out) return fail(MFFT_ERR_VALUE, "in and out must not be NULL");
    const int lr = log2_exact(rows), lc = log2_exact(cols);
    if (lr < 0 || lc < 0 || lr + lc > mfft::kMaxLog2N)
        return fail(MFFT_ERR_VALUE, "rows and cols must be powers of two with rows * cols <= 2^%d (got %lld x %lld)",
                    mfft::kMaxLog2N, (long long)rows, (long long)cols);
    if (batch < 1) return fail(MFFT_ERR_VALUE, "batch must be >= 1");
    if (batch > ((int64_t)1 << 37) / (rows * cols)) return fail(MFFT_ERR_VALUE, "batch too large");
    if (!mfft::launch_fits(batch * ((rows + 31) / 32) * ((cols + 31) / 32), 256))  // 256 threads per 32 x 32 tile
        return fail(MFFT_ERR_UNSUPPORTED, "batch=%lld of %lld x %lld needs a launch of 2^32 work-items or more; "
                    "split the batch", (long long)batch, (long long)rows, (long long)cols);
    if (direction != MFFT_FORWARD && direction != MFFT_INVERSE)
        return fail(MFFT_ERR_VALUE, "unsupported direction %d", direction);
    const size_t bytes = (size_t)(rows * cols * batch) * 8;
    if ((const char*)in < (const char*)out + bytes && (const char*)out < (const char*)in + bytes)
        return fail(MFFT_ERR_VALUE, "in and out must not overlap");
    if ((((uintptr_t)in) | ((uintptr_t)out)) & 7) return fail(MFFT_ERR_VALUE, "in and out must be 8-byte aligned");
    const hipError_t e = mfft::launch_twiddle_transpose(direction == MFFT_FORWARD ? -1 : 1, (const float2*)in,
                                                        (float2*)out, rows, cols, batch, (hipStream_t)stream);
    return e == hipSuccess ? MFFT_OK : hip_fail(e, "kernel launch");
}

namespace {
// The shared contract of the standalone real epilogues (the reference's
// _validate_real_half, runner.py:1661-1678): n a power of two in [4, 2^20],
// batch >= 1, device pointers that do not overlap, 8-byte aligned.
int real_epilogue(int kind, const void* in, void* out, int64_t n, int64_t batch, float scale, void* stream) {
    g_err.clear();
    if (!in || !out) return fail(MFFT_ERR_VALUE, "in and out must not be NULL");
    const int logn = log2_exact(n);
    if (logn < 2 || logn > mfft::kMaxLog2N)
        return fail(MFFT_ERR_VALUE, "the real epilogues need N a power of two in [4, 2^%d], got %lld",
                    mfft::kMaxLog2N, (long long)n);
    if (batch < 1) return fail(MFFT_ERR_VALUE, "batch must be >= 1");
    if (batch > ((int64_t)1 << 37) / n) return fail(MFFT_ERR_VALUE, "batch too large (over 2^40 bytes)");
    const int64_t np = n >> 1;
    const int64_t per_row = kind == 0 ? np + 1 : np;  // output values (threads) per row
    if (!mfft::launch_fits((batch * per_row + 255) / 256, 256))
        return fail(MFFT_ERR_UNSUPPORTED, "batch=%lld of n=%lld needs a launch of 2^32 work-items or more; "
                    "split the batch", (long long)batch, (long long)n);
    if (!std::isfinite(scale)) return fail(MFFT_ERR_VALUE, "scale must be finite");
    const size_t in_bytes = (size_t)batch * (size_t)(kind == 1 ? np + 1 : np) * 8;
    const size_t out_bytes = (size_t)batch * (size_t)(kind == 0 ? np + 1 : np) * 8;
    if ((const char*)in < (const char*)out + out_bytes && (const char*)out < (const char*)in + in_bytes)
        return fail(MFFT_ERR_VALUE, "in and out must not overlap");
    if ((((uintptr_t)in) | ((uintptr_t)out)) & 7) return fail(MFFT_ERR_VALUE, "in and out must be 8-byte aligned");
    const hipError_t e = mfft::launch_real_epilogue(kind, in, out, n, batch, scale, (hipStream_t)stream);
    return e == hipSuccess ? MFFT_OK : hip_fail(e, "kernel launch");
}
}  // namespace

int mfft_r2c_stitch(const void* z, void* x, int64_t n, int64_t batch, float scale, void* stream) {
    return real_epilogue(0, z, x, n, batch, scale, stream);
}

int mfft_c2r_pre(const void* x, void* z, int64_t n, int64_t batch, void* stream) {
    return real_epilogue(1, x, z, n, batch, 1.0f, stream);
}

int mfft_c2r_unpack(const void* u, void* out, int64_t n, int64_t batch, float scale, void* stream) {
    return real_epilogue(2, u, out, n, batch, scale, stream);
}

int mfft_stream_copy(const void* in, void* out, int64_t bytes, void* stream) {
    g_err.clear();
    if (!in || !out) return fail(MFFT_ERR_VALUE, "in and out must not be NULL");
    if (bytes < 0 || bytes % 16) return fail(MFFT_ERR_VALUE, "bytes must be a non-negative multiple of 16, got %lld",
                                             (long long)bytes);
    if (bytes > ((int64_t)1 << 40)) return fail(MFFT_ERR_VALUE, "bytes over 2^40");
    if (!mfft::launch_fits((bytes / 16 + 2047) / 2048, 256))  // 256 threads per 32 KiB
        return fail(MFFT_ERR_UNSUPPORTED, "a copy of %lld bytes needs a launch of 2^32 work-items or more; split it",
                    (long long)bytes);
    if ((((uintptr_t)in) | ((uintptr_t)out)) & 15) return fail(MFFT_ERR_VALUE, "in and out must be 16-byte aligned");
    if ((const char*)in < (const char*)out + bytes && (const char*)out < (const char*)in + bytes)
        return fail(MFFT_ERR_VALUE, "in and out must not overlap");
    const hipError_t e = mfft::launch_stream_copy(in, out, bytes, (hipStream_t)stream);
    return e == hipSuccess ? MFFT_OK : hip_fail(e, "kernel launch");
}

int mfft_device_props_get(int device, mfft_device_props* out) {
    g_err.clear();
    if (!out) return fail(MFFT_ERR_VALUE, "out must not be NULL");
    std::memset(out, 0, sizeof(*out));
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return fail(MFFT_ERR_VALUE, "device %d out of range (%d devices)", device, count);
    hipDeviceProp_t pr;
    e = hipGetDeviceProperties(&pr, device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    std::snprintf(out->name, sizeof(out->name), "%s", pr.name);
    std::snprintf(out->gcn_arch_name, sizeof(out->gcn_arch_name), "%s", pr.gcnArchName);
    out->multiprocessor_count = pr.multiProcessorCount;
    out->warp_size = pr.warpSize;
    out->shared_mem_per_block = (int64_t)pr.sharedMemPerBlock;
    out->shared_mem_per_multiprocessor = (int64_t)pr.maxSharedMemoryPerMultiProcessor;
    out->total_global_mem = (int64_t)pr.totalGlobalMem;
    out->clock_rate_khz = pr.clockRate;
    out->memory_clock_rate_khz = pr.memoryClockRate;
    out->memory_bus_width = pr.memoryBusWidth;
    out->l2_cache_size = pr.l2CacheSize;
    int v = 0;
    if (hipDriverGetVersion(&v) == hipSuccess) out->driver_version = v;
    v = 0;
    if (hipRuntimeGetVersion(&v) == hipSuccess) out->runtime_version = v;
    out->abi_version = MFFT_ABI_VERSION;
    return MFFT_OK;
}

}  // extern "C"
