/*
 * mfft.h -- C ABI of the MI355X (gfx950) FFT operator library.
 *
 * The reference (TruNcat3/kunlunxin-fft) has no C ABI: its boundary is the
 * Python plan API in src/xpu/entry.py.  Each entry point below replaces one
 * piece of what that API does underneath, so that a host binding (the
 * package's Python ctypes layer, or any C/C++/FFI caller) can keep the
 * reference's plan/execute semantics:
 *
 *   mfft_plan_create   <- plan_fft(...) resolution + the runner's per-call
 *                         twiddle build (entry.py:292-426, runner.py:93-97,
 *                         1650-1658) and the 4-step plan caches
 *                         (adapter_hybrid.py:60-108, entry.py:228-233)
 *   mfft_execute       <- execute_fft_plan(plan, x) (entry.py:501-628) with
 *                         the inverse conjugation, norm epilogue
 *                         (entry.py:617-628, 656-668) and the dedicated real
 *                         flows (entry.py:555-587) fused into the kernels
 *   mfft_plan_destroy  <- dropping the plan / its cache entry (entry.py:631-653)
 *   mfft_bit_reverse_permute
 *                      <- runner.bit_reverse_permute (runner.py:1542-1552)
 *   mfft_device_props  <- the device facts DeviceProfile / env fingerprint
 *                         read (config.py:55-95, envcheck.py:62-88)
 *   mfft_last_error    <- the exception message of the Python API; error
 *                         classes map to ValueError / TypeError / RuntimeError
 *                         (validate.py:19-68, context.py:52-56)
 *
 * Data layout: interleaved complex64 (float re, float im) for complex
 * buffers, float32 for real ones, rows of a batch contiguous:
 *   c2c  in [batch][n] complex64      -> out [batch][n] complex64
 *   r2c  in [batch][n] float32        -> out [batch][n/2+1] complex64
 *   c2r  in [batch][n/2+1] complex64  -> out [batch][n] float32
 * (c2r ignores the imaginary parts of bins 0 and n/2, as torch.fft does).
 *
 * Ownership and threading: a plan owns its device twiddle tables and any
 * workspace; mfft_execute allocates nothing and never synchronises the host.
 * It enqueues on `stream` (a hipStream_t; NULL = the default stream) of the
 * device that was current at plan creation, which must be current at
 * execute.  `in` and `out` must not overlap; `in` is never written.
 * A plan is immutable after creation.  A plan that needs no workspace
 * (mfft_plan_workspace_size = 0: every LDS_FUSED plan and FOUR_STEP C2C with
 * schedule 0, 1 or 3) can
 * be executed from any number of host threads and streams at once.  Executes
 * of a plan that needs workspace and overlap in time (two streams or two
 * host threads) share the plan's workspace and race: serialise them, give
 * each its own workspace (mfft_execute_ws), or create one plan per stream.
 */
#ifndef MFFT_H_
#define MFFT_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MFFT_ABI_VERSION 2

/* return codes (0 = success); the Python layer maps them to exceptions */
enum {
    MFFT_OK = 0,
    MFFT_ERR_VALUE = 1,       /* bad size, enum, pointer, overlap -> ValueError */
    MFFT_ERR_TYPE = 2,        /* reserved for dtype errors       -> TypeError  */
    MFFT_ERR_RUNTIME = 3,     /* HIP failure, wrong device       -> RuntimeError */
    MFFT_ERR_UNSUPPORTED = 4  /* flow cannot run this shape      -> ValueError */
};

/* transform_type: src/xpu/config.py:34 TRANSFORM_TYPES */
enum { MFFT_C2C = 0, MFFT_R2C = 1, MFFT_C2R = 2 };
/* transform_direction: config.py:35 */
enum { MFFT_FORWARD = 0, MFFT_INVERSE = 1 };
/* norm: config.py:36 NORMALIZATIONS, scales of entry.py:81-102 */
enum { MFFT_NORM_NONE = 0, MFFT_NORM_FORWARD = 1, MFFT_NORM_BACKWARD = 2, MFFT_NORM_ORTHO = 3 };

/* Kernel families (flow ids).  The first four keep the reference's global
 * stage flows (one launch per stage, M0 / M5 of src/xpu/runner.py); the others
 * are the MI355X flows that replace M1/M2/M3 and the hybrid 4-step. */
enum {
    MFFT_FLOW_AUTO = 0,        /* LDS_FUSED when the core fits one workgroup, else FOUR_STEP */
    MFFT_FLOW_RADIX2_DIT = 1,  /* M0 fft_dit: bit reversal folded into stage 0 (runner.py:118-162) */
    MFFT_FLOW_RADIX2_DIF = 2,  /* M0 fft_dif: bit reversal folded into the last stage (runner.py:165-206) */
    MFFT_FLOW_RADIX4_DIT = 3,  /* M5 fft_dit_radix4: digit reversal folded into stage 0 (runner.py:1399-1470) */
    MFFT_FLOW_RADIX4_DIF = 4,  /* M5 fft_dif_radix4 (runner.py:1473-1540) */
    MFFT_FLOW_LDS_FUSED = 5,   /* one pass: whole transform resident in LDS/registers (core n <= 32768) */
    MFFT_FLOW_FOUR_STEP = 6,   /* two passes: column FFTs + twiddle, then row FFTs (core n >= 256) */
    MFFT_FLOW_DENSE_MFMA = 7   /* M2 fft_{dit,dif}_matrix (runner.py:379-442, kernels.py:487-532): one pass,
                                  every butterfly a dense DFT-8 matrix product on the fp32 matrix cores;
                                  the first two passes form the 8 x 8 factored DFT-64 (core n 2..16384) */
};

/* Flow parameters (params[i], all optional, 0 = library default):
 *   RADIX2_* / RADIX4_*: params[0] = threads per block (64..1024, power of two)
 *   LDS_FUSED:           params[0] = elements per thread (4, 8, 16 or 32; 32 from 2^10,
 *                                    >= 16 from 2^13, 32 at 2^15),
 *                        params[1] = start stagger (0..16): in launches of at
 *                                    least two waves of workgroups, the first
 *                                    wave's workgroups on the upper half of
 *                                    every XCD's CUs start params[1] x 8128
 *                                    clocks late, so that CUs stop loading,
 *                                    computing and storing in lockstep,
 *                        params[2] = staged form (0 or 1; core length /
 *                                    elements per thread < 16, any
 *                                    transform type): the workgroup's rows,
 *                                    one contiguous run, go in and out
 *                                    through LDS with consecutive lanes on
 *                                    consecutive elements
 *   DENSE_MFMA:          no parameters
 *   FOUR_STEP:           params[0] = n1 (column FFT length; n2 = core_n/n1),
 *                        params[1] = batch rows per chunk (both passes run
 *                                    chunk by chunk, and a real transform's
 *                                    stitch or pre-twiddle runs between the
 *                                    chunks; 0 = whole batch),
 *                        params[2] = schedule: 0 = one column group per
 *                                    workgroup; 1 = persistent workgroups (one
 *                                    resident wave of them) that load their
 *                                    next column group while transforming the
 *                                    current one; 2 = fused: both passes in
 *                                    one launch, each transform's pass-1
 *                                    output in a ring of slots per XCD in
 *                                    the workspace, which stays in that XCD's
 *                                    L2, and its pass 2 on the same XCD
 *                                    (n1, n2 in [128, 512] within 2x; the
 *                                    counters and the ring are workspace);
 *                                    3 = narrow: as 0 with four columns per
 *                                    workgroup and at most 16 elements per
 *                                    thread, four times the workgroups for
 *                                    small batches (a real transform's
 *                                    stitch then runs as its own launch),
 *                        params[3] = schedules 0, 1, 3: pass-2 row order: 0 =
 *                                    forward; 1 = reverse, so the batch rows
 *                                    pass 1 wrote last (the most likely still
 *                                    in the MALL) are read first; schedule 2:
 *                                    bits 0-7 = queue lag, 1..63 transforms
 *                                    that pass 1 runs ahead of pass 2 on an
 *                                    XCD (0 = one more than the XCD's resident
 *                                    blocks hold in flight), bits 8-15 = queue
 *                                    items a workgroup takes per dequeue,
 *                                    1..64 (0 = 1), bits 16-23 = Z slots per
 *                                    XCD, lag + 1..64 (0 = lag + 1 + the
 *                                    transforms the resident blocks hold),
 *                                    bits 24-30 = workgroups per CU, 1..16
 *                                    (0 = as many as fit) */
#define MFFT_MAX_PARAMS 4

typedef struct mfft_plan mfft_plan;

typedef struct {
    int64_t n, batch, core_n;     /* core_n: complex core length (n, or n/2 for r2c/c2r) */
    int32_t transform_type, transform_direction, norm;
    int32_t flow;                 /* resolved flow id (never MFFT_FLOW_AUTO) */
    int32_t device;
    int32_t launches;             /* kernel launches per mfft_execute */
    int32_t elems_per_thread;     /* LDS_FUSED: elements per thread */
    int32_t threads_per_block;
    int64_t n1, n2, chunk_rows;   /* FOUR_STEP split */
    int64_t workspace_bytes;      /* device scratch held by the plan */
    int64_t table_bytes;          /* device twiddle tables held by the plan */
    double scale;                 /* output scale applied in the final store */
} mfft_plan_info;

typedef struct {
    char name[256];               /* hipDeviceProp_t::name */
    char gcn_arch_name[256];      /* e.g. "gfx950:sramecc+:xnack-" */
    int32_t multiprocessor_count; /* CUs */
    int32_t warp_size;            /* 64 on CDNA */
    int64_t shared_mem_per_block; /* LDS bytes a workgroup may use */
    int64_t shared_mem_per_multiprocessor;
    int64_t total_global_mem;
    int32_t clock_rate_khz;
    int32_t memory_clock_rate_khz;
    int32_t memory_bus_width;
    int32_t l2_cache_size;
    int32_t driver_version;       /* hipDriverGetVersion */
    int32_t runtime_version;      /* hipRuntimeGetVersion */
    int32_t abi_version;          /* MFFT_ABI_VERSION */
} mfft_device_props;

/* Create a plan on the current device.  Validates everything before any
 * allocation: n a power of two (c2c 1..2^20, r2c/c2r 2..2^20), batch >= 1,
 * enums in range, r2c forward-only and c2r inverse-only (entry.py:157-172),
 * and that `flow` can run the shape: at most 2^40 bytes of complex64 rows,
 * and no launch of 2^32 work-items or more (one dispatch's count is 32-bit;
 * MFFT_ERR_UNSUPPORTED, split the batch).  Uploads the twiddle tables and
 * allocates the workspace: the only allocations the library makes per plan.
 * Apart from them, the library holds one static device buffer of
 * MFFT_NOALLOC_SCRATCH_BYTES per device for mfft_execute_noalloc. */
int mfft_plan_create(mfft_plan** out, int64_t n, int64_t batch, int transform_type,
                     int transform_direction, int norm, int flow,
                     const int32_t* params, int nparams);

/* Enqueue one transform of all `batch` rows.  No allocation, no host sync.
 * FOUR_STEP schedule 2 (params[2] = 2) only: a launch whose bounded wait
 * gives up writes NaN from then on and this call still returns MFFT_OK (the
 * failure is not known when the work is enqueued); synchronise, then check
 * mfft_plan_sync_overruns == 0 before using the output. */
int mfft_execute(const mfft_plan* plan, const void* in, void* out, void* stream);

/* Caller-owned workspace.  The reference exposes neither a stream nor a
 * workspace (its execute_fft_plan, src/xpu/entry.py:501-628, allocates per
 * call on the framework's stream); these entry points close that gap for
 * callers that manage device memory themselves.  A plan needs workspace only
 * for the stage flows (RADIX2/RADIX4: one batch x core_n complex64 buffer),
 * for real transforms whose core is not fused into the LDS kernel (one more
 * such buffer) and for the fused FOUR_STEP schedule (its launch counters and
 * its ring of XCDs x slots x core_n complex64); LDS_FUSED and FOUR_STEP C2C
 * with schedules 0, 1 and 3 need none.
 *
 * mfft_plan_create_ex: mfft_plan_create with `flags`; with
 * MFFT_PLAN_CALLER_WORKSPACE the plan allocates only its twiddle tables (and
 * the fused four-step's overrun count), and every execute of a plan that needs
 * workspace must go through mfft_execute_ws (mfft_execute refuses it). */
#define MFFT_PLAN_CALLER_WORKSPACE 1
int mfft_plan_create_ex(mfft_plan** out, int64_t n, int64_t batch, int transform_type,
                        int transform_direction, int norm, int flow,
                        const int32_t* params, int nparams, int flags);

/* Bytes of workspace an execute of this plan needs (0: none). */
int mfft_plan_workspace_size(const mfft_plan* plan, int64_t* bytes);

/* mfft_execute with the caller's workspace instead of the plan's own:
 * `workspace` is device memory on the plan's device, 256-byte aligned, of at
 * least mfft_plan_workspace_size bytes, overlapping neither `in` nor `out`
 * (it may be NULL when that size is 0).  The library only uses it for the
 * duration of the enqueued work, so executes of one plan on different
 * streams with different workspaces do not race. */
int mfft_execute_ws(const mfft_plan* plan, const void* in, void* out, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* mfft_execute (workspace NULL) or mfft_execute_ws (workspace given) with a
 * HIP event recorded on `stream` before the first and after every kernel
 * launch (the profiling counterpart of the reference's phase ledger,
 * src/xpu/ledger.py:262-296).  Waits for the stream, then writes the
 * duration of each launch in milliseconds to launch_ms[0..k) with
 * k = min(launches, cap) and stores k in *n_launches.  Same work and results
 * as the untimed call; creates and destroys its events (no device memory). */
int mfft_execute_timed(const mfft_plan* plan, const void* in, void* out, void* workspace,
                       int64_t workspace_bytes, void* stream, float* launch_ms, int cap, int* n_launches);

/* Allocation-free execute.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory at execute time (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same work and results as mfft_execute / mfft_execute_ws, but the scratch
 * of a plan that needs one (mfft_plan_workspace_size > 0: the stage flows,
 * the real flows around a non-fused core, and the fused FOUR_STEP schedule's
 * launch counters and Z ring) comes from a static device
 * buffer of MFFT_NOALLOC_SCRATCH_BYTES that the library holds on every
 * device it runs on until the process ends; the call itself allocates
 * nothing (no hipMalloc, no allocating library routine).  A plan needing
 * more scratch than that is refused with MFFT_ERR_VALUE before any launch.
 * Every call on one device shares that device's buffer: calls that overlap
 * in time on one device (two streams, two host threads) race, so serialise
 * them.  The buffer keeps whatever the last call left in it; no kernel
 * reads scratch it has not written in the same call (the fused schedule's
 * counters are zeroed by a fill kernel at the start of every call, never by
 * a memset, so a captured call replays correctly).  The first call on a
 * device looks the buffer's address up once
 * (with that device current, as every execute requires). */
#define MFFT_NOALLOC_SCRATCH_BYTES ((int64_t)32 << 20)
int mfft_execute_noalloc(const mfft_plan* plan, const void* in, void* out, void* stream);

/* Release the plan's device memory.  NULL is a no-op.  It does not
 * synchronise the device: the caller makes sure that no execute of the plan
 * is still pending on any stream (synchronise the streams it ran on, or the
 * device), as for freeing any memory a pending kernel reads.  Plan creation
 * likewise waits only for its own uploads (a private stream of the device),
 * never for other streams' work. */
int mfft_plan_destroy(mfft_plan* plan);

/* Describe a plan (resolved flow, launch count, memory held). */
int mfft_plan_query(const mfft_plan* plan, mfft_plan_info* info);

/* FOUR_STEP schedule 2 only (no counterpart in the reference: a diagnostic of
 * this library's fused schedule): how many waits of this plan's launches so
 * far (pass 2 for its pass-1 output, pass 1 for its Z slot) gave up at their
 * limit instead of seeing the work they wait for complete -- 0 unless
 * something is wrong; a launch with such a wait writes NaN from then on.  Copies one int from the device
 * (synchronous); *count = 0 for plans of any other flow. */
int mfft_plan_sync_overruns(const mfft_plan* plan, int64_t* count);

/* out[r][bit_reverse(i)] = in[r][i] over `batch` rows of n complex64
 * (runner.bit_reverse_permute, runner.py:1542-1552); n a power of two. */
int mfft_bit_reverse_permute(const void* in, void* out, int64_t n, int64_t batch, void* stream);

/* The dedicated real-transform epilogues as standalone launches, for a
 * caller that runs the half-length (n/2-point) complex core itself
 * (runner.r2c_stitch / c2r_pre / c2r_unpack, runner.py:1687-1767).  The
 * plans fuse the same arithmetic into their kernels; these take no plan and
 * allocate nothing (the roots exp(-2 pi i k / n) are computed in the
 * kernel).  n a power of two in [4, 2^20], `batch` rows, device pointers
 * that do not overlap, enqueued on `stream`.
 *   mfft_r2c_stitch: z [batch][n/2] complex64 (the unnormalised forward
 *     FFT of the packed pairs x[2m] + i x[2m+1]) -> x [batch][n/2+1]
 *     complex64, the real input's spectrum times `scale` (imaginary parts
 *     of bins 0 and n/2 exactly 0).
 *   mfft_c2r_pre: x [batch][n/2+1] complex64 half spectrum (imaginary parts
 *     of bins 0 and n/2 ignored) -> z [batch][n/2] complex64, the input of
 *     the half-length core.
 *   mfft_c2r_unpack: u [batch][n/2] complex64, the unnormalised FORWARD
 *     n/2-point FFT of mfft_c2r_pre's output -> out [batch][n] float32 real
 *     samples times `scale` (2 * the norm's inverse scale: 2/n for
 *     "backward"); read in mirror order, which turns the forward core into
 *     the inverse one. */
int mfft_r2c_stitch(const void* z, void* x, int64_t n, int64_t batch, float scale, void* stream);
int mfft_c2r_pre(const void* x, void* z, int64_t n, int64_t batch, void* stream);
int mfft_c2r_unpack(const void* u, void* out, int64_t n, int64_t batch, float scale, void* stream);

/* The twiddle + transpose boundary of a composed four-step whose sub-FFTs
 * run elsewhere (the reference's run_hybrid, adapter_hybrid.py:294-301, a
 * fused "transpose + twiddle" pass between two vendor sub-FFT stages): for
 * each of `batch` row-major rows x cols complex64 matrices S,
 *   out[c][r] = S[r][c] * exp(-+2 pi i r c / (rows * cols))
 * (- for MFFT_FORWARD, + for MFFT_INVERSE); rows and cols powers of two with
 * rows * cols <= 2^20; in and out must not overlap. */
int mfft_twiddle_transpose(const void* in, void* out, int64_t rows, int64_t cols, int64_t batch, int direction,
                           void* stream);

/* Measurement only; no counterpart in the reference, for benchmark callers:
 * out = in over `bytes` (a multiple of 16; 16-byte aligned, non-overlapping
 * buffers), a streaming copy with non-temporal loads and stores.  Its rate
 * is the practical ceiling of a transform that reads and writes every byte
 * once (bench.py divides its per-size rates by it). */
int mfft_stream_copy(const void* in, void* out, int64_t bytes, void* stream);

/* Device facts for the profile / environment fingerprint. */
int mfft_device_props_get(int device, mfft_device_props* out);

/* Message of the last failing call on this host thread ("" if none). */
const char* mfft_last_error(void);

/* MFFT_ABI_VERSION of the loaded library. */
int mfft_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MFFT_H_ */
