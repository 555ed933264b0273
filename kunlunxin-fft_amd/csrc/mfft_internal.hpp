// mfft_internal.hpp -- host-side plan record and the launchers each kernel
// source file provides.  Every launcher only enqueues on `stream` and returns
// hipGetLastError()'s verdict through the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mfft.h"

struct mfft_plan {
    int64_t n = 0, batch = 0;
    int64_t core_n = 0;  // complex core length
    int transform_type = MFFT_C2C, transform_direction = MFFT_FORWARD, norm = MFFT_NORM_BACKWARD;
    int flow = MFFT_FLOW_AUTO;
    int device = 0;
    float scale = 1.0f;  // applied by the final store of the core (c2c, c2r) or the stitch (r2c)
    int block = 256;     // stage flows: threads per block
    int elems = 16;      // LDS_FUSED: elements per thread
    int stagger = 0;     // LDS_FUSED: start stagger of half the first wave, s_sleep(127) units
    bool staged = false; // LDS_FUSED: rows in and out through LDS, lane-consecutive
    int launches = 0;
    int64_t n1 = 0, n2 = 0, chunk_rows = 0;
    int schedule = 0;    // FOUR_STEP: 0 one column group per block, 1 persistent, 2 fused (one launch)
    int pass2_rev = 0;   // FOUR_STEP: pass 2 walks the batch rows in reverse order (schedules 0, 1)
    int fused_lag = 0;   // FOUR_STEP schedule 2: transforms pass 1 runs ahead of pass 2
    int fused_take = 0;  // FOUR_STEP schedule 2: queue items a block takes per dequeue
    int fused_ring = 0;  // FOUR_STEP schedule 2: Z slots per XCD (>= fused_lag + 1)
    int fused_grid = 0;  // FOUR_STEP schedule 2: blocks of the launch (resident, a multiple of num_xcc)
    int num_cus = 0;     // compute units of `device` (persistent / fused grid size)
    int clock_khz = 0;   // constant wall-clock rate of `device` (fused schedule wait bound)
    int num_xcc = 8;     // XCDs of `device` (fused schedule work queues)
    bool r2c_fused = false, c2r_fused = false;  // LDS kernel with the real mode fused
    bool real4_fused = false;  // real transform whose stitch / pre-twiddle is fused into the four-step passes

    // device memory owned by the plan
    float2* tw = nullptr;       // stage flows: W_core^m, m in [0, core_n); LDS flow: pass table
    float2* tw_n1 = nullptr;    // four-step pass-1 Stockham pass table (length n1)
    float2* tw_n2 = nullptr;    // four-step pass-2 Stockham pass table (length n2)
    float2* tw_lo = nullptr;    // W_core^m, m < 2^h             (four-step twiddle, low digit)
    float2* tw_hi = nullptr;    // W_core^(m*2^h)                (four-step twiddle, high digit)
    int tw_h = 0;
    float2* tw_real = nullptr;  // exp(-2*pi*i*k/n), k in [0, n/2]  (r2c stitch / c2r pre)
    float2* tw_ra = nullptr;    // real four-step: r2c W_n^k1 (k1 < n1); c2r W_n^n2 (n2 < n2)
    float2* tw_rb = nullptr;    // real four-step: r2c W_n^(n1 k2) (k2 <= n2); c2r W_n^(n2 n1) (n1 < n1)
    float2* ws_a = nullptr;     // core-sized scratch (real flows: core output / input)
    float2* ws_b = nullptr;     // core-sized scratch (stage-flow ping-pong)
    int* overrun = nullptr;     // fused four-step: waits that gave up, over all launches of the plan
    char* ws_f = nullptr;       // fused four-step: launch counters, then the Z ring
    int64_t ws_bytes = 0, table_bytes = 0;  // device memory held by the plan
    // Scratch an execute needs: ws_a and/or ws_b, each core_bytes, and the
    // fused schedule's ws_f (fused_bytes: counters, then the ring at
    // fused_ring_off); caller workspaces hold ws_a at offset 0, ws_b at
    // work_b_off and ws_f at work_f_off.
    bool need_a = false, need_b = false, need_f = false;
    int64_t core_bytes = 0, work_b_off = 0, work_f_off = 0, fused_bytes = 0, fused_ring_off = 0, work_bytes = 0;
    bool caller_ws = false;  // created with MFFT_PLAN_CALLER_WORKSPACE: holds no ws_a / ws_b / ws_f
};

namespace mfft {

// Optional per-launch event recording (mfft_execute_timed): every launcher
// calls mark(stream) right after each kernel launch.  Off (nullptr) otherwise.
struct LaunchTimer {
    hipEvent_t* ev;  // cap + 1 events; ev[0] is recorded before the first launch
    int cap;
    int count;       // launches marked so far
};
extern thread_local LaunchTimer* g_timer;
inline void mark(hipStream_t s) {
    LaunchTimer* t = g_timer;
    if (t && t->count < t->cap) {
        (void)hipEventRecord(t->ev[t->count + 1], s);
        ++t->count;
    }
}

constexpr int kMaxLog2N = 20;        // reference range: 8 .. 2^20 (docs/user-guide/transforms.md)
// A dispatch packet carries its launch's work-item count in 32 bits, and
// the runtime takes some larger launches with the count wrapped (2^32 + 1024
// work-items ran as 1024, without an error, on MI355X), so every launch
// checks its size and a plan refuses shapes whose launches would not fit.
constexpr int64_t kMaxLaunchItems = ((int64_t)1 << 32) - 1;
inline bool launch_fits(int64_t blocks, int64_t threads_per_block) {
    return blocks >= 0 && threads_per_block > 0 && blocks <= kMaxLaunchItems / threads_per_block;
}
constexpr int kMaxLdsLog2 = 15;      // single-pass LDS kernel: core length <= 32768
constexpr int kMinFourStepLog2 = 8;  // four-step needs n1, n2 >= 16

// ---- stage_kernels.hip: reference global-stage flows, real epilogues ------
// Radix-2 / radix-4 global-stage core over `rows` rows of length n:
// reads `src` (never written), writes `dst`, ping-pongs through `scratch`.
hipError_t launch_radix2(bool dif, int dir, const float2* src, float2* dst, float2* scratch,
                         const float2* tw, int64_t n, int64_t rows, float scale, int block,
                         hipStream_t stream, int* launches);
hipError_t launch_radix4(bool dif, int dir, const float2* src, float2* dst, float2* scratch,
                         const float2* tw, int64_t n, int64_t rows, float scale, int block,
                         hipStream_t stream, int* launches);
hipError_t launch_bitrev(const float2* src, float2* dst, int64_t n, int64_t rows, hipStream_t stream);
// dst = src, `bytes` a multiple of 16 (16-byte aligned, non-overlapping)
hipError_t launch_stream_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream);
// G[c][r] = S[r][c] * W_(rows*cols)^(dir * r * c) for `batch` rows x cols matrices
hipError_t launch_twiddle_transpose(int dir, const float2* s, float2* g, int64_t rows, int64_t cols, int64_t batch,
                                    hipStream_t stream);
// R2C stitch: z [rows][n/2] (unnormalised N/2 FFT of packed pairs) -> x [rows][n/2+1]
hipError_t launch_r2c_stitch(const float2* z, float2* x, const float2* tw_real, int64_t n,
                             int64_t rows, float scale, hipStream_t stream);
// C2R pre-twiddle: x [rows][n/2+1] -> z [rows][n/2], the inverse core's input
hipError_t launch_c2r_pre(const float2* x, float2* z, const float2* tw_real, int64_t n,
                          int64_t rows, hipStream_t stream);
// The standalone epilogues, roots computed in the kernel: kind 0 stitch
// (z [rows][n/2] -> x [rows][n/2+1], times scale), 1 pre-twiddle
// (x [rows][n/2+1] -> z [rows][n/2]), 2 unpack (u [rows][n/2] -> real
// [rows][n], mirror order, times scale)
hipError_t launch_real_epilogue(int kind, const void* in, void* out, int64_t n, int64_t rows, float scale,
                                hipStream_t stream);

// ---- lds_kernels.hip: single-pass LDS-resident Stockham kernel ------------
// mode 0: c2c core; 1: r2c (core forward + fused stitch); 2: c2r (fused
// pre-twiddle + inverse core).  `log2l` is the core length's log2.
bool lds_supported(int log2l, int elems);  // every mode (C2C, R2C, C2R) alike
int lds_default_elems(int log2l);
int lds_threads_per_block(int log2l, int elems);
hipError_t launch_lds(int mode, int dir, int log2l, int elems, const void* src, void* dst,
                      const float2* tw, const float2* tw_real, int64_t rows, float scale,
                      hipStream_t stream, int num_cus = 0, int stagger = 0, bool staged = false);
// the staged form exists for these (fewer than 16 threads per transform)
bool lds_staged_supported(int log2l, int elems);

// ---- mfma_kernels.hip: dense-dot core on the fp32 matrix cores -----------
constexpr int kMaxMfmaLog2 = 14;  // core length 2 .. 16384
bool mfma_supported(int log2l);
// c2c core over `rows` rows of length 2^log2l; tw = W_L^m for m < L
hipError_t launch_mfma(int dir, int log2l, const float2* src, float2* dst, const float2* tw, int64_t rows,
                       float scale, hipStream_t stream);

// ---- fourstep_kernels.hip: two-pass column/row FFT -----------------------
bool fourstep_supported(int log2n1, int log2n2);
bool fourstep_fused_supported(int log2n1, int log2n2);  // schedule 2: n1, n2 in [128, 512], within 2x
constexpr int kMaxStagger = 16;  // LDS_FUSED start stagger limit (16 x 8128 clocks)
constexpr int kFusedWaitMs = 20;  // longest pass-2 wait of the fused schedule before it gives up
constexpr bool kFusedScheduleEnabled = true;
// fused-schedule launch counters: [0, kFusedSlots) work queues (one per
// XCD), [kFusedFail] the launch's failure word, then two per transform of a
// launch (pass-1 groups done, pass-2 groups done)
constexpr int kFusedSlots = 16;
constexpr int kFusedFail = kFusedSlots;
constexpr int kFusedHead = kFusedSlots + 1;
constexpr int kFusedFailMark = 1 << 20;  // added to a pass-1 count by a group that skipped its store
constexpr int kFusedMaxRing = 64;        // Z slots per XCD
int fourstep_fused_occupancy(int log2n1, int log2n2);  // resident blocks per CU of the fused kernel
int fourstep_col_loge(int logl, int schedule);  // log2 elements per thread of a pass of length 2^logl
void fourstep_default_split(int log2n, int* log2n1, int* log2n2);
// fws: the fused schedule's scratch (counters, then the Z ring), or NULL for
// the other schedules
hipError_t launch_fourstep(int dir, const float2* src, float2* dst, char* fws, const mfft_plan* p,
                           int64_t rows, float scale, hipStream_t stream, int* launches);
// A real transform with the stitch / pre-twiddle fused into the four-step
// core (plans with real4_fused): R2C x -> permuted Z (work) -> bins;
// C2R bins -> Z in the output rows -> the row pass in place.
hipError_t launch_fourstep_real(const float2* src, float2* dst, float2* work, const mfft_plan* p, float scale,
                                hipStream_t stream);

}  // namespace mfft
