// fourstep_kernels.hip -- two-pass (Bailey 4-step) FFT for core lengths
// 2^8 .. 2^20, the MI355X form of the reference's hybrid path
// (src/xpu/adapter_hybrid.py:224-270, scripts/issue10_wp3_perf.py:428-461).
//
// N = N1*N2, n = n1*N2 + n2, k = k1 + N1*k2:
//   X[k1 + N1*k2] = sum_n2 W_N2^(n2*k2) * [ W_N^(n2*k1) * sum_n1 x[n1*N2+n2] W_N1^(n1*k1) ]
// Pass 1 (column pass): for each n2, an N1-point FFT down the column
//   x[n1*N2 + n2] (row stride N2), times W_N^(n2*k1), stored transposed as
//   Z[n2*N1 + k1] -- one contiguous run of N1 per column, so the store is
//   unit-stride.  The twiddle and the layout hand-off are fused into this
//   store (the reference's k_twiddle_fused idea, issue10_wp3_perf.py:214-242).
// Pass 2 (row pass): for each k1, an N2-point FFT over Z[k1 + N1*n2] (stride
//   N1), stored to X[k1 + N1*k2] -- the same addresses it read, so pass 2 runs
//   in place on the output buffer and the plan needs no workspace.
// Both passes are one kernel template: a block owns C adjacent columns (lanes
// run along the columns, so every row access is a C*8-byte contiguous run),
// keeps them in LDS, and runs the same Stockham passes as the single-pass
// kernel on each column.  Inverse = conjugated roots; the norm scale is applied
// by pass 2's store.  The big twiddle W_N^e (e < N) is the product of two
// small tables, W_N^(e mod 2^h) * W_N^(2^h * (e >> h)); pass 1 applies it in
// registers after its last Stockham pass, as W_N^(n2*b) * (W_N^(n2*NS))^q,
// so each thread does a few table lookups instead of two per element.
// Stockham twiddles come from per-pass tables (rows W^k, W^2k, W^4k, W^8k).
#include "mfft_device.hpp"
#include "mfft_internal.hpp"

namespace mfft {

// column-group width and elements per thread for a pass of length 2^logl
constexpr int col_loge(int logl) { return logl >= 8 ? 4 : (logl >= 6 ? 3 : 2); }
constexpr int col_logc(int logl) { return logl >= 9 ? 3 : 4; }
int fourstep_col_loge(int logl) { return col_loge(logl); }

namespace {

__device__ __forceinline__ int pad(int i) { return i + (i >> 4); }

// Workgroups are dispatched to the 8 XCDs round-robin (block p -> XCD p % 8),
// and each XCD has its own L2.  With 8 columns per block a 128-byte row
// segment is shared by logical blocks 2k and 2k+1; this map puts both on the
// same XCD (physical blocks 16q + x and 16q + 8 + x), dispatched together, so
// the line is fetched once into that XCD's L2.  A bijection on every full
// group of 16 blocks; the tail keeps its order.
__device__ __forceinline__ int xcd_pair_block(int p, int total) {
    if (p >= (total & ~15)) return p;
    const int r = p & 15;
    return (p & ~15) + ((r & 7) << 1) + (r >> 3);
}

template <int LOGL, int LOGE, int LOGC>
struct ColCfg {
    static_assert(LOGE < LOGL, "a column pass needs more than one thread per column");
    static constexpr int L = 1 << LOGL;
    static constexpr int E = 1 << LOGE;
    static constexpr int C = 1 << LOGC;
    static constexpr int T = L / E;  // threads per column
    static constexpr int WG = C * T;
    static constexpr int P = sched_passes(LOGL, LOGE);
    // Column pitch in float2 units, == 32/C (mod 32): a half-wave (32 lanes)
    // covers C columns x 32/C rows, and with this pitch the C columns start
    // 64/C dwords apart, tiling the 64 LDS banks without conflicts.
    static constexpr int PITCH0 = L + (L >> 4);
    static constexpr int PITCH = PITCH0 + ((32 / C - PITCH0 % 32) + 32) % 32;
    static constexpr int logr(int p) { return sched_logr(LOGL, LOGE, p); }
    static constexpr int lns(int p) { return sched_lns(LOGE, p); }
};

// W_N^e for e < N as the product of the two small tables
__device__ __forceinline__ float2 big_root(const float2* __restrict__ lo, const float2* __restrict__ hi,
                                          int h, uint32_t e) {
    return cmul(lo[e & ((1u << h) - 1)], hi[e >> h]);
}

// KIND 0: pass 1 (column FFT of length L = N1 over S = N2 columns, twiddle,
//         transposed store).  KIND 1: pass 2 (in place, L = N2, S = N1 columns).
template <int LOGL, int LOGE, int LOGC, int DIR, int KIND>
__global__ __launch_bounds__((ColCfg<LOGL, LOGE, LOGC>::WG)) void fourstep_pass_kernel(
    const float2* src, float2* dst, const float2* __restrict__ tw,
    const float2* __restrict__ tw_lo, const float2* __restrict__ tw_hi, int tw_h, int logn,
    int log_s, float scale) {
    using C = ColCfg<LOGL, LOGE, LOGC>;
    constexpr int L = C::L, E = C::E, T = C::T, P = C::P, NC = C::C;
    __shared__ float2 lds[NC * C::PITCH];

    const int tid = threadIdx.x;
    const int c = tid & (NC - 1);
    const int j = tid >> LOGC;
    const int groups = (1 << log_s) >> LOGC;  // column groups per transform
    const int bid = xcd_pair_block((int)blockIdx.x, (int)gridDim.x);
    const int64_t row = bid / groups;
    const int c0 = (bid - (int)(row * groups)) << LOGC;
    const int64_t base = row << logn;
    const float2* s = src + base + c0 + c;
    float2* lt = lds + c * C::PITCH;

    float2 v[E];
    {
        constexpr int R0 = 1 << C::logr(0);
        constexpr int NB0 = E / R0;
        static_for<0, NB0>([&](auto m) {
            static_for<0, R0>([&](auto q) {
                const int i = j + m.value * T + q.value * (L / R0);
                v[m.value * R0 + q.value] = s[(int64_t)i << log_s];
            });
        });
    }
    // KIND 1 runs in place (src == dst): every element of this block's columns
    // is in registers before the first barrier, all stores come after it, and
    // no other block touches these columns.

    static_for<0, P>([&](auto pp) {
        constexpr int p = pp.value;
        constexpr int LR = C::logr(p);
        constexpr int R = 1 << LR;
        constexpr int NB = E / R;
        constexpr int LNS = C::lns(p);
        constexpr int NS = 1 << LNS;
        if constexpr (p > 0) {
            static_for<0, NB>([&](auto m) {
                static_for<0, R>([&](auto q) {
                    const int i = j + m.value * T + q.value * (L / R);
                    v[m.value * R + q.value] = lt[pad(i)];
                });
            });
        }
        static_for<0, NB>([&](auto m) {
            const int b = j + m.value * T;
            if constexpr (NS > 1) {
                constexpr int TW_OFF = sched_tw_off(LOGL, LOGE, p);
                pass_twiddle<R, DIR, m.value * R>(v, tw + TW_OFF, NS, b & (NS - 1));
            }
            dft<R, DIR, m.value * R, 1>(v);
            if constexpr (KIND == 0 && p == P - 1) {
                // four-step twiddle W_N^(n2*k1) on the pass-1 outputs, in
                // registers: k1 = b + q*NS, so W = W_N^(n2*b) * (W_N^(n2*NS))^q
                const uint32_t n2 = (uint32_t)(c0 + c);
                const float2 w0 = big_root(tw_lo, tw_hi, tw_h, n2 * (uint32_t)b);
                float2 sp[R];
                static_for<0, LR>([&](auto i) {
                    sp[1 << i.value] = big_root(tw_lo, tw_hi, tw_h, n2 * (uint32_t)(NS << i.value));
                });
                static_for<3, R>([&](auto q) {
                    constexpr int hb = high_bit(q.value);
                    if constexpr (hb != q.value) sp[q.value] = cmul(sp[q.value - hb], sp[hb]);
                });
                v[m.value * R] = cmul_tw<DIR>(v[m.value * R], w0);
                static_for<1, R>([&](auto q) {
                    v[m.value * R + q.value] = cmul_tw<DIR>(v[m.value * R + q.value], cmul(w0, sp[q.value]));
                });
            }
        });
        if constexpr (p < P - 1 || KIND == 0) {
            if constexpr (p > 0) __syncthreads();
            static_for<0, NB>([&](auto m) {
                const int b = j + m.value * T;
                const int base_o = ((b >> LNS) << (LNS + LR)) + (b & (NS - 1));
                static_for<0, R>([&](auto q) { lt[pad(base_o + q.value * NS)] = v[m.value * R + q.value]; });
            });
            __syncthreads();
        }
    });

    if constexpr (KIND == 0) {
        // transposed store (the twiddle was applied in registers): lanes run
        // along k1 inside one column, one contiguous run of L per column
        static_for<0, E>([&](auto r) {
            const int e = tid + r.value * C::WG;
            const int cc = e >> LOGL;
            const int k1 = e & (L - 1);
            dst[base + ((int64_t)(c0 + cc) << LOGL) + k1] = lds[cc * C::PITCH + pad(k1)];
        });
    } else {
        constexpr int LR = C::logr(P - 1);
        constexpr int R = 1 << LR;
        constexpr int NB = E / R;
        constexpr int NS = L / R;
        float2* d = dst + base + c0 + c;
        static_for<0, NB>([&](auto m) {
            const int b = j + m.value * T;
            static_for<0, R>([&](auto q) {
                d[(int64_t)(b + q.value * NS) << log_s] = cscale(v[m.value * R + q.value], scale);
            });
        });
    }
}


template <int LOGL, int DIR, int KIND>
hipError_t launch_pass(const float2* src, float2* dst, const mfft_plan* p, int64_t rows,
                       int log_s, float scale, hipStream_t stream) {
    constexpr int LOGE = col_loge(LOGL);
    constexpr int LOGC = col_logc(LOGL);
    using C = ColCfg<LOGL, LOGE, LOGC>;
    const int logn = ilog2((int)p->core_n);
    const int64_t groups = ((int64_t)1 << log_s) >> LOGC;
    const int64_t blocks = rows * groups;
    const float2* tw = KIND == 0 ? p->tw_n1 : p->tw_n2;
    fourstep_pass_kernel<LOGL, LOGE, LOGC, DIR, KIND><<<(unsigned)blocks, C::WG, 0, stream>>>(
        src, dst, tw, p->tw_lo, p->tw_hi, p->tw_h, logn, log_s, scale);
    mark(stream);
    return hipGetLastError();
}

template <int DIR, int KIND>
hipError_t dispatch_len(int logl, const float2* src, float2* dst, const mfft_plan* p, int64_t rows,
                        int log_s, float scale, hipStream_t stream) {
    switch (logl) {
        case 4: return launch_pass<4, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        case 5: return launch_pass<5, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        case 6: return launch_pass<6, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        case 7: return launch_pass<7, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        case 8: return launch_pass<8, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        case 9: return launch_pass<9, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        case 10: return launch_pass<10, DIR, KIND>(src, dst, p, rows, log_s, scale, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool fourstep_supported(int log2n1, int log2n2) {
    // each pass length in [16, 1024]; the other factor must hold a full column group
    if (log2n1 < 4 || log2n1 > 10 || log2n2 < 4 || log2n2 > 10) return false;
    return log2n2 >= col_logc(log2n1) && log2n1 >= col_logc(log2n2);
}

void fourstep_default_split(int log2n, int* log2n1, int* log2n2) {
    *log2n1 = log2n / 2;
    *log2n2 = log2n - *log2n1;
}

hipError_t launch_fourstep(int dir, const float2* src, float2* dst, const mfft_plan* p, int64_t rows,
                           float scale, hipStream_t stream, int* launches) {
    const int l1 = ilog2((int)p->n1), l2 = ilog2((int)p->n2);
    const int64_t chunk = p->chunk_rows > 0 ? p->chunk_rows : rows;
    const int64_t n = p->core_n;
    int count = 0;
    for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
        const int64_t rc = rows - r0 < chunk ? rows - r0 : chunk;
        const float2* s = src + r0 * n;
        float2* d = dst + r0 * n;
        hipError_t e;
        e = dir < 0 ? dispatch_len<-1, 0>(l1, s, d, p, rc, l2, 1.0f, stream)
                    : dispatch_len<1, 0>(l1, s, d, p, rc, l2, 1.0f, stream);
        if (e != hipSuccess) return e;
        e = dir < 0 ? dispatch_len<-1, 1>(l2, d, d, p, rc, l1, scale, stream)
                    : dispatch_len<1, 1>(l2, d, d, p, rc, l1, scale, stream);
        if (e != hipSuccess) return e;
        count += 2;
    }
    if (launches) *launches = count;
    return hipSuccess;
}

}  // namespace mfft
