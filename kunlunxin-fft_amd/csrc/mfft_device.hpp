// mfft_device.hpp -- device building blocks shared by every gfx950 kernel:
// interleaved complex64 arithmetic, compile-time roots of unity, and the
// in-register radix-R DFT used as the butterfly of every Stockham pass.
//
// Sign convention: DIR = -1 is the forward transform (exp(-2*pi*i*j*k/N),
// src/xpu/runner.py:93-97), DIR = +1 the unnormalised inverse.  Twiddle
// tables in device memory always hold the forward roots; the inverse uses
// their conjugates, folded into the complex product at no cost.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

namespace mfft {

template <int I>
using ic = std::integral_constant<int, I>;

// Calls f(ic<B>{}), f(ic<B+1>{}), ..., f(ic<E-1>{}) -- a loop whose index is
// a compile-time constant, so register arrays are indexed statically.
template <int B, int E, typename F>
__host__ __device__ __forceinline__ constexpr void static_for(F&& f) {
    if constexpr (B < E) {
        f(ic<B>{});
        static_for<B + 1, E>(f);
    }
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v >> 1); }

constexpr int brev_bits(int x, int bits) {
    int r = 0;
    for (int i = 0; i < bits; ++i) {
        r = (r << 1) | (x & 1);
        x >>= 1;
    }
    return r;
}

// ---- compile-time cos/sin of 2*pi*j/R (Taylor series on [-pi, pi]) -------
constexpr double kPi = 3.14159265358979323846264338327950288;

constexpr double taylor_sin(double x) {
    double term = x, sum = x;
    for (int i = 1; i < 24; ++i) {
        term *= -x * x / ((2.0 * i) * (2.0 * i + 1.0));
        sum += term;
    }
    return sum;
}

constexpr double taylor_cos(double x) {
    double term = 1.0, sum = 1.0;
    for (int i = 1; i < 24; ++i) {
        term *= -x * x / ((2.0 * i - 1.0) * (2.0 * i));
        sum += term;
    }
    return sum;
}

// angle 2*pi*j/R reduced to (-pi, pi]
constexpr double root_angle(int j, int R) {
    int jj = ((j % R) + R) % R;
    double a = 2.0 * kPi * (double)jj / (double)R;
    return a > kPi ? a - 2.0 * kPi : a;
}

// ---- complex64 helpers ------------------------------------------------------
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
__device__ __forceinline__ float2 cconj(float2 a) { return make_float2(a.x, -a.y); }

// a * w (DIR = -1) or a * conj(w) (DIR = +1), w a forward-table root
template <int DIR>
__device__ __forceinline__ float2 cmul_tw(float2 a, float2 w) {
    if constexpr (DIR < 0) {
        return make_float2(a.x * w.x - a.y * w.y, a.x * w.y + a.y * w.x);
    } else {
        return make_float2(a.x * w.x + a.y * w.y, a.y * w.x - a.x * w.y);
    }
}

// a * exp(DIR * 2*pi*i*J/R) with exact rotations for multiples of pi/2 and
// the symmetric pi/4 constants; everything resolved at compile time.
template <int R, int J, int DIR>
__device__ __forceinline__ float2 rot(float2 a) {
    constexpr int j = ((J % R) + R) % R;
    if constexpr (j == 0) {
        return a;
    } else if constexpr (2 * j == R) {
        return make_float2(-a.x, -a.y);
    } else if constexpr (4 * j == R) {  // exp(DIR*i*pi/2) = DIR*i
        return DIR < 0 ? make_float2(a.y, -a.x) : make_float2(-a.y, a.x);
    } else if constexpr (4 * j == 3 * R) {  // exp(DIR*i*3pi/2) = -DIR*i
        return DIR < 0 ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
    } else if constexpr (8 * j == R || 8 * j == 3 * R || 8 * j == 5 * R || 8 * j == 7 * R) {
        constexpr float h = 0.70710678118654752440f;
        constexpr float c = (8 * j == R || 8 * j == 7 * R) ? h : -h;
        constexpr float s0 = (8 * j == R || 8 * j == 3 * R) ? h : -h;  // sin(2*pi*j/R)
        constexpr float s = DIR < 0 ? -s0 : s0;
        return make_float2(c * (a.x) - s * (a.y), c * (a.y) + s * (a.x));
    } else {
        constexpr double ang = root_angle(j, R);
        constexpr float c = (float)taylor_cos(ang);
        constexpr float s = (float)(DIR < 0 ? -taylor_sin(ang) : taylor_sin(ang));
        return make_float2(a.x * c - a.y * s, a.x * s + a.y * c);
    }
}

// In-register DFT of length R over v[OFF + q*STR], q in [0, R), natural order
// in and out.  A radix-2 decimation-in-frequency network with compile-time
// twiddles, followed by the bit-reversal reorder (pure register renaming).
template <int R, int DIR, int OFF, int STR, int E>
__device__ __forceinline__ void dft(float2 (&v)[E]) {
    static_assert(R >= 1 && (R & (R - 1)) == 0, "radix must be a power of two");
    constexpr int LOGR = ilog2(R);
    if constexpr (R > 1) {
        static_for<0, LOGR>([&](auto s) {
            constexpr int h = R >> (s.value + 1);
            static_for<0, R / 2>([&](auto p) {
                constexpr int blk = (p.value / h) * 2 * h;
                constexpr int jj = p.value % h;
                constexpr int i0 = OFF + (blk + jj) * STR;
                constexpr int i1 = OFF + (blk + jj + h) * STR;
                const float2 a = v[i0];
                const float2 b = v[i1];
                v[i0] = cadd(a, b);
                v[i1] = rot<2 * h, jj, DIR>(csub(a, b));
            });
        });
        float2 t[R];
        static_for<0, R>([&](auto q) { t[q.value] = v[OFF + brev_bits(q.value, LOGR) * STR]; });
        static_for<0, R>([&](auto q) { v[OFF + q.value * STR] = t[q.value]; });
    }
}

// ---- Stockham schedule shared by the host (table builder) and the kernels --
// A transform of length 2^logl with up to 2^loge elements per thread runs P
// passes; pass p has radix 2^logr(p) and accumulated span NS = 2^lns(p), the
// product of the radices before it.  Every pass but one has radix 2^le; the
// remainder goes last, or first when `rf` is set (the LDS kernel's r2c mode,
// whose stitch wants a full-radix last pass).
constexpr int sched_le(int logl, int loge) { return loge < logl ? loge : logl; }
constexpr int sched_passes(int logl, int le) { return logl == 0 ? 1 : (logl + le - 1) / le; }
constexpr int sched_logr(int logl, int le, int p, bool rf = false) {
    return (rf ? p > 0 : p < sched_passes(logl, le) - 1) ? le : logl - le * (sched_passes(logl, le) - 1);
}
constexpr int sched_lns(int le, int p) { return le * p; }
constexpr int sched_lns_rf(int logl, int le, int p, bool rf) {
    return rf && p > 0 ? sched_logr(logl, le, 0, true) + le * (p - 1) : le * p;
}
// Pass twiddle table: pass p >= 1 owns logr(p) rows of NS entries, row i
// holding W_{NS*R}^(2^i * k) for k < NS (forward roots).  Offset of pass p:
constexpr int sched_tw_off(int logl, int le, int p, bool rf = false) {
    int off = 0;
    for (int q = 1; q < p; ++q) off += sched_logr(logl, le, q, rf) << sched_lns_rf(logl, le, q, rf);
    return off;
}
// The LDS kernel runs the remainder first in r2c mode when whole waves make
// up a transform (then its last pass can pair lanes for the stitch).
constexpr bool lds_remainder_first(int logl, int le, bool r2c) { return r2c && le >= 4 && logl - le >= 6; }
constexpr int sched_tw_size(int logl, int le, bool rf = false) {
    return sched_tw_off(logl, le, sched_passes(logl, le), rf);
}

// highest power of two <= q (q >= 1)
constexpr int high_bit(int q) { return q <= 1 ? 1 : 2 * high_bit(q >> 1); }

// Non-temporal (streaming) global access of one complex64: the `nt` form
// of the load/store, whose lines are not kept in the caches on a miss.  Data
// read exactly once uses it so that it does not evict what a later pass
// still reads (the four-step's intermediate in the 256 MB MALL).
typedef float nt_float2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float2 load_nt(const float2* p) {
    const nt_float2 v = __builtin_nontemporal_load(reinterpret_cast<const nt_float2*>(p));
    return make_float2(v.x, v.y);
}
__device__ __forceinline__ void store_nt(float2* p, float2 x) {
    const nt_float2 v = {x.x, x.y};
    __builtin_nontemporal_store(v, reinterpret_cast<nt_float2*>(p));
}

// Output store of one complex64; WT: write-through, as an agent-scope
// relaxed atomic store, which the compiler issues with the sc1 policy.  The
// line then goes on to memory (and the MALL, which still allocates it) while
// the kernel runs, instead of staying dirty in the XCD's L2 until the
// write-back at the end of the kernel, which the next launch on the stream
// waits for.  Measured in the benchmark's cycle of sizes: the C2C LDS
// kernel 3-4% faster per launch up to 2^13 points (2-3% slower at 2^14 and
// 2^15, which keep plain stores) and each four-step pass 1-3% faster.  Rows
// that are not line-aligned (R2C's bins) keep plain stores: partial lines
// written through cost more than they save.
template <bool WT>
__device__ __forceinline__ void store_out(float2* p, float2 x) {
    if constexpr (WT)
        __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), __builtin_bit_cast(unsigned long long, x),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = x;
}

// Real transforms on a half-length complex core (kernels.py:1127-1229
// formulas).  R2C stitch: bin k from core outputs zk = Z[k], zj = Z[L-k]
// and w = exp(-2 pi i k / n): X[k] = a - i w c with a = (zk + conj zj)/2,
// c = (zk - conj zj)/2; `edge` (bins 0 and L) zeroes the imaginary part.
__device__ __forceinline__ float2 r2c_bin(float2 zk, float2 zj, float2 w, float scale, bool edge) {
    const float ar = 0.5f * (zk.x + zj.x), ai = 0.5f * (zk.y - zj.y);
    const float cr = 0.5f * (zk.x - zj.x), ci = 0.5f * (zk.y + zj.y);
    const float xr = ar + (w.x * ci + w.y * cr);
    const float xi = edge ? 0.0f : ai - (w.x * cr - w.y * ci);
    return make_float2(xr * scale, xi * scale);
}
// C2R pre-twiddle: core input Z[k] from bins xk = X[k], xj = X[L-k] and
// t = exp(-2 pi i k / n): Z[k] = a + i conj(t) c (callers zero the imaginary
// parts of bins 0 and L).
__device__ __forceinline__ float2 c2r_pre_bin(float2 xk, float2 xj, float2 t) {
    const float ar = 0.5f * (xk.x + xj.x), ai = 0.5f * (xk.y - xj.y);
    const float cr = 0.5f * (xk.x - xj.x), ci = 0.5f * (xk.y + xj.y);
    const float wr = t.x, wi = -t.y;
    return make_float2(ar - (wr * ci + wi * cr), ai + (wr * cr - wi * ci));
}

// p + bytes for a wave-uniform p and a 32-bit lane offset: the address then
// takes the scalar-base + 32-bit vector-offset form (one VGPR per access, no
// 64-bit address arithmetic per element).  Offsets stay below 2^23 bytes
// because they never leave one transform of at most 2^20 points (or one
// twiddle table).
template <typename T>
__device__ __forceinline__ T* byte_off(T* p, uint32_t bytes) {
    using B = std::conditional_t<std::is_const<T>::value, const char, char>;
    return reinterpret_cast<T*>(reinterpret_cast<B*>(p) + bytes);
}
// For a wave-uniform element offset (kept in SGPRs): stops the loop optimizer
// from turning per-element addresses into one 64-bit pointer register per
// access.  (An offset, not a pointer, so the pointer stays a known global one.)
__device__ __forceinline__ int64_t opaque_uniform(int64_t x) {
    asm volatile("" : "+s"(x));
    return x;
}

// Multiply v[OFF + q] (q = 1..R-1) by W^(q*k) of a pass whose table rows
// `tp[i*NS + k]` hold W^(2^i * k): loads the log2(R) power-of-two roots
// (coalesced across lanes) and composes the rest, w_q = w_(q - hb) * w_hb,
// one complex product each.
// Radix 32 instead multiplies v[q] by w_(2^i) for every set bit i of q, so
// only log2(R) roots are live (the composed form would hold R of them).
// SROW: address each table row as a scalar base plus the lane's 32-bit
// offset.  Otherwise the compiler forms a 64-bit per-lane pointer per row
// (row offsets beyond the load's immediate range), which costs the 16-wave
// 32768-point kernels, at their 128-VGPR budget, a spilled register; where
// registers are not that scarce the default form schedules better (measured
// 1-3% faster at 2^10-2^17).
template <int R, int DIR, int OFF, bool SROW = false, int E>
__device__ __forceinline__ void pass_twiddle(float2 (&v)[E], const float2* __restrict__ tp, int ns, int k) {
    constexpr int LOGR = ilog2(R);
    auto root = [&](int i) -> float2 {
        if constexpr (SROW) return *byte_off(tp + opaque_uniform((int64_t)i * ns), (uint32_t)k * 8u);
        else return tp[i * ns + k];
    };
    if constexpr (R <= 16) {
        float2 w[R];
        static_for<0, LOGR>([&](auto i) { w[1 << i.value] = root(i.value); });
        static_for<3, R>([&](auto q) {
            constexpr int hb = high_bit(q.value);
            if constexpr (hb != q.value) w[q.value] = cmul(w[q.value - hb], w[hb]);
        });
        static_for<1, R>([&](auto q) { v[OFF + q.value] = cmul_tw<DIR>(v[OFF + q.value], w[q.value]); });
    } else {
        static_for<0, LOGR>([&](auto i) {
            const float2 w = root(i.value);
            static_for<1, R>([&](auto q) {
                if constexpr ((q.value >> i.value) & 1) v[OFF + q.value] = cmul_tw<DIR>(v[OFF + q.value], w);
            });
        });
    }
}

// 32-bit bit reversal of the low `bits` bits (bits in [1, 31]).
__device__ __forceinline__ uint32_t brev_low(uint32_t x, int bits) {
    return __brev(x) >> (32 - bits);
}

}  // namespace mfft
