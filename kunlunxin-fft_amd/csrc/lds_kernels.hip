// lds_kernels.hip -- single-pass LDS-resident FFT for core lengths 1..32768.
//
// One HBM read and one HBM write per element: every transform stays inside
// one workgroup from its first load to its last store.  This is the MI355X
// replacement for the reference's M1 (stages fused in global memory with
// barriers, kernels.py:426-484), M2 (first log2(T) stages as a dense matmul,
// kernels.py:487-532) and M3 (tail stages as XOR-gather maps, kernels.py:
// 925-990): all log2(N) stages run here, with no global round trip between
// them.
//
// Algorithm: Stockham auto-sort (natural order in and out, no bit reversal
// pass).  Pass p with radix R and accumulated span NS handles butterflies
// b in [0, L/R): inputs b + q*L/R, twiddles W_{NS*R}^(q*(b % NS)), an
// in-register radix-R DFT, outputs (b/NS)*NS*R + b%NS + q*NS.  Each thread
// owns E = L/T elements (T threads per transform), i.e. E/R butterflies per
// pass.  Twiddles come from a per-pass table holding, for each span NS, the
// rows W^(k), W^(2k), W^(4k), W^(8k) (k < NS) -- a few coalesced loads per
// butterfly; the other powers are composed with one complex product each.
// Pass 0 reads HBM directly and the last pass writes HBM directly --
// both are unit-stride across the lanes of a transform -- and the passes in
// between exchange through LDS.  With fewer than 16 threads per transform
// those runs are shorter than 128 bytes (and the bin rows of the real modes
// are not aligned); the staged form instead moves the block's rows, one
// contiguous run of memory, through LDS with consecutive lanes on
// consecutive elements, on the way in and out.  LDS addresses carry one pad slot per 16 elements and an odd
// per-transform pitch, which spreads the stride-R Stockham writes over banks.
//
// Modes fused into the same kernel (src/xpu/entry.py:555-587 semantics):
//   0  c2c: core + norm scale in the final store (inverse = conjugated roots)
//   1  r2c: the real input viewed as n/2 complex (x[2k] + i x[2k+1]) is the
//      core input for free; the stitch of kernels.py:1127-1177 runs from LDS
//      (16 or 32 elements per thread and whole waves per transform: in
//      registers across lane pairs, the remainder radix running first; 32
//      elements and 32 lanes per transform: through the output row) and
//      writes the n/2+1 bins with the scale
//   2  c2r: the pre-twiddle of kernels.py:1180-1229 is applied while loading
//      the n/2+1 bins; the inverse core writes the n real samples as n/2
//      complex pairs with scale 2*norm_scale
#include "mfft_device.hpp"
#include "mfft_internal.hpp"

namespace mfft {
namespace {

// Shortest transform whose 16-element exchange goes through LDS one
// component at a time (split), halving its LDS so more blocks share a CU.
constexpr int kSplit16MinLog = 13;

template <int LOGL, int LOGE, int MODE = 0>
struct LdsCfg {
    static constexpr int L = 1 << LOGL;
    static constexpr int LE = sched_le(LOGL, LOGE);  // log2 elements per thread
    static constexpr int E = 1 << LE;
    static constexpr int T = L / E;                        // threads per transform
    static constexpr int WG = T >= 256 ? T : 256;          // threads per block
    static constexpr int TPB = WG / T;                     // transforms per block
    static constexpr int P = sched_passes(LOGL, LE);       // passes
    static constexpr bool RF = lds_remainder_first(LOGL, LE, MODE == 1);  // remainder radix first
    // Real and imaginary parts exchanged separately through a float array:
    // half the LDS, twice the barriers.  Always with 32 elements per thread;
    // with 16 from kSplit16MinLog points, except for an r2c kernel without
    // lane pairing, whose 16-element stitch reads whole complex values out
    // of LDS (at 32 elements it stitches through its output row instead).
    static constexpr bool SPLIT =
        LE == 5 || (LE == 4 && LOGL >= kSplit16MinLog && (MODE != 1 || sched_logr(LOGL, LE, P - 1, RF) == LE));
    // Exchange padding: one slot per 16 elements in float2 rows and in the
    // split rows of 16-element threads (pad; a half-wave's stride-16 writes
    // then tile the 64 banks), one per 32 in the split rows of 32-element
    // threads (pad32), so the stride-32 writes of a radix-32 pass land 33
    // floats apart, one bank each, and the two 32-lane transforms of a wave
    // sit half a bank row apart (1056 == 32 mod 64).
    static constexpr int FSH = LE == 5 ? 5 : 4;
    static constexpr int PITCH = LE == 5 ? L + (L >> 5) : L + (L >> 4) + 1;
    static constexpr int LDS_FLOATS = TPB * PITCH * (SPLIT ? 1 : 2);
    // Waves per SIMD the register allocation must allow.  A split-exchange
    // block uses at most 70 KB of LDS, so up to 16 waves of it fit a CU when
    // each wave stays within 128 VGPRs.  The 16-element split blocks (two
    // 16-wave blocks of 16384 points, four 8-wave blocks of 8192) fill a CU
    // when each wave stays within 64 VGPRs: the lane-paired r2c stitch took
    // 71-73 and lost a block per CU (N = 2^15 measured 13% slower).
    static constexpr int MIN_WAVES = SPLIT ? (LE == 4 ? 8 : 4) : 1;
    // Lane pairing of the real modes with 8, 16 or 32 elements per thread
    // (the 32-element registers have no room for the mirror values, and it
    // saves the 8- and 16-element kernels an LDS round trip): when whole waves make
    // up a transform and the pass next to HBM has the full radix (c2r: the
    // first pass, always; r2c: the last, as its remainder runs first), thread
    // t plays Stockham index pair_j(t), which puts the indices j and T - j
    // in lanes l and l ^ 32 of one wave.  The mirror L - k of every bin
    // k = j + T*q a thread holds is then its partner lane's element
    // E - 1 - q, one lane swap away (j = 0 and j = T/2 pair with
    // themselves).
    static constexpr bool PAIR =
        LE >= 3 && T >= 64 && (MODE == 2 || (MODE == 1 && sched_logr(LOGL, LE, P - 1, RF) == LE));
    static constexpr int logr(int p) { return sched_logr(LOGL, LE, p, RF); }
    static constexpr int lns(int p) { return sched_lns_rf(LOGL, LE, p, RF); }
};

__device__ __forceinline__ int pad(int i) { return i + (i >> 4); }
// pad(i + K) from pi = pad(i), for a compile-time K: when K is a multiple of
// 16 it is pi + K + K/16, a constant offset the LDS instruction encodes, so
// a run of accesses shares one address register.
template <int K>
__device__ __forceinline__ int pad_add(int pi, int i) {
    if constexpr (K % 16 == 0) return pi + K + K / 16;
    else return pad(i + K);
}
// the same with one slot per 2^SH elements (split exchange rows)
template <int SH>
__device__ __forceinline__ int padf(int i) { return i + (i >> SH); }
template <int SH, int K>
__device__ __forceinline__ int padf_add(int pi, int i) {
    if constexpr (K % (1 << SH) == 0) return pi + K + (K >> SH);
    else return padf<SH>(i + K);
}

// Stockham index of thread t of a T-thread transform under lane pairing:
// lanes 0-31 of wave w take 32w + l, lanes 32-63 take T - (32w + l - 32),
// except that lane 32 of wave 0 takes T/2 (T - 0 would be index 0 again).
template <int T>
__device__ __forceinline__ int pair_j(int t) {
    const int l = t & 63;
    const int u = ((t >> 6) << 5) + (l & 31);
    return l < 32 ? u : (u == 0 ? T / 2 : T - u);
}
// the value lane l ^ 32 holds
__device__ __forceinline__ float2 swap_halves(float2 x) {
    return make_float2(__shfl_xor(x.x, 32), __shfl_xor(x.y, 32));
}

// STAGED (fewer than 16 threads per transform): the block's TPB rows are
// one contiguous run of memory (L complex values per row in and out of the
// core; L + 1 bins per row of the R2C output and the C2R input); they come
// in and go out through LDS, lane-consecutive, instead of straight between
// HBM and the registers of pass 0 / the last pass or the stitch.
template <int LOGL, int LOGE, int DIR, int MODE, bool STAGED = false>
__global__ __launch_bounds__((LdsCfg<LOGL, LOGE, MODE>::WG), (LdsCfg<LOGL, LOGE, MODE>::MIN_WAVES)) void lds_fft_kernel(
    const void* __restrict__ src_v, void* __restrict__ dst_v, const float2* __restrict__ tw,
    const float2* __restrict__ tw_real, int64_t rows, float scale, int stag_wave, int stag_cus, int stag_n) {
    using C = LdsCfg<LOGL, LOGE, MODE>;
    constexpr int L = C::L, E = C::E, T = C::T, P = C::P;
    static_assert(!STAGED || (T < 16 && !C::SPLIT && !C::PAIR && C::TPB * L == C::WG * E),
                  "the staged form is for transforms of fewer than 16 threads");
    // rows of L + 1 bins (R2C output, C2R input) of the staged form, flat in LDS
    static_assert(!STAGED || C::TPB * (L + 1) <= (C::LDS_FLOATS / 2), "staged bin rows exceed the LDS rows");
    constexpr bool NEED_LDS = (P > 1) || (MODE == 1) || STAGED;
    // write-through output stores (store_out) for C2C up to 2^13 points,
    // where every store instruction writes whole 128-byte lines: the staged
    // form, or 16 or more threads per transform (with fewer, the direct
    // stores are 8-64-byte pieces of lines, and written through one by one
    // they took N = 16 from 126 to 158 us per 256 MiB).  Measured over the
    // benchmark's cycles: C2C 2.5% less time in all; at 2^14 and 2^15 the
    // kernel itself is 2-3% slower with them; C2R's real rows gain by
    // themselves but the transform after them (R2C, whose bin rows of L + 1
    // values are not line-aligned and take partial-line writes) loses more,
    // so both real modes keep plain stores.
    constexpr bool WT = MODE == 0 && LOGL <= 13 && (STAGED || T >= 16);
    static_assert(!(C::SPLIT && MODE == 1 && C::LE != 5 && !C::PAIR),
                  "16-element r2c kernels without lane pairing stitch whole complex values out of LDS");
    __shared__ float2 lds_raw[NEED_LDS ? (C::LDS_FLOATS + 1) / 2 : 1];
    float2* const lds = lds_raw;
    float* const ldsf = reinterpret_cast<float*>(lds_raw);

    // Start stagger (block-uniform): the blocks of the first wave (the first
    // stag_wave in dispatch order) that land on the upper half of the
    // stag_cus CUs of their XCD (blocks go round-robin over the 8 XCDs, so
    // block b is the (b / 8)-th of its XCD) sleep stag_n x 8128 clocks before
    // loading.  With few blocks per CU every CU otherwise loads, computes and
    // stores in lockstep, round after round, and HBM idles through the common
    // compute phase; offsetting half of every XCD's CUs by about half a
    // block period makes one half load and store while the other computes.
    if (stag_n > 0 && (int)blockIdx.x < stag_wave && (int)((blockIdx.x >> 3) % stag_cus) >= (stag_cus >> 1)) {
        for (int q = 0; q < stag_n; ++q) __builtin_amdgcn_s_sleep(127);
    }
    const int tid = threadIdx.x;
    const int tl = tid / T;
    const int j = C::PAIR ? pair_j<T>(tid & (T - 1)) : tid & (T - 1);
    const int64_t row = (int64_t)blockIdx.x * C::TPB + tl;
    const bool active = row < rows;
    float2* lt = lds + (NEED_LDS ? tl * C::PITCH : 0);
    float* ltf = ldsf + (NEED_LDS ? tl * C::PITCH : 0);

    float2 v[E];

    // ---- pass-0 operands straight from HBM
    {
        constexpr int R0 = 1 << C::logr(0);
        constexpr int NB0 = E / R0;
        if constexpr (STAGED && MODE == 2) {
            // the block's TPB rows of L + 1 bins, lane-consecutive, into a
            // flat LDS array; each core input then pairs bin i with bin L - i
            // out of LDS (bin 0 with bin L, both imaginary parts ignored)
            const float2* src = (const float2*)src_v + (int64_t)blockIdx.x * C::TPB * (L + 1);
            const int64_t here = rows - (int64_t)blockIdx.x * C::TPB;
            static_for<0, E + 1>([&](auto r) {
                const int k = tid + r.value * C::WG;
                if (k < C::TPB * (L + 1) && k / (L + 1) < here) lds[k] = load_nt(src + k);
            });
            __syncthreads();
            const float2* xb = lds + tl * (L + 1);
            static_for<0, NB0>([&](auto m) {
                static_for<0, R0>([&](auto q) {
                    const int i = j + m.value * T + q.value * (L / R0);
                    float2 xk = xb[i];
                    float2 xj = xb[L - i];
                    if (i == 0) {
                        xk.y = 0.0f;
                        xj.y = 0.0f;
                    }
                    v[m.value * R0 + q.value] = c2r_pre_bin(xk, xj, tw_real[i]);
                });
            });
        } else if constexpr (MODE == 2 && C::PAIR) {
            // Each bin is loaded once (non-temporal), v[q] = X[j + T*q]; the
            // mirror of bin j + T*q is the partner lane's v[E-1-q], except for
            // j = T/2 (its own v[E-1-q]) and j = 0 (its own v[E-q], and bin L
            // for q = 0, loaded by that thread).  The pairs (s, E-1-s) are
            // turned into core inputs from s = E/2 - 1 down to 0, so what
            // j = 0 reads is still the bin: v[E-s] belongs to a later pair,
            // and v[s+1], already turned, was kept in `prev`.
            static_assert(R0 == E && NB0 == 1, "lane pairing needs a full radix first pass");
            const float2* xb = (const float2*)src_v + row * (L + 1);
            static_for<0, E>([&](auto q) {
                v[q.value] = active ? load_nt(xb + j + q.value * T) : make_float2(0.0f, 0.0f);
            });
            const bool jz = j == 0, jh = j == T / 2;
            const float2 xny = (active && jz) ? load_nt(xb + L) : make_float2(0.0f, 0.0f);
            // exp(-2 pi i (j + T*s) / 2L) = tw_real[j] * exp(-2 pi i s / 2E):
            // one table load and compile-time rotations
            const float2 tj = tw_real[j];
            float2 prev = make_float2(0.0f, 0.0f);
            static_for<0, E / 2>([&](auto ss) {
                constexpr int s = E / 2 - 1 - ss.value;
                constexpr int sb = E - 1 - s;
                const float2 a = v[s], b = v[sb];
                const float2 pa = swap_halves(b), pb = swap_halves(a);
                // selects, not branches: the lane's own values for j = 0
                // (bin 0 pairs with bin L, both imaginary parts ignored; bin
                // L/2 is its own mirror) and j = T/2, the partner's otherwise
                float2 xa = a;
                float2 ma, mb;
                if constexpr (s == 0) {
                    xa.y = jz ? 0.0f : a.y;
                    ma = jz ? make_float2(xny.x, 0.0f) : (jh ? b : pa);
                } else {
                    ma = jz ? v[E - s] : (jh ? b : pa);
                }
                if constexpr (s == E / 2 - 1) mb = jz ? b : (jh ? a : pb);
                else mb = jz ? prev : (jh ? a : pb);
                v[s] = c2r_pre_bin(xa, ma, rot<2 * E, s, -1>(tj));
                v[sb] = c2r_pre_bin(b, mb, rot<2 * E, sb, -1>(tj));
                prev = a;
                // keeps the scheduler from hoisting later pairs' lane swaps,
                // whose results would not fit the registers beside v
                __builtin_amdgcn_sched_barrier(0);
            });
        } else if constexpr (MODE == 2 && P > 1 && C::LE < 5) {
            // Each bin is loaded once (non-temporal); the partner bin L - i
            // of the pre-twiddle comes from the thread that loaded it,
            // through LDS, one component at a time (the exchange rows hold L
            // floats): real parts first, kept in px, then imaginary parts,
            // on which the pre-twiddle is applied.  Bin L, the partner of
            // bin 0, is loaded by thread 0, which holds bin 0.
            const float2* xb = (const float2*)src_v + row * (L + 1);
            static_for<0, NB0>([&](auto m) {
                static_for<0, R0>([&](auto q) {
                    const int i = j + m.value * T + q.value * (L / R0);
                    v[m.value * R0 + q.value] = active ? load_nt(xb + i) : make_float2(0.0f, 0.0f);
                });
            });
            const float2 xny = (active && j == 0) ? load_nt(xb + L) : make_float2(0.0f, 0.0f);
            const int pjf = padf<C::FSH>(j);
            float px[E];
            static_for<0, 2>([&](auto comp) {
                if constexpr (comp.value > 0) __syncthreads();  // the real parts have been read
                static_for<0, NB0>([&](auto m) {
                    static_for<0, R0>([&](auto q) {
                        const float2 x = v[m.value * R0 + q.value];
                        ltf[padf_add<C::FSH, m.value * T + q.value * (L / R0)>(pjf, j)] =
                            comp.value == 0 ? x.x : x.y;
                    });
                });
                __syncthreads();
                static_for<0, NB0>([&](auto m) {
                    static_for<0, R0>([&](auto q) {
                        constexpr int e = m.value * R0 + q.value;
                        const int i = j + m.value * T + q.value * (L / R0);
                        const float y = ltf[padf<C::FSH>((L - i) & (L - 1))];
                        if constexpr (comp.value == 0) {
                            px[e] = y;
                        } else {
                            float2 xk = v[e];
                            float2 xj = make_float2(px[e], y);
                            if (e == 0 && j == 0) {  // bin 0 pairs with bin L; both imaginary parts ignored
                                xj = xny;
                                xk.y = 0.0f;
                                xj.y = 0.0f;
                            }
                            v[e] = c2r_pre_bin(xk, xj, tw_real[i]);
                        }
                    });
                });
            });
        } else if constexpr (MODE == 2) {
            // single-pass lengths, and 32 elements per thread with one
            // transform per 32 lanes (no lane pairing; the partner values
            // would not fit the register budget): both bins straight from
            // global memory
            const float2* xb = (const float2*)src_v + row * (L + 1);
            static_for<0, NB0>([&](auto m) {
                static_for<0, R0>([&](auto q) {
                    const int i = j + m.value * T + q.value * (L / R0);
                    float2 z = make_float2(0.0f, 0.0f);
                    if (active) {
                        float2 xk = xb[i];
                        float2 xj = xb[L - i];
                        if (i == 0) {
                            xk.y = 0.0f;
                            xj.y = 0.0f;
                        }
                        z = c2r_pre_bin(xk, xj, tw_real[i]);
                    }
                    v[m.value * R0 + q.value] = z;
                });
            });
        } else if constexpr (STAGED) {
            // C2C, and R2C's real rows viewed as L complex values: element k
            // of the block's run belongs to row k / L; one load instruction
            // covers 64 consecutive elements
            const float2* src = (const float2*)src_v + (int64_t)blockIdx.x * C::TPB * L;
            const int64_t here = rows - (int64_t)blockIdx.x * C::TPB;  // transforms of this block that exist
            static_for<0, E>([&](auto r) {
                const int k = tid + r.value * C::WG;
                if ((k >> LOGL) < here) lds[(k >> LOGL) * C::PITCH + pad(k & (L - 1))] = load_nt(src + k);
            });
            __syncthreads();
            const int pj = pad(j);
            static_for<0, NB0>([&](auto m) {
                static_for<0, R0>([&](auto q) {
                    v[m.value * R0 + q.value] = lt[pad_add<m.value * T + q.value * (L / R0)>(pj, j)];
                });
            });
        } else {
            // non-temporal: every input element is read exactly once, and
            // keeping it out of L2 and the MALL measured 5-10% faster
            const float2* src = (const float2*)src_v + row * L;
            static_for<0, NB0>([&](auto m) {
                static_for<0, R0>([&](auto q) {
                    const int i = j + m.value * T + q.value * (L / R0);
                    v[m.value * R0 + q.value] = active ? load_nt(src + i) : make_float2(0.0f, 0.0f);
                });
            });
        }
    }

    // ---- Stockham passes
    static_for<0, P>([&](auto pp) {
        constexpr int p = pp.value;
        constexpr int LR = C::logr(p);
        constexpr int R = 1 << LR;
        constexpr int NB = E / R;
        constexpr int LNS = C::lns(p);
        constexpr int NS = 1 << LNS;
        const int pj = pad(j), pjf = padf<C::FSH>(j);
        if constexpr (p > 0 && !C::SPLIT) {
            static_for<0, NB>([&](auto m) {
                static_for<0, R>([&](auto q) {
                    v[m.value * R + q.value] = lt[pad_add<m.value * T + q.value * (L / R)>(pj, j)];
                });
            });
        }
        static_for<0, NB>([&](auto m) {
            if constexpr (NS > 1) {
                const int b = j + m.value * T;
                constexpr int TW_OFF = sched_tw_off(LOGL, C::LE, p, C::RF);
                pass_twiddle<R, DIR, m.value * R, (C::WG == 1024 && E == 32)>(v, tw + TW_OFF, NS, b & (NS - 1));
            }
            dft<R, DIR, m.value * R, 1>(v);
        });
        if constexpr ((p < P - 1 || (MODE == 1 && !C::PAIR)) && !C::SPLIT) {
            // every thread has read this pass's inputs (pass 0 of c2r: the partner bins)
            if constexpr (p > 0 || (MODE == 2 && !C::PAIR) || STAGED) __syncthreads();
            static_for<0, NB>([&](auto m) {
                const int b = j + m.value * T;
                const int base = ((b >> LNS) << (LNS + LR)) + (b & (NS - 1));
                const int pb = pad(base);
                static_for<0, R>([&](auto q) { lt[pad_add<q.value * NS>(pb, base)] = v[m.value * R + q.value]; });
            });
            __syncthreads();
        }
        if constexpr (p < P - 1 && C::SPLIT) {
            // Exchange with the next pass one component at a time.  The real
            // parts are written from v[].x (this pass's layout) and read back
            // into v[].x (the next pass's layout) while v[].y still holds this
            // pass's imaginary parts; then the same for .y.
            constexpr int LR1 = C::logr(p + 1);
            constexpr int R1 = 1 << LR1;
            constexpr int NB1 = E / R1;
            static_for<0, 2>([&](auto comp) {
                __syncthreads();  // the previous readers of this LDS are done
                static_for<0, NB>([&](auto m) {
                    const int b = j + m.value * T;
                    const int base = ((b >> LNS) << (LNS + LR)) + (b & (NS - 1));
                    const int pb = padf<C::FSH>(base);
                    static_for<0, R>([&](auto q) {
                        const float2 x = v[m.value * R + q.value];
                        ltf[padf_add<C::FSH, q.value * NS>(pb, base)] = comp.value == 0 ? x.x : x.y;
                    });
                });
                __syncthreads();
                static_for<0, NB1>([&](auto m) {
                    static_for<0, R1>([&](auto q) {
                        const float x = ltf[padf_add<C::FSH, m.value * T + q.value * (L / R1)>(pjf, j)];
                        if constexpr (comp.value == 0) v[m.value * R1 + q.value].x = x;
                        else v[m.value * R1 + q.value].y = x;
                    });
                });
            });
        }
    });

    // ---- epilogue
    if constexpr (MODE == 1 && C::PAIR) {
        // r2c under lane pairing: v[q] = Z[j + T*q] and the mirror of
        // Z[j + T*q] is the partner lane's v[E-1-q] (own v[E-1-q] for
        // j = T/2, own v[(E-q) mod E] for j = 0), so every bin is stitched
        // in registers and stored once; thread j = 0 also writes bin L.
        static_assert(C::logr(P - 1) == C::LE, "lane pairing needs a full radix last pass");
        float2* xo = (float2*)dst_v + row * (L + 1);
        const bool jz = j == 0, jh = j == T / 2;
        // A transform spans whole waves, so `active` is wave-uniform and the
        // lane swaps run with every lane of the wave or none.
        if (active) {
            const float2 tj = tw_real[j];  // tw_real[j + T*s] = tj * exp(-2 pi i s / 2E)
            static_for<0, E / 2>([&](auto ss) {
                constexpr int s = ss.value;
                constexpr int sb = E - 1 - s;
                const float2 a = v[s], b = v[sb];
                const float2 pa = swap_halves(b), pb = swap_halves(a);
                const float2 ma = jz ? v[(E - s) % E] : (jh ? b : pa);
                const float2 mb = jz ? v[s + 1] : (jh ? a : pb);
                xo[j + s * T] = r2c_bin(a, ma, rot<2 * E, s, -1>(tj), scale, s == 0 && jz);
                xo[j + sb * T] = r2c_bin(b, mb, rot<2 * E, sb, -1>(tj), scale, false);
                __builtin_amdgcn_sched_barrier(0);
            });
            if (jz) xo[L] = r2c_bin(v[0], v[0], tw_real[L], scale, true);
        }
    } else if constexpr (MODE == 1 && C::SPLIT) {
        // r2c with 32 elements per thread and no lane pairing (the last
        // pass has a smaller radix, or 32 lanes hold a transform): the split
        // LDS rows hold one component at a time and the registers have no
        // room for the mirror values, so the core outputs z go to the output
        // row itself (L of its L + 1 bins), and each thread then turns disjoint mirror pairs
        // (k, L - k) into bins in place: it alone reads and writes those two
        // addresses, so no thread overwrites a value another still needs.
        // The row was last written by this block's own waves (same CU and
        // L1), so completed stores and a barrier make them visible; the
        // reads mostly hit L2.
        constexpr int LR = C::logr(P - 1);
        constexpr int R = 1 << LR;
        constexpr int NB = E / R;
        constexpr int NS = L / R;
        float2* xo = (float2*)dst_v + row * (L + 1);
        if (active) {
            static_for<0, NB>([&](auto m) {
                const int b = j + m.value * T;
                static_for<0, R>([&](auto q) { xo[b + q.value * NS] = v[m.value * R + q.value]; });
            });
        }
        __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are complete
        __syncthreads();                // ... and every other thread's
        if (active) {
            for (int k = j; k <= L / 2; k += T) {
                const float2 zk = xo[k];
                const float2 zj = xo[(L - k) & (L - 1)];
                xo[k] = r2c_bin(zk, zj, tw_real[k], scale, k == 0);
                if (k == 0) xo[L] = r2c_bin(zk, zj, tw_real[L], scale, true);
                else if (k != L / 2) xo[L - k] = r2c_bin(zj, zk, tw_real[L - k], scale, false);
            }
        }
    } else if constexpr (MODE == 1 && STAGED) {
        // the stitch of every bin this thread owns into registers, then the
        // block's TPB rows of L + 1 bins out through a flat LDS array,
        // lane-consecutive
        float2 bins[E];
        static_for<0, E>([&](auto m) {
            const int k = j + m.value * T;
            bins[m.value] = r2c_bin(lt[pad(k)], lt[pad((L - k) & (L - 1))], tw_real[k], scale, k == 0);
        });
        const float2 last = r2c_bin(lt[pad(0)], lt[pad(0)], tw_real[L], scale, true);
        __syncthreads();  // every stitch read of the core outputs is done
        float2* xs = lds + tl * (L + 1);
        static_for<0, E>([&](auto m) { xs[j + m.value * T] = bins[m.value]; });
        if (j == 0) xs[L] = last;
        __syncthreads();
        float2* xo = (float2*)dst_v + (int64_t)blockIdx.x * C::TPB * (L + 1);
        const int64_t here = rows - (int64_t)blockIdx.x * C::TPB;
        static_for<0, E + 1>([&](auto r) {
            const int k = tid + r.value * C::WG;
            if (k < C::TPB * (L + 1) && k / (L + 1) < here) xo[k] = lds[k];
        });
    } else if constexpr (MODE == 1) {
        // r2c stitch out of LDS: bins k in [0, L], X[k] = a - i*w*c
        float2* xo = (float2*)dst_v + row * (L + 1);
        if (active) {
            auto stitch = [&](int k) {
                const float2 zk = lt[pad(k & (L - 1))];
                const float2 zj = lt[pad((L - k) & (L - 1))];
                xo[k] = r2c_bin(zk, zj, tw_real[k], scale, k == 0 || k == L);
            };
            static_for<0, E>([&](auto m) { stitch(j + m.value * T); });
            if (j == 0) stitch(L);
        }
    } else if constexpr (STAGED) {
        constexpr int LR = C::logr(P - 1);
        constexpr int R = 1 << LR;
        constexpr int NB = E / R;
        constexpr int NS = L / R;
        __syncthreads();  // every read of the last pass's operands from LDS is done
        static_for<0, NB>([&](auto m) {
            const int b = j + m.value * T;
            const int pb = pad(b);
            static_for<0, R>([&](auto q) { lt[pad_add<q.value * NS>(pb, b)] = v[m.value * R + q.value]; });
        });
        __syncthreads();
        float2* dst = (float2*)dst_v + (int64_t)blockIdx.x * C::TPB * L;
        const int64_t here = rows - (int64_t)blockIdx.x * C::TPB;
        static_for<0, E>([&](auto r) {
            const int k = tid + r.value * C::WG;
            if ((k >> LOGL) < here)
                store_out<WT>(dst + k, cscale(lds[(k >> LOGL) * C::PITCH + pad(k & (L - 1))], scale));
        });
    } else {
        constexpr int LR = C::logr(P - 1);
        constexpr int R = 1 << LR;
        constexpr int NB = E / R;
        constexpr int NS = L / R;
        float2* dst = (float2*)dst_v + row * L;
        if (active) {
            static_for<0, NB>([&](auto m) {
                const int b = j + m.value * T;
                static_for<0, R>([&](auto q) {
                    store_out<WT>(dst + b + q.value * NS, cscale(v[m.value * R + q.value], scale));
                });
            });
        }
    }
}

// Arguments of one LDS launch, passed down the template dispatch.
struct LdsArgs {
    const void* src;
    void* dst;
    const float2* tw;
    const float2* tw_real;
    int64_t rows;
    float scale;
    hipStream_t stream;
    int num_cus;  // compute units of the device (start stagger)
    int stagger;  // start stagger, s_sleep(127) units (0 = off)
    bool staged;  // C2C of fewer than 16 threads per transform: in and out through LDS
};

template <int LOGL, int LOGE, int DIR, int MODE, bool STAGED = false>
hipError_t launch_one(const LdsArgs& a) {
    using C = LdsCfg<LOGL, LOGE>;
    const int64_t blocks = (a.rows + C::TPB - 1) / C::TPB;
    if (blocks <= 0) return hipSuccess;
    if (!launch_fits(blocks, C::WG)) return hipErrorInvalidConfiguration;
    int wave_blocks = 0, n = 0;
    if (a.stagger > 0 && a.num_cus >= 16) {
        // blocks one wave of the grid holds (occupancy query, once per kernel)
        static const int per_cu = [] {
            int b = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, lds_fft_kernel<LOGL, LOGE, DIR, MODE, STAGED>, C::WG,
                                                             0) !=
                hipSuccess) {
                (void)hipGetLastError();
                b = 0;
            }
            return b;
        }();
        const int64_t wave = (int64_t)per_cu * a.num_cus;
        // only when the launch runs at least two waves of blocks
        if (wave > 0 && blocks >= 2 * wave) wave_blocks = (int)wave, n = a.stagger;
    }
    lds_fft_kernel<LOGL, LOGE, DIR, MODE, STAGED><<<(unsigned)blocks, C::WG, 0, a.stream>>>(
        a.src, a.dst, a.tw, a.tw_real, a.rows, a.scale, wave_blocks, a.num_cus / 8, n);
    mark(a.stream);
    return hipGetLastError();
}

template <int LOGL, int LOGE>
hipError_t dispatch_mode(int mode, int dir, const LdsArgs& a) {
    if constexpr (LdsCfg<LOGL, LOGE>::T < 16) {
        if (a.staged) {
            if (mode == 0)
                return dir < 0 ? launch_one<LOGL, LOGE, -1, 0, true>(a) : launch_one<LOGL, LOGE, 1, 0, true>(a);
            if (mode == 1) return launch_one<LOGL, LOGE, -1, 1, true>(a);
            return launch_one<LOGL, LOGE, 1, 2, true>(a);
        }
    }
    if (a.staged) return hipErrorInvalidValue;  // refused at plan creation
    if (mode == 0) return dir < 0 ? launch_one<LOGL, LOGE, -1, 0>(a) : launch_one<LOGL, LOGE, 1, 0>(a);
    if (mode == 1) return launch_one<LOGL, LOGE, -1, 1>(a);
    return launch_one<LOGL, LOGE, 1, 2>(a);
}

// 32 elements per thread (split exchange)
template <int LOGL>
hipError_t dispatch_split(int mode, int dir, const LdsArgs& a) {
    if (a.staged) return hipErrorInvalidValue;  // 32 elements: at least 32 threads per transform
    if (mode == 0) return dir < 0 ? launch_one<LOGL, 5, -1, 0>(a) : launch_one<LOGL, 5, 1, 0>(a);
    if (mode == 1) return launch_one<LOGL, 5, -1, 1>(a);
    if (mode == 2) return launch_one<LOGL, 5, 1, 2>(a);
    return hipErrorInvalidValue;
}

template <int LOGL>
hipError_t dispatch_elems(int loge, int mode, int dir, const LdsArgs& a) {
    if constexpr (LOGL >= 10) {
        if (loge == 5) return dispatch_split<LOGL>(mode, dir, a);
    }
    switch (loge) {
        case 2: return dispatch_mode<LOGL, 2>(mode, dir, a);
        case 3: return dispatch_mode<LOGL, 3>(mode, dir, a);
        default: return dispatch_mode<LOGL, 4>(mode, dir, a);
    }
}

}  // namespace

bool lds_supported(int log2l, int elems) {
    if (log2l < 0 || log2l > kMaxLdsLog2) return false;
    if (elems != 0 && elems != 4 && elems != 8 && elems != 16 && elems != 32) return false;
    // 32 elements per thread (split exchange) exist for 2^10..2^15 (the r2c
    // stitch then runs through the output row); 8192 and 16384 points take
    // 16 or 32; 32768 only 32
    if (elems == 32 && log2l < 10) return false;
    if (log2l >= 13 && elems != 0 && elems < 16) return false;
    if (log2l == 15 && elems != 0 && elems != 32) return false;
    return true;
}

int lds_default_elems(int log2l) {
    if (log2l <= 4) return 16;  // one thread holds the whole transform (min(L, 16))
    if (log2l <= 6) return 8;
    if (log2l >= 15) return 32;
    return 16;
}

int lds_threads_per_block(int log2l, int elems) {
    int le = ilog2(elems);
    if (le > log2l) le = log2l;
    const int t = 1 << (log2l - le);
    return t >= 256 ? t : 256;
}

bool lds_staged_supported(int log2l, int elems) {
    const int le = ilog2(elems) < log2l ? ilog2(elems) : log2l;
    return lds_supported(log2l, elems) && elems != 0 && elems != 32 && (log2l - le) < 4;
}

hipError_t launch_lds(int mode, int dir, int log2l, int elems, const void* src, void* dst,
                      const float2* tw, const float2* tw_real, int64_t rows, float scale,
                      hipStream_t stream, int num_cus, int stagger, bool staged) {
    const int loge = ilog2(elems);
    const LdsArgs a{src, dst, tw, tw_real, rows, scale, stream, num_cus, stagger, staged};
    switch (log2l) {
        case 0: return dispatch_elems<0>(loge, mode, dir, a);
        case 1: return dispatch_elems<1>(loge, mode, dir, a);
        case 2: return dispatch_elems<2>(loge, mode, dir, a);
        case 3: return dispatch_elems<3>(loge, mode, dir, a);
        case 4: return dispatch_elems<4>(loge, mode, dir, a);
        case 5: return dispatch_elems<5>(loge, mode, dir, a);
        case 6: return dispatch_elems<6>(loge, mode, dir, a);
        case 7: return dispatch_elems<7>(loge, mode, dir, a);
        case 8: return dispatch_elems<8>(loge, mode, dir, a);
        case 9: return dispatch_elems<9>(loge, mode, dir, a);
        case 10: return dispatch_elems<10>(loge, mode, dir, a);
        case 11: return dispatch_elems<11>(loge, mode, dir, a);
        case 12: return dispatch_elems<12>(loge, mode, dir, a);
        case 13: return dispatch_elems<13>(loge, mode, dir, a);
        case 14: return dispatch_elems<14>(loge, mode, dir, a);
        case 15: return dispatch_split<15>(mode, dir, a);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mfft
