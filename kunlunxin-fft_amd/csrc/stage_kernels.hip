// stage_kernels.hip -- the reference's global-stage flows on gfx950, plus the
// standalone real-transform prologue/epilogue kernels.
//
// These keep the index maps of the reference's M0 / M5 flows (one launch and
// one HBM round trip per stage), because they are the selector's baseline and
// its closed fallback:
//   radix-2 DIT stage  src/xpu/kernels.py:100-163  (j = k % n, i = (k/n)*2n + j,
//                      b = X[i+n]*W[j*M], Y[i] = a+b, Y[i+n] = a-b, M = N/2n;
//                      bit reversal folded into stage 0's loads)
//   radix-2 DIF stage  kernels.py:166-236  ((a+b, (a-b)*W); bit or mixed digit
//                      reversal folded into the last stage's stores)
//   radix-4 DIT/DIF    kernels.py:239-423  (span 4n, twiddles W^(d*j*M), d=1..3;
//                      mixed radix-4/2 digit reversal of kernels.py:41-78)
// Differences on purpose: data are interleaved complex64 (one 8-byte load per
// element instead of two planar ones), the batch is folded into a 1-D grid,
// the twiddle table holds all N roots (so W^(3jM) needs no conjugate fold), and
// the inverse / norm epilogue is fused into the stages (conjugated roots and a
// scaled final store) instead of two extra passes.
#include "mfft_device.hpp"
#include "mfft_internal.hpp"

namespace mfft {
namespace {

// mixed radix-4/2 digit reversal for DIT input (kernels.py:41-56 semantics):
// radix-4 digits low to high, an odd top bit lands in bit 0.
__device__ __forceinline__ uint32_t dit_digit_reverse(uint32_t x, int bits) {
    uint32_t rev = 0;
    for (int q = 0; q < bits / 2; ++q) rev |= ((x >> (2 * q)) & 3u) << (bits - 2 * q - 2);
    if (bits & 1) rev |= (x >> (bits - 1)) & 1u;
    return rev;
}

// DIF output digit reversal (kernels.py:59-78 semantics): with odd bits the
// 1-bit digit sits at the bottom of the index and takes the top weight.
__device__ __forceinline__ uint32_t dif_digit_reverse(uint32_t x, int bits) {
    if ((bits & 1) == 0) return dit_digit_reverse(x, bits);
    uint32_t rev = (x & 1u) << (bits - 1);
    for (int q = 1; q <= bits / 2; ++q) rev |= ((x >> (2 * q - 1)) & 3u) << (bits - 1 - 2 * q);
    return rev;
}

// REV: 0 = natural, 1 = bit reversal, 2 = mixed DIF digit reversal
template <int REV>
__device__ __forceinline__ uint32_t permute_out(uint32_t i, int bits) {
    if constexpr (REV == 1) return brev_low(i, bits);
    else if constexpr (REV == 2) return dif_digit_reverse(i, bits);
    else return i;
}

template <int DIR, bool BITREV_IN>
__global__ void r2_dit_stage(const float2* __restrict__ x, float2* __restrict__ y,
                             const float2* __restrict__ tw, int64_t total, int logn, int log_ns,
                             float scale) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g >> (logn - 1);
    const uint32_t k = (uint32_t)(g & (((int64_t)1 << (logn - 1)) - 1));
    const uint32_t ns = 1u << log_ns;
    const uint32_t j = k & (ns - 1);
    const uint32_t i = ((k >> log_ns) << (log_ns + 1)) + j;
    uint32_t sa = i, sb = i + ns;
    if constexpr (BITREV_IN) {
        sa = brev_low(sa, logn);
        sb = brev_low(sb, logn);
    }
    const float2* xr = x + (row << logn);
    float2* yr = y + (row << logn);
    const float2 a = xr[sa];
    const float2 b = cmul_tw<DIR>(xr[sb], tw[(size_t)j << (logn - 1 - log_ns)]);
    yr[i] = cscale(cadd(a, b), scale);
    yr[i + ns] = cscale(csub(a, b), scale);
}

template <int DIR, int REV_OUT>
__global__ void r2_dif_stage(const float2* __restrict__ x, float2* __restrict__ y,
                             const float2* __restrict__ tw, int64_t total, int logn, int log_ns,
                             float scale) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g >> (logn - 1);
    const uint32_t k = (uint32_t)(g & (((int64_t)1 << (logn - 1)) - 1));
    const uint32_t ns = 1u << log_ns;
    const uint32_t j = k & (ns - 1);
    const uint32_t i = ((k >> log_ns) << (log_ns + 1)) + j;
    const float2* xr = x + (row << logn);
    float2* yr = y + (row << logn);
    const float2 a = xr[i];
    const float2 b = xr[i + ns];
    const float2 d = cmul_tw<DIR>(csub(a, b), tw[(size_t)j << (logn - 1 - log_ns)]);
    yr[permute_out<REV_OUT>(i, logn)] = cscale(cadd(a, b), scale);
    yr[permute_out<REV_OUT>(i + ns, logn)] = cscale(d, scale);
}

template <int DIR, bool DIGREV_IN>
__global__ void r4_dit_stage(const float2* __restrict__ x, float2* __restrict__ y,
                             const float2* __restrict__ tw, int64_t total, int logn, int log_ns,
                             float scale) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g >> (logn - 2);
    const uint32_t off = (uint32_t)(g & (((int64_t)1 << (logn - 2)) - 1));
    const uint32_t ns = 1u << log_ns;
    const uint32_t j = off & (ns - 1);
    const uint32_t i = ((off >> log_ns) << (log_ns + 2)) + j;
    const float2* xr = x + (row << logn);
    float2* yr = y + (row << logn);
    const uint32_t jm = j << (logn - 2 - log_ns);  // j*M, M = N/(4n)
    float2 v[4];
    static_for<0, 4>([&](auto d) {
        uint32_t s = i + d.value * ns;
        if constexpr (DIGREV_IN) s = dit_digit_reverse(s, logn);
        v[d.value] = xr[s];
        if constexpr (d.value > 0) v[d.value] = cmul_tw<DIR>(v[d.value], tw[d.value * jm]);
    });
    dft<4, DIR, 0, 1>(v);
    static_for<0, 4>([&](auto d) { yr[i + d.value * ns] = cscale(v[d.value], scale); });
}

template <int DIR, bool DIGREV_OUT>
__global__ void r4_dif_stage(const float2* __restrict__ x, float2* __restrict__ y,
                             const float2* __restrict__ tw, int64_t total, int logn, int log_ns,
                             float scale) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g >> (logn - 2);
    const uint32_t off = (uint32_t)(g & (((int64_t)1 << (logn - 2)) - 1));
    const uint32_t ns = 1u << log_ns;
    const uint32_t j = off & (ns - 1);
    const uint32_t i = ((off >> log_ns) << (log_ns + 2)) + j;
    const float2* xr = x + (row << logn);
    float2* yr = y + (row << logn);
    const uint32_t jm = j << (logn - 2 - log_ns);
    float2 v[4];
    static_for<0, 4>([&](auto d) { v[d.value] = xr[i + d.value * ns]; });
    dft<4, DIR, 0, 1>(v);
    static_for<0, 4>([&](auto d) {
        float2 o = v[d.value];
        if constexpr (d.value > 0) o = cmul_tw<DIR>(o, tw[d.value * jm]);
        uint32_t s = i + d.value * ns;
        if constexpr (DIGREV_OUT) s = dif_digit_reverse(s, logn);
        yr[s] = cscale(o, scale);
    });
}

__global__ void bitrev_kernel(const float2* __restrict__ x, float2* __restrict__ y, int64_t total,
                              int logn) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g >> logn;
    const uint32_t i = (uint32_t)(g & (((int64_t)1 << logn) - 1));
    const uint32_t r = logn > 0 ? brev_low(i, logn) : 0u;
    y[(row << logn) + r] = x[g];
}

// R2C stitch (kernels.py:1127-1177 formula): X[k] = a - i*w*c with
// a = (Z[k] + conj Z[j])/2, c = (Z[k] - conj Z[j])/2, j = (np-k) % np,
// w = exp(-2*pi*i*k/n); imaginary parts of bins 0 and np are exactly 0.
// One thread per mirror pair (k, np-k), k in [0, np/2]: bin np-k takes the
// same two core outputs with their roles swapped, so every core output is
// read once (non-temporal: it is not read again).  Pair 0 also writes bin
// np (both from Z[0]); pair np/2 is one bin.  The pairs of the whole batch
// are one flat range, np/2 + 1 per row (a launch holds fewer than 2^32, so
// the row is a 32-bit quotient): short rows share a block instead of each
// taking one (N = 16: 5 pairs a row, not 256 threads).
__global__ __launch_bounds__(256) void r2c_stitch_kernel(const float2* __restrict__ z, float2* __restrict__ x,
                                                         const float2* __restrict__ tw_real, int64_t np,
                                                         uint32_t total, float scale) {
    const uint32_t g = blockIdx.x * 256u + threadIdx.x;
    if (g >= total) return;
    const int64_t half = np >> 1;
    const uint32_t pairs = (uint32_t)half + 1u;
    const uint32_t row = g / pairs;
    const int64_t k = g - row * pairs;
    const float2* zr = z + (int64_t)row * np;
    float2* xr = x + (int64_t)row * (np + 1);
    const int64_t j = (np - k) & (np - 1);
    const float2 zk = load_nt(zr + k);
    const float2 zj = load_nt(zr + j);
    xr[k] = r2c_bin(zk, zj, tw_real[k], scale, k == 0);
    if (k == 0) xr[np] = r2c_bin(zk, zj, tw_real[np], scale, true);
    else if (k != half) xr[np - k] = r2c_bin(zj, zk, tw_real[np - k], scale, false);
}

// C2R pre-twiddle (kernels.py:1180-1229 formula): Z[k] = a + i*w'*c with
// a = (X[k] + conj X[j])/2, c = (X[k] - conj X[j])/2, j = np-k,
// w' = exp(+2*pi*i*k/n); imaginary parts of bins 0 and np are ignored.
// Paired like the stitch: thread k in [0, np/2] reads X[k] and X[np-k] once
// and writes Z[k] and Z[np-k] (pair 0 only Z[0]; pair np/2 one value), over
// the same flat range of pairs as the stitch.
__global__ __launch_bounds__(256) void c2r_pre_kernel(const float2* __restrict__ x, float2* __restrict__ z,
                                                      const float2* __restrict__ tw_real, int64_t np, uint32_t total) {
    const uint32_t g = blockIdx.x * 256u + threadIdx.x;
    if (g >= total) return;
    const int64_t half = np >> 1;
    const uint32_t pairs = (uint32_t)half + 1u;
    const uint32_t row = g / pairs;
    const int64_t k = g - row * pairs;
    const float2* xr = x + (int64_t)row * (np + 1);
    float2* zr = z + (int64_t)row * np;
    float2 xk = load_nt(xr + k);
    float2 xj = load_nt(xr + (np - k));
    if (k == 0) {
        xk.y = 0.0f;
        xj.y = 0.0f;
    }
    zr[k] = c2r_pre_bin(xk, xj, tw_real[k]);
    if (k != 0 && k != half) zr[np - k] = c2r_pre_bin(xj, xk, tw_real[np - k]);
}

// The standalone real-flow epilogues of the reference's runner
// (r2c_stitch, c2r_pre, c2r_unpack; src/xpu/runner.py:1687-1767), for a
// caller that runs the half-length core itself.  One thread per output
// value over the flattened batch; the root exp(-2 pi i k / n) comes from
// sinpi/cospi of k / (n/2), exact in float for a power-of-two n, instead of
// a per-plan table, so these need no plan and no allocation.
__device__ __forceinline__ float2 real_root(int64_t k, float inv_np) {
    float sn, cs;
    sincospif((float)k * inv_np, &sn, &cs);  // angle pi k / np = 2 pi k / n
    return make_float2(cs, -sn);
}

// x[row][k], k in [0, np]: the stitch of z[row][k mod np] and z[row][(np-k) mod np]
__global__ __launch_bounds__(256) void r2c_stitch_free_kernel(const float2* __restrict__ z, float2* __restrict__ x,
                                                              int64_t np, int64_t total, float inv_np, float scale) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g / (np + 1);
    const int64_t k = g - row * (np + 1);
    const float2* zr = z + row * np;
    x[g] = r2c_bin(zr[k & (np - 1)], zr[(np - k) & (np - 1)], real_root(k, inv_np), scale, k == 0 || k == np);
}

// z[row][k], k in [0, np): the pre-twiddle of x[row][k] and x[row][np-k]
// (imaginary parts of bins 0 and np ignored)
__global__ __launch_bounds__(256) void c2r_pre_free_kernel(const float2* __restrict__ x, float2* __restrict__ z,
                                                           int64_t np, int64_t total, float inv_np) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g / np;
    const int64_t k = g - row * np;
    const float2* xr = x + row * (np + 1);
    float2 xk = xr[k];
    float2 xj = xr[np - k];
    if (k == 0) {
        xk.y = 0.0f;
        xj.y = 0.0f;
    }
    z[g] = c2r_pre_bin(xk, xj, real_root(k, inv_np));
}

// out[row][2k], out[row][2k+1] = scale * u[row][(np-k) mod np]: the forward
// core's output read in mirror order is the unnormalised inverse transform
// (conj(fft(conj Z))[k] = fft(Z)[(np-k) mod np]), stored as real pairs
__global__ __launch_bounds__(256) void c2r_unpack_kernel(const float2* __restrict__ u, float2* __restrict__ out,
                                                         int64_t np, int64_t total, float scale) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= total) return;
    const int64_t row = g / np;
    const int64_t k = g - row * np;
    out[g] = cscale(u[row * np + ((np - k) & (np - 1))], scale);
}

// Fused twiddle + transpose between the two sub-FFT stages of a composed
// four-step (the reference's one-pass "transpose + twiddle" boundary of
// run_hybrid, adapter_hybrid.py:294-301): for each of `batch` matrices
// S[r][c] (rows x cols, n = rows * cols), G[c][r] = S[r][c] * W_n^(DIR r c).
// 32 x 32 tiles through LDS (one pad column), so both the read of S and the
// write of G are 256-byte runs.  The root comes from sinpi/cospi of the
// index product reduced exactly modulo n (2 e / n is exact in float), not
// from a table.
template <int DIR>
__global__ __launch_bounds__(256) void twiddle_transpose_kernel(const float2* __restrict__ s, float2* __restrict__ g,
                                                               int rows, int cols, int tiles_r, int tiles_c,
                                                               uint32_t nmask, float inv_half_n) {
    __shared__ float2 tile[32][33];
    const int t = blockIdx.x;
    const int per = tiles_r * tiles_c;
    const int64_t bt = t / per;
    const int rem = t - (int)(bt * per);
    const int tr = rem / tiles_c, tc = rem - tr * tiles_c;
    const int r0 = tr * 32, c0 = tc * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
    const float2* sb = s + bt * (int64_t)rows * cols;
    float2* gb = g + bt * (int64_t)rows * cols;
    for (int k = 0; k < 4; ++k) {
        const int r = r0 + ty + 8 * k, c = c0 + tx;
        if (r < rows && c < cols) {
            const uint32_t e = ((uint32_t)r * (uint32_t)c) & nmask;
            float sn, cs;
            sincospif((float)e * inv_half_n, &sn, &cs);  // angle 2 pi e / n
            const float2 w = make_float2(cs, DIR < 0 ? -sn : sn);
            tile[ty + 8 * k][tx] = cmul(load_nt(sb + (int64_t)r * cols + c), w);
        }
    }
    __syncthreads();
    for (int k = 0; k < 4; ++k) {
        const int c = c0 + ty + 8 * k, r = r0 + tx;
        if (r < rows && c < cols) gb[(int64_t)c * rows + r] = tile[tx][ty + 8 * k];
    }
}

// Streaming copy of n16 16-byte words, the rate this device moves bytes
// read once and written once: each thread moves 8 words 256 apart, with
// non-temporal loads and stores.  Of the forms measured on MI355X (8- or
// 16-byte lanes, 4 to 16 words per thread, temporal or non-temporal
// stores; 256 MiB each way after an untimed 256 MiB write) this one was the
// fastest, 6.1-6.2 TB/s read + write.  Not on any transform path: it is
// the practical ceiling the bench measures its transforms against.
typedef float nt_float4 __attribute__((ext_vector_type(4)));
// Whole blocks take a branch-free path: a bounds check per word makes each
// load its own branch, which the compiler closes with a wait for that load,
// so the eight loads no longer overlap (measured 4.3 against 6.1 TB/s).
__global__ __launch_bounds__(256) void stream_copy_kernel(const nt_float4* __restrict__ x,
                                                          nt_float4* __restrict__ y, int64_t n16) {
    const int64_t blk = (int64_t)blockIdx.x * 2048;
    const int64_t base = blk + threadIdx.x;
    nt_float4 v[8];
    if (blk + 2048 <= n16) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = __builtin_nontemporal_load(x + base + q * 256);
#pragma unroll
        for (int q = 0; q < 8; ++q) __builtin_nontemporal_store(v[q], y + base + q * 256);
        return;
    }
    for (int q = 0; q < 8; ++q) {
        const int64_t i = base + q * 256;
        if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(x + i), y + i);
    }
}

inline unsigned grid_for(int64_t total, int block) { return (unsigned)((total + block - 1) / block); }

}  // namespace

hipError_t launch_radix2(bool dif, int dir, const float2* src, float2* dst, float2* scratch,
                         const float2* tw, int64_t n, int64_t rows, float scale, int block,
                         hipStream_t stream, int* launches) {
    const int logn = ilog2((int)n);
    const int64_t total = rows * (n >> 1);
    if (!launch_fits((total + block - 1) / block, block)) return hipErrorInvalidConfiguration;
    const unsigned grid = grid_for(total, block);
    const float2* cur = src;
    int count = 0;
    for (int s = 0; s < logn; ++s) {
        float2* out = ((logn - 1 - s) % 2 == 0) ? dst : scratch;
        const bool last = s == logn - 1;
        const float sc = last ? scale : 1.0f;
        if (!dif) {
            const int log_ns = s;  // half-spans 1, 2, ..., N/2
            if (dir < 0) {
                if (s == 0) r2_dit_stage<-1, true><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
                else r2_dit_stage<-1, false><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
            } else {
                if (s == 0) r2_dit_stage<1, true><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
                else r2_dit_stage<1, false><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
            }
        } else {
            const int log_ns = logn - 1 - s;  // half-spans N/2, ..., 1
            if (dir < 0) {
                if (last) r2_dif_stage<-1, 1><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
                else r2_dif_stage<-1, 0><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
            } else {
                if (last) r2_dif_stage<1, 1><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
                else r2_dif_stage<1, 0><<<grid, block, 0, stream>>>(cur, out, tw, total, logn, log_ns, sc);
            }
        }
        mark(stream);
        ++count;
        cur = out;
    }
    if (launches) *launches = count;
    return hipGetLastError();
}

hipError_t launch_radix4(bool dif, int dir, const float2* src, float2* dst, float2* scratch,
                         const float2* tw, int64_t n, int64_t rows, float scale, int block,
                         hipStream_t stream, int* launches) {
    const int logn = ilog2((int)n);
    const int n4 = logn / 2;          // radix-4 stages
    const bool tail = (logn & 1) != 0;  // one radix-2 stage when log2 N is odd
    const int stages = n4 + (tail ? 1 : 0);
    const int64_t total4 = rows * (n >> 2);
    const int64_t total2 = rows * (n >> 1);
    if (!launch_fits((total2 + block - 1) / block, block)) return hipErrorInvalidConfiguration;
    const unsigned grid4 = grid_for(total4, block);
    const unsigned grid2 = grid_for(total2, block);
    const float2* cur = src;
    for (int s = 0; s < stages; ++s) {
        float2* out = ((stages - 1 - s) % 2 == 0) ? dst : scratch;
        const bool last = s == stages - 1;
        const float sc = last ? scale : 1.0f;
        if (!dif) {
            // runner.py:1367-1383: spans 4, 16, ..., then a radix-2 span-N tail
            if (s < n4) {
                const int log_ns = 2 * s;
                const bool first = s == 0;
                if (dir < 0) {
                    if (first) r4_dit_stage<-1, true><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                    else r4_dit_stage<-1, false><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                } else {
                    if (first) r4_dit_stage<1, true><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                    else r4_dit_stage<1, false><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                }
            } else {
                if (dir < 0) r2_dit_stage<-1, false><<<grid2, block, 0, stream>>>(cur, out, tw, total2, logn, logn - 1, sc);
                else r2_dit_stage<1, false><<<grid2, block, 0, stream>>>(cur, out, tw, total2, logn, logn - 1, sc);
            }
        } else {
            // runner.py:1386-1396: radix-4 groups N, N/4, ..., then a group-2 tail
            if (s < n4) {
                const int log_ns = logn - 2 - 2 * s;
                const bool digrev = last;  // no tail: the last radix-4 stage permutes
                if (dir < 0) {
                    if (digrev) r4_dif_stage<-1, true><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                    else r4_dif_stage<-1, false><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                } else {
                    if (digrev) r4_dif_stage<1, true><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                    else r4_dif_stage<1, false><<<grid4, block, 0, stream>>>(cur, out, tw, total4, logn, log_ns, sc);
                }
            } else {
                if (dir < 0) r2_dif_stage<-1, 2><<<grid2, block, 0, stream>>>(cur, out, tw, total2, logn, 0, sc);
                else r2_dif_stage<1, 2><<<grid2, block, 0, stream>>>(cur, out, tw, total2, logn, 0, sc);
            }
        }
        mark(stream);
        cur = out;
    }
    if (launches) *launches = stages;
    return hipGetLastError();
}

hipError_t launch_bitrev(const float2* src, float2* dst, int64_t n, int64_t rows, hipStream_t stream) {
    const int logn = ilog2((int)n);
    const int64_t total = rows * n;
    if (total == 0) return hipSuccess;
    if (!launch_fits((total + 255) / 256, 256)) return hipErrorInvalidConfiguration;
    bitrev_kernel<<<grid_for(total, 256), 256, 0, stream>>>(src, dst, total, logn);
    mark(stream);
    return hipGetLastError();
}

hipError_t launch_stream_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
    const int64_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    const int64_t blocks = (n16 + 2047) / 2048;
    if (!launch_fits(blocks, 256)) return hipErrorInvalidConfiguration;
    stream_copy_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const nt_float4*)src, (nt_float4*)dst, n16);
    mark(stream);
    return hipGetLastError();
}

hipError_t launch_real_epilogue(int kind, const void* in, void* out, int64_t n, int64_t rows, float scale,
                                hipStream_t stream) {
    const int64_t np = n >> 1;
    const int64_t total = rows * (kind == 0 ? np + 1 : np);
    if (total == 0) return hipSuccess;
    if (!launch_fits((total + 255) / 256, 256)) return hipErrorInvalidConfiguration;
    const unsigned grid = grid_for(total, 256);
    const float inv_np = 1.0f / (float)np;
    if (kind == 0)
        r2c_stitch_free_kernel<<<grid, 256, 0, stream>>>((const float2*)in, (float2*)out, np, total, inv_np, scale);
    else if (kind == 1)
        c2r_pre_free_kernel<<<grid, 256, 0, stream>>>((const float2*)in, (float2*)out, np, total, inv_np);
    else
        c2r_unpack_kernel<<<grid, 256, 0, stream>>>((const float2*)in, (float2*)out, np, total, scale);
    mark(stream);
    return hipGetLastError();
}

hipError_t launch_twiddle_transpose(int dir, const float2* s, float2* g, int64_t rows, int64_t cols, int64_t batch,
                                    hipStream_t stream) {
    const int64_t n = rows * cols;
    const int tiles_r = (int)((rows + 31) / 32), tiles_c = (int)((cols + 31) / 32);
    const int64_t blocks = batch * tiles_r * tiles_c;
    if (blocks == 0) return hipSuccess;
    if (!launch_fits(blocks, 256)) return hipErrorInvalidConfiguration;
    const uint32_t nmask = (uint32_t)(n - 1);
    const float inv_half_n = 2.0f / (float)n;
    if (dir < 0)
        twiddle_transpose_kernel<-1><<<(unsigned)blocks, 256, 0, stream>>>(s, g, (int)rows, (int)cols, tiles_r,
                                                                          tiles_c, nmask, inv_half_n);
    else
        twiddle_transpose_kernel<1><<<(unsigned)blocks, 256, 0, stream>>>(s, g, (int)rows, (int)cols, tiles_r,
                                                                         tiles_c, nmask, inv_half_n);
    mark(stream);
    return hipGetLastError();
}

hipError_t launch_r2c_stitch(const float2* z, float2* x, const float2* tw_real, int64_t n,
                             int64_t rows, float scale, hipStream_t stream) {
    const int64_t np = n >> 1;
    const int64_t total = rows * ((np >> 1) + 1);  // pairs k in [0, np/2] of every row
    if (total <= 0) return hipSuccess;
    if (!launch_fits((total + 255) / 256, 256)) return hipErrorInvalidConfiguration;
    r2c_stitch_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(z, x, tw_real, np, (uint32_t)total,
                                                                           scale);
    mark(stream);
    return hipGetLastError();
}

hipError_t launch_c2r_pre(const float2* x, float2* z, const float2* tw_real, int64_t n,
                          int64_t rows, hipStream_t stream) {
    const int64_t np = n >> 1;
    const int64_t total = rows * ((np >> 1) + 1);
    if (total <= 0) return hipSuccess;
    if (!launch_fits((total + 255) / 256, 256)) return hipErrorInvalidConfiguration;
    c2r_pre_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(x, z, tw_real, np, (uint32_t)total);
    mark(stream);
    return hipGetLastError();
}

}  // namespace mfft
