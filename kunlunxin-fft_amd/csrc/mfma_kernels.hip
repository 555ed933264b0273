// mfma_kernels.hip -- dense-dot FFT core on the fp32 matrix cores, for core
// lengths 2..16384: the MI355X form of the reference's M2 flow
// ("matrix-resident" / "dense-dot-fft64": kernels.py:487-532 and 594-630,
// the DFT_T * P_bitrev block matrices of matrices.py:64-92), where the first
// log2(T) stages are a dense matrix product.
//
// Algorithm: Stockham auto-sort with radix-8 passes (the remainder radix, 2
// or 4, last), whole transform resident in LDS between passes, pass 0 read
// from HBM and the last pass written to HBM.  Every butterfly is a dense
// matrix product on the matrix cores: a complex DFT_8 is a real 16 x 16
// matrix acting on 8 interleaved complex values, and one chain of four
// v_mfma_f32_16x16x4_f32 (K = 4 each) applies it to 16 butterfly columns at
// once.  A radix-4 (radix-2) pass packs two (four) butterflies into one
// column with a block-diagonal matrix, so every pass costs the same four
// MFMAs per 128 points.  The first two passes are the 8 x 8 factored DFT_64
// (DFT_8, twiddle W_64, DFT_8); transforms of 64 points are exactly that.
// The pass twiddles W_{NS*R}^(q*(b mod NS)) are multiplied in on the vector
// ALU before each product, from one table of W_L^m (m < L).
//
// MFMA operand layout (v_mfma_f32_16x16x4_f32, one block; lane l = 16 g + j,
// j < 16, g < 4): A[i][k] is held by lane i + 16 k, B[k][j] by lane
// j + 16 k, and D[i][j] by lane j + 16 (i / 4), element i % 4.  The four
// MFMAs c = 0..3 of a chain cover the contraction index 4c + k; index
// (c, k) stands for component c & 1 of input point 2k + (c >> 1), and
// output row i for component i & 1 of output point i >> 1.  So lane (j, g)
// supplies points 2g and 2g+1 of column j as its four B values
// (re, im, re, im), and receives output points 2g and 2g+1 of the same
// column as its four D values: the distribution in and out is the same.
//
// Inverse = conjugated roots (matrix and twiddles); the norm scale is
// applied in the final store.
#include "mfft_device.hpp"
#include "mfft_internal.hpp"

namespace mfft {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int LOGL>
struct MfmaCfg {
    static constexpr int L = 1 << LOGL;
    static constexpr int P = sched_passes(LOGL, 3);  // radix-8 passes, remainder last
    static constexpr int PTS = L > 4096 ? L : 4096;  // points per block
    static constexpr int W = L > 4096 ? L / 1024 : 4;  // waves per block
    static constexpr int WG = 64 * W;
    static constexpr int TPB = PTS / L;              // transforms per block
    static constexpr int G = PTS / (128 * W);        // 16-column groups per wave and pass (8)
    static constexpr int LDS = PTS + (PTS >> 4);     // float2, one pad slot per 16
    static constexpr int logr(int p) { return sched_logr(LOGL, 3, p); }
    static_assert(G * 128 * W == PTS, "groups must tile the block");
};

__device__ __forceinline__ int pad(int i) { return i + (i >> 4); }

// cos and sin of 2*pi*e/8
__device__ __forceinline__ float cos8(int e) {
    constexpr float h = 0.70710678118654752440f;
    switch (e & 7) {
        case 0: return 1.0f;
        case 1: case 7: return h;
        case 2: case 6: return 0.0f;
        case 3: case 5: return -h;
        default: return -1.0f;
    }
}
__device__ __forceinline__ float sin8(int e) { return cos8(e - 2); }

// This lane's A operands of the four MFMAs for a radix-R pass: entries of
// the real 16 x 16 form of the block-diagonal complex matrix that maps the
// 8 points of a column (8/R butterflies of R points) to their DFT_R outputs,
// W = exp(DIR * 2 pi i qo qi / R).  A[i][k] of MFMA c sits in lane i + 16k:
// row i = (output point i >> 1, component i & 1), contraction index
// (c, k) = (input point 2k + (c >> 1), component c & 1).
template <int R, int DIR>
__device__ __forceinline__ void dft_operands(float (&a)[4], int lane) {
    const int i = lane & 15, k = lane >> 4;
    const int po = i >> 1, co = i & 1;
    static_for<0, 4>([&](auto cc) {
        constexpr int c = cc.value;
        const int pi = 2 * k + (c >> 1), ci = c & 1;
        float v = 0.0f;
        if (po / R == pi / R) {
            const int e = ((po % R) * (pi % R) * (8 / R)) & 7;
            const float wr = cos8(e), wi = DIR < 0 ? -sin8(e) : sin8(e);
            // y.re = wr x.re - wi x.im ; y.im = wi x.re + wr x.im
            v = co == 0 ? (ci == 0 ? wr : -wi) : (ci == 0 ? wi : wr);
        }
        a[c] = v;
    });
}

template <int LOGL, int DIR>
__global__ __launch_bounds__(MfmaCfg<LOGL>::WG) void mfma_fft_kernel(const float2* __restrict__ src,
                                                                     float2* __restrict__ dst,
                                                                     const float2* __restrict__ tw, int64_t rows,
                                                                     float scale) {
    using C = MfmaCfg<LOGL>;
    constexpr int L = C::L, P = C::P, G = C::G, W = C::W;
    __shared__ float2 lds[P > 1 ? C::LDS : 1];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int64_t row0 = (int64_t)blockIdx.x * C::TPB;

    f4 d[G];
    static_for<0, P>([&](auto pp) {
        constexpr int p = pp.value;
        constexpr int LR = C::logr(p);
        constexpr int R = 1 << LR;
        constexpr int LQ = LOGL - LR;  // log2 of the butterflies per transform
        constexpr int LNS = 3 * p;     // span of the passes before
        constexpr int NS = 1 << LNS;
        const int s = (2 * g) >> LR;   // the lane's butterfly within its column
        const int q0 = (2 * g) & (R - 1);  // the lane's first point (second: q0 + 1)
        float a[4];
        dft_operands<R, DIR>(a, lane);

        // operands: butterfly bb of the block is (transform t, butterfly b)
        static_for<0, G>([&](auto gg) {
            const int gi = wave + gg.value * W;
            const int bb = gi * (128 / R) + s * 16 + j;
            const int t = bb >> LQ;
            const int b = bb & ((1 << LQ) - 1);
            float2 x0, x1;
            if constexpr (p == 0) {
                const int64_t row = row0 + t;
                const float2* xr = src + row * L + b;
                const bool active = row < rows;
                x0 = active ? load_nt(xr + (q0 << LQ)) : make_float2(0.0f, 0.0f);
                x1 = active ? load_nt(xr + ((q0 + 1) << LQ)) : make_float2(0.0f, 0.0f);
            } else {
                const int base = t * L + b;
                x0 = lds[pad(base + (q0 << LQ))];
                x1 = lds[pad(base + ((q0 + 1) << LQ))];
            }
            if constexpr (NS > 1) {
                // W_{NS R}^(q (b mod NS)) = W_L^(q m), m = (b mod NS) L / (NS R)
                const int m = (b & (NS - 1)) << (LOGL - LNS - LR);
                x0 = cmul_tw<DIR>(x0, tw[q0 * m]);
                x1 = cmul_tw<DIR>(x1, tw[(q0 + 1) * m]);
            }
            d[gg.value] = f4{x0.x, x0.y, x1.x, x1.y};
        });
        static_for<0, G>([&](auto gg) {
            f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            static_for<0, 4>([&](auto c) {
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c.value], d[gg.value][c.value], acc, 0, 0, 0);
            });
            d[gg.value] = acc;
        });
        // every operand of this pass has been read from LDS before it is overwritten
        if constexpr (p > 0 && p < P - 1) __syncthreads();
        static_for<0, G>([&](auto gg) {
            const int gi = wave + gg.value * W;
            const int bb = gi * (128 / R) + s * 16 + j;
            const int t = bb >> LQ;
            const int b = bb & ((1 << LQ) - 1);
            // outputs q0 and q0 + 1 of butterfly b: (b / NS) NS R + b mod NS + k NS
            const int o = ((b >> LNS) << (LNS + LR)) + (b & (NS - 1)) + (q0 << LNS);
            const float2 y0 = make_float2(d[gg.value][0], d[gg.value][1]);
            const float2 y1 = make_float2(d[gg.value][2], d[gg.value][3]);
            if constexpr (p == P - 1) {
                const int64_t row = row0 + t;
                if (row < rows) {
                    float2* yr = dst + row * L + o;
                    yr[0] = cscale(y0, scale);
                    yr[NS] = cscale(y1, scale);
                }
            } else {
                lds[pad(t * L + o)] = y0;
                lds[pad(t * L + o + NS)] = y1;
            }
        });
        if constexpr (p < P - 1) __syncthreads();
    });
}

template <int LOGL, int DIR>
hipError_t launch_one(const float2* src, float2* dst, const float2* tw, int64_t rows, float scale,
                      hipStream_t stream) {
    using C = MfmaCfg<LOGL>;
    const int64_t blocks = (rows + C::TPB - 1) / C::TPB;
    if (blocks <= 0) return hipSuccess;
    if (!launch_fits(blocks, C::WG)) return hipErrorInvalidConfiguration;
    mfma_fft_kernel<LOGL, DIR><<<(unsigned)blocks, C::WG, 0, stream>>>(src, dst, tw, rows, scale);
    mark(stream);
    return hipGetLastError();
}

template <int LOGL>
hipError_t dispatch_dir(int dir, const float2* src, float2* dst, const float2* tw, int64_t rows, float scale,
                        hipStream_t stream) {
    return dir < 0 ? launch_one<LOGL, -1>(src, dst, tw, rows, scale, stream)
                   : launch_one<LOGL, 1>(src, dst, tw, rows, scale, stream);
}

}  // namespace

bool mfma_supported(int log2l) { return log2l >= 1 && log2l <= kMaxMfmaLog2; }

hipError_t launch_mfma(int dir, int log2l, const float2* src, float2* dst, const float2* tw, int64_t rows,
                       float scale, hipStream_t stream) {
    switch (log2l) {
        case 1: return dispatch_dir<1>(dir, src, dst, tw, rows, scale, stream);
        case 2: return dispatch_dir<2>(dir, src, dst, tw, rows, scale, stream);
        case 3: return dispatch_dir<3>(dir, src, dst, tw, rows, scale, stream);
        case 4: return dispatch_dir<4>(dir, src, dst, tw, rows, scale, stream);
        case 5: return dispatch_dir<5>(dir, src, dst, tw, rows, scale, stream);
        case 6: return dispatch_dir<6>(dir, src, dst, tw, rows, scale, stream);
        case 7: return dispatch_dir<7>(dir, src, dst, tw, rows, scale, stream);
        case 8: return dispatch_dir<8>(dir, src, dst, tw, rows, scale, stream);
        case 9: return dispatch_dir<9>(dir, src, dst, tw, rows, scale, stream);
        case 10: return dispatch_dir<10>(dir, src, dst, tw, rows, scale, stream);
        case 11: return dispatch_dir<11>(dir, src, dst, tw, rows, scale, stream);
        case 12: return dispatch_dir<12>(dir, src, dst, tw, rows, scale, stream);
        case 13: return dispatch_dir<13>(dir, src, dst, tw, rows, scale, stream);
        case 14: return dispatch_dir<14>(dir, src, dst, tw, rows, scale, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mfft
