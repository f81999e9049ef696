// Reproducible 2D convolution and its two gradients on the int8 MFMA contraction.
//
// Definition: repro_conv_cuda/repro_conv_math.cuh:1-18. With W = N*OH*OW windows and
// Kc = C*KH*KW positions per window:
//   forward      Y = im2col(x)[W][Kc] * weight[F][Kc]^T       scales per window, per filter
//   weight grad  dW = dY^T[F][W] * im2col(x)[W][Kc]           scales per filter, per position
//   input grad   dX[pixel] = sum over the (window, position) pairs that read the pixel of
//                T[w][k] = sum_f D[w][f] * Wq[f][k]            one scale per image of dY,
//                                                              one for all weights
//                (computed as the GEMM of T^T = Wq^T D^T, stored [k][w])
// The first two are exactly the reproducible GEMM on the im2col matrix, so they run the GEMM
// pipeline on packed operands. The input gradient runs the same slicing and contraction with
// group scales (every window of an image shares the image's scale; all positions share the
// weights' scale) and keeps the exact int64 T; col2im_round then adds each pixel's terms in
// int64 (exact, order-free) and rounds once with E = e_image + e_weights - 14 (S - 1).
//
// The packing kernels move fp32 values only (HBM-bound): im2col with zero padding, and the
// [N][F][OH*OW] <-> [W][F] transposes of dY and Y.
#include "rg_internal.h"
#include "rg_fastdiv.h"
#include "repro_conv.h"
#include "repro_gemm_math.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>

namespace rg {
namespace {

constexpr int THREADS = 256;
constexpr size_t CONV_ALIGN = 256;
size_t align_up(size_t x) { return (x + CONV_ALIGN - 1) / CONV_ALIGN * CONV_ALIGN; }

// Shape and output geometry, with the divisors of the kernels' index arithmetic. Every tensor
// (input, weights, output, its W x F rows) holds fewer than 2^31 elements (checked by valid()),
// so their indices are 32-bit; the im2col matrix (W x K) may not, and is filled in window
// ranges of fewer than 2^31 elements.
struct Geom {
    int N, C, H, W, F, KH, KW, SY, SX, PY, PX;
    int OH, OW, P;      // output size, P = OH * OW windows per image
    int K;              // C * KH * KW positions per window
    long long windows;  // N * P
    FastDiv dK, dP, dOW, dKHW, dKW, dF, dFP, dW, dH, dC, dN, dSY, dSX;
};

Geom geom(const rg_conv_shape& s) {
    Geom g;
    g.N = s.N; g.C = s.C; g.H = s.H; g.W = s.W;
    g.F = s.F; g.KH = s.KH; g.KW = s.KW;
    g.SY = s.SY; g.SX = s.SX; g.PY = s.PY; g.PX = s.PX;
    g.OH = (s.H + 2 * s.PY - s.KH) / s.SY + 1;
    g.OW = (s.W + 2 * s.PX - s.KW) / s.SX + 1;
    g.P = g.OH * g.OW;
    g.K = s.C * s.KH * s.KW;
    g.windows = (long long)s.N * g.P;
    g.dK = make_fastdiv(g.K);
    g.dP = make_fastdiv(g.P);
    g.dOW = make_fastdiv(g.OW);
    g.dKHW = make_fastdiv(g.KH * g.KW);
    g.dKW = make_fastdiv(g.KW);
    g.dF = make_fastdiv(g.F);
    g.dFP = make_fastdiv((uint32_t)((long long)g.F * g.P));
    g.dW = make_fastdiv(g.W);
    g.dH = make_fastdiv(g.H);
    g.dN = make_fastdiv(g.N);
    g.dC = make_fastdiv(g.C);
    g.dSY = make_fastdiv(g.SY);
    g.dSX = make_fastdiv(g.SX);
    return g;
}

size_t grid_for(size_t n) { return std::min<size_t>((n + THREADS - 1) / THREADS, 65536); }

// cols[w][k] = x at position k = (c, ky, kx) of window w = (n, oy, ox), zero in the padding,
// for the windows w0 .. w0 + count - 1. A block moves a tile of 64 windows x 64 positions
// through LDS: it reads along the windows (consecutive windows of an output row are consecutive
// pixels of x, so the loads coalesce) and writes along the positions (256 contiguous bytes of a
// row of cols per wave). nanw / nank (either may be null, both zeroed before): a NaN read for
// window w at position k sets nanw[w] and nank[k] to 1, the rows whose maximum a NaN wins in the
// forward pass (windows) and the weight gradient (positions).
constexpr int IM2COL_TILE = 64;

__global__ void __launch_bounds__(THREADS)
im2col_kernel(const float* __restrict__ x, float* __restrict__ cols, Geom g, uint32_t w0,
              uint32_t count, unsigned* __restrict__ nanw, unsigned* __restrict__ nank) {
    __shared__ float tile[IM2COL_TILE][IM2COL_TILE + 1];
    __shared__ long long koff[IM2COL_TILE];           // (c*H + ky)*W + kx of each position
    __shared__ int kys[IM2COL_TILE], kxs[IM2COL_TILE];
    const int t = threadIdx.x;
    const uint32_t wt = blockIdx.y * IM2COL_TILE;     // first window of the tile, from w0
    const int kt = blockIdx.x * IM2COL_TILE;          // first position of the tile
    if (t < IM2COL_TILE) {
        const int k = min(kt + t, g.K - 1);
        const int c = (int)fdiv(k, g.dKHW), r = k - c * (g.KH * g.KW);
        const int ky = (int)fdiv(r, g.dKW), kx = r - ky * g.KW;
        koff[t] = ((long long)c * g.H + ky) * g.W + kx;
        kys[t] = ky;
        kxs[t] = kx;
    }
    __syncthreads();
    {
        const int wl = t % IM2COL_TILE;
        const uint32_t w = w0 + wt + wl;
        const bool live = wt + wl < count;
        const uint32_t n = fdiv(w, g.dP);
        const int p = (int)(w - n * (uint32_t)g.P);
        const int oy = (int)fdiv(p, g.dOW), ox = p - oy * g.OW;
        const int y0 = oy * g.SY - g.PY, x0 = ox * g.SX - g.PX;
        const long long base = (long long)n * g.C * g.H * g.W + (long long)y0 * g.W + x0;
        constexpr int STEP = THREADS / IM2COL_TILE;
#pragma unroll
        for (int j = 0; j < IM2COL_TILE / STEP; ++j) {
            const int kl = t / IM2COL_TILE + j * STEP;
            const int y = y0 + kys[kl], xx = x0 + kxs[kl];
            float v = 0.0f;
            if (live && kl < g.K - kt && (unsigned)y < (unsigned)g.H && (unsigned)xx < (unsigned)g.W)
                v = x[base + koff[kl]];
            if (__builtin_isnan(v)) {  // every writer stores the same 1
                if (nanw) nanw[w] = 1u;
                if (nank) nank[kt + kl] = 1u;
            }
            tile[wl][kl] = v;
        }
    }
    __syncthreads();
    if (g.K % 4 == 0 && g.K - kt >= IM2COL_TILE && (reinterpret_cast<uintptr_t>(cols) & 15) == 0) {
        // Rows stay 16-byte aligned: 16 lanes store one row's 64 positions as float4s.
        const int q = t % (IM2COL_TILE / 4);
        float* out = cols + ((size_t)w0 + wt) * g.K + kt + 4 * q;
        constexpr int STEP = THREADS / (IM2COL_TILE / 4);
#pragma unroll
        for (int j = 0; j < IM2COL_TILE / STEP; ++j) {
            const int wl = t / (IM2COL_TILE / 4) + j * STEP;
            if (wt + wl < count)
                *reinterpret_cast<float4*>(out + (size_t)wl * g.K) =
                    make_float4(tile[wl][4 * q], tile[wl][4 * q + 1], tile[wl][4 * q + 2],
                                tile[wl][4 * q + 3]);
        }
    } else {
        const int kl = t % IM2COL_TILE;
        if (kl < g.K - kt) {
            float* out = cols + ((size_t)w0 + wt) * g.K + kt + kl;
            constexpr int STEP = THREADS / IM2COL_TILE;
#pragma unroll
            for (int j = 0; j < IM2COL_TILE / STEP; ++j) {
                const int wl = t / IM2COL_TILE + j * STEP;
                if (wt + wl < count) out[(size_t)wl * g.K] = tile[wl][kl];
            }
        }
    }
}

// p[0 .. n) = 0 (the NaN flags, before im2col_kernel sets some).
__global__ void __launch_bounds__(THREADS) zero_flags_kernel(unsigned* __restrict__ p, long long n) {
    for (long long i = (long long)blockIdx.x * THREADS + threadIdx.x; i < n;
         i += (long long)gridDim.x * THREADS)
        p[i] = 0u;
}

// dst[b][c][r] = src[b][r][c] for `batch` matrices of rows x cols, through a 32 x 33 LDS tile
// so both the reads and the writes of a wavefront are consecutive. Grid: x over the 32 x 32
// tiles of one matrix, y over the matrices.
__global__ void __launch_bounds__(THREADS)
transpose_kernel(const float* __restrict__ src, float* __restrict__ dst, int rows, int cols,
                 int tiles_c) {
    __shared__ float tile[32][33];
    const int tr = blockIdx.x / tiles_c, tc = blockIdx.x - tr * tiles_c;
    const size_t off = (size_t)blockIdx.y * rows * cols;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = tr * 32 + ty + 8 * i, c = tc * 32 + tx;
        if (r < rows && c < cols) tile[ty + 8 * i][tx] = src[off + (size_t)r * cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tc * 32 + ty + 8 * i, r = tr * 32 + tx;
        if (r < rows && c < cols) dst[off + (size_t)c * rows + r] = tile[tx][ty + 8 * i];
    }
}

// rows[w][f] = t[n][f][p] for w = n * P + p (dY to one row per window).
__global__ void __launch_bounds__(THREADS)
nfp_to_rows_kernel(const float* __restrict__ t, float* __restrict__ rows, Geom g) {
    const uint32_t total = (uint32_t)(g.windows * g.F);
    for (uint32_t i = blockIdx.x * THREADS + threadIdx.x; i < total; i += gridDim.x * THREADS) {
        const uint32_t w = fdiv(i, g.dF);
        const uint32_t f = i - w * (uint32_t)g.F;
        const uint32_t n = fdiv(w, g.dP), p = w - n * (uint32_t)g.P;
        rows[i] = t[(n * (uint32_t)g.F + f) * (uint32_t)g.P + p];
    }
}

// t[n][f][p] = rows[n * P + p][f] (GEMM output to NCHW).
__global__ void __launch_bounds__(THREADS)
rows_to_nfp_kernel(const float* __restrict__ rows, float* __restrict__ t, Geom g) {
    const uint32_t total = (uint32_t)(g.windows * g.F);
    for (uint32_t i = blockIdx.x * THREADS + threadIdx.x; i < total; i += gridDim.x * THREADS) {
        const uint32_t n = fdiv(i, g.dFP);
        const uint32_t r = i - n * (uint32_t)(g.F * g.P);
        const uint32_t f = fdiv(r, g.dP), p = r - f * (uint32_t)g.P;
        t[i] = rows[(n * (uint32_t)g.P + p) * (uint32_t)g.F + f];
    }
}

// Output position o of the window that reads input coordinate v at kernel offset k along one
// axis (stride s, padding pad, n_out outputs), or -1 when no window does.
__device__ __forceinline__ int window_at(int v, int pad, int k, const FastDiv& ds, int s, int n_out) {
    const int r = v + pad - k;
    if (r < 0) return -1;
    const int o = (int)fdiv((uint32_t)r, ds);
    return (o * s == r && o < n_out) ? o : -1;
}

// dX[n][c][y][x]: the exact int64 sum of T[w][k] (summed over the split parts) over every
// window w that reads pixel (y, x) at position k = (c, ky, kx), rounded once. T is stored
// transposed, [k][w]: for one (ky, kx) the threads of a pixel row read consecutive windows.
// Pixels are taken channel by channel across the images, (c, n, y, x), so that the KH*KW rows
// of T^T of a channel are read from start to end.
// ea: the positions' exponents (all the weights' one), eb: the windows' (their image's).
// KHT x KWT: the filter size when known at compile time (0: g.KH x g.KW), so that the loads
// of every (ky, kx) are predicated and in flight together.
template <int KHT, int KWT>
__global__ void __launch_bounds__(THREADS)
col2im_round_kernel(const int64_t* __restrict__ part, int split, const int* __restrict__ ea,
                    const int* __restrict__ eb, float* __restrict__ dx, Geom g, int e0) {
    const int KH = KHT ? KHT : g.KH, KW = KWT ? KWT : g.KW;
    constexpr int UNROLL_Y = KHT > 0 ? KHT : 1, UNROLL_X = KWT > 0 ? KWT : 1;
    const uint32_t total = (uint32_t)((long long)g.N * g.C * g.H * g.W);
    const size_t MN = (size_t)g.windows * g.K;
    const int eW = ea[0];
    for (uint32_t i = blockIdx.x * THREADS + threadIdx.x; i < total; i += gridDim.x * THREADS) {
        const uint32_t q1 = fdiv(i, g.dW);
        const int xx = (int)(i - q1 * (uint32_t)g.W);
        const uint32_t q2 = fdiv(q1, g.dH);
        const int y = (int)(q1 - q2 * (uint32_t)g.H);
        const uint32_t c = fdiv(q2, g.dN);
        const uint32_t n = q2 - c * (uint32_t)g.N;
        const int64_t* pc = part + (size_t)c * KH * KW * g.windows + (size_t)n * g.P;
        const int e = eb[(size_t)n * g.P] + eW + e0;
        int64_t t = 0;
        for (int s = 0; s < split; ++s, pc += MN) {
            // Every position loads (a window that does not exist reads the start of its row of
            // T^T, in bounds, and adds zero), so the KH*KW loads are independent.
#pragma unroll UNROLL_Y
            for (int ky = 0; ky < KH; ++ky) {
                const int oy = window_at(y, g.PY, ky, g.dSY, g.SY, g.OH);
#pragma unroll UNROLL_X
                for (int kx = 0; kx < KW; ++kx) {
                    const int ox = window_at(xx, g.PX, kx, g.dSX, g.SX, g.OW);
                    const bool ok = oy >= 0 && ox >= 0;
                    const int64_t v = pc[(size_t)(ky * KW + kx) * g.windows + (ok ? oy * g.OW + ox : 0)];
                    t += ok ? v : 0;
                }
            }
        }
        dx[((size_t)n * g.C + c) * g.H * g.W + (size_t)y * g.W + xx] =
            repro_gemm::round_to_float_fast(t, e);
    }
}

// Direct kernels, for small filters: one launch each, every block computing the scales it
// needs itself, products summed in binary64. A fixed-point value has |X| <= 127 * 128^(S-1)
// < 2^21, so a product is an integer below 2^42 in magnitude and a sum of at most
// DIRECT_MAX_TERMS = 2^11 of them stays below 2^53: every partial sum is an exactly
// representable integer, so the binary64 accumulation is the exact integer sum in any order.
// Quantised values are kept in LDS as binary32 (integers below 2^22: exact).
constexpr int DIRECT_MAX_TERMS = 2048;
constexpr int FWD_DIRECT_MAX_WEIGHTS = 4096;  // K * (F padded to the pass width), binary64 in LDS
constexpr int DIRECT_PATCH_FLOATS = 6144;     // staged input (forward) or dY (input gradient)

// Forward tiling: filters are taken FC at a time (FC = F rounded up to a power of two, at most
// 8; F is padded with zero weights to a multiple of FC), G wavefront groups split those passes
// (strided by G), and the block's THREADS / G threads of a group take consecutive windows.
int fwd_pass_width(int F) { return F >= 8 ? 8 : (F > 4 ? 8 : (F > 2 ? 4 : F)); }
int fwd_padded_filters(int F) {
    const int fc = fwd_pass_width(F);
    return (F + fc - 1) / fc * fc;
}
int fwd_groups(int F) {
    const int passes = fwd_padded_filters(F) / fwd_pass_width(F);
    return passes >= 4 ? 4 : (passes >= 2 ? 2 : 1);
}

// Largest value of m over the block (every thread's m), in every thread; red: THREADS / 64
// floats of LDS.
__device__ __forceinline__ float block_max(float m, float* red) {
    m = wave_max(m);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by an earlier call
    if (lane == 0) red[wv] = m;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < THREADS / 64; ++i) m = fmaxf(m, red[i]);
    return m;
}

// max |p[i]| over this thread's share of [0, n) (i = first, first + step, ...), four loads in
// flight per round trip.
__device__ __forceinline__ float strided_absmax(const float* __restrict__ p, uint32_t n,
                                                uint32_t first, uint32_t step) {
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    uint32_t i = first;
    for (; i + 3 * step < n; i += 4 * step) {
        const float a = p[i], b = p[i + step], c = p[i + 2 * step], d = p[i + 3 * step];
        m0 = fmaxf(m0, fabsf(a));
        m1 = fmaxf(m1, fabsf(b));
        m2 = fmaxf(m2, fabsf(c));
        m3 = fmaxf(m3, fabsf(d));
    }
    for (; i < n; i += step) m0 = fmaxf(m0, fabsf(p[i]));
    return fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
}

// q = n / d and *r = n % d for 0 <= n < 2^20, 1 <= d < 2^20, inv = 1.0f / d: the binary32
// quotient is within 1/8 of n / d, so truncating it is off by at most one, which the
// remainder's sign and size correct.
__device__ __forceinline__ int small_divmod(int n, int d, float inv, int* r) {
    int q = (int)((float)n * inv);
    int rem = n - q * d;
    if (rem < 0) {
        --q;
        rem += d;
    } else if (rem >= d) {
        ++q;
        rem -= d;
    }
    *r = rem;
    return q;
}

// dst[i] = op(src[index(i)], i) for this thread's share of [0, n), four loads in flight; an
// index of -1 reads as 0.
template <class Index, class Op, class T>
__device__ __forceinline__ void gather4(T* __restrict__ dst, const float* __restrict__ src, int n,
                                        Index index, Op op) {
    for (int i0 = threadIdx.x; i0 < n; i0 += 4 * THREADS) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * THREADS;
            const long long at = i < n ? index(i) : -1;
            v[u] = at >= 0 ? src[at] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * THREADS;
            if (i < n) dst[i] = op(v[u], i);
        }
    }
}

// Forward (repro_conv_math.cuh:68-99). A block takes nw = THREADS / G consecutive windows of
// one image: it derives every filter's exponent and quantised weights (LDS, binary64, [k][f]
// with the filters padded to Fp), stages the input its windows read with the zero padding
// written out (LDS, [c][row][col], rows from oy_lo * SY - PY, columns from -PX), takes each
// window's maximum and exponent, and each thread accumulates its window's products for its
// group's filters, FC at a time; the FC weights of one k are one contiguous run read by every
// lane alike (LDS broadcast). Padding values are zeros: they change neither the maximum nor the
// sums, and leave the inner loops without bounds checks.
template <int FC>
__global__ void __launch_bounds__(THREADS)
fwd_direct_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ out,
                  Geom g, int S, FastDiv dtiles, int G, int Fp) {
    extern __shared__ double wq[];                               // [K][Fp]
    int* ef = reinterpret_cast<int*>(wq + g.K * Fp);             // [F]
    const int nw = THREADS / G;
    int* sew = ef + g.F;                                         // [nw] window exponents
    float* patch = reinterpret_cast<float*>(sew + nw);           // [C][rows][PW]
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const uint32_t n = fdiv(blockIdx.x, dtiles);
    const int w0 = (int)(blockIdx.x - n * dtiles.d) * nw;
    const int w1 = min(g.P, w0 + nw);
    const int oy_lo = (int)fdiv((uint32_t)w0, g.dOW);
    const int rows = ((int)fdiv((uint32_t)(w1 - 1), g.dOW) - oy_lo) * g.SY + g.KH;
    const int PW = (g.OW - 1) * g.SX + g.KW;
    const int yp0 = oy_lo * g.SY - g.PY;  // image row of patch row 0 (column 0 is x = -PX)
    for (int f = wv; f < g.F; f += THREADS / 64) {
        const float m = wave_max(strided_absmax(w + f * g.K, g.K, lane, 64));
        if (lane == 0) ef[f] = repro_gemm::scale_exponent(m);
    }
    const float* xn = x + (size_t)n * g.C * g.H * g.W;
    {
        const int plane = rows * PW;
        const float invp = 1.0f / (float)plane, invw = 1.0f / (float)PW;
        gather4(patch, xn, g.C * plane,
                [&](int i) -> long long {
                    int r, col;
                    const int c = small_divmod(i, plane, invp, &r);
                    const int row = small_divmod(r, PW, invw, &col);
                    const int y = yp0 + row, xx = col - g.PX;
                    if (y < 0 || y >= g.H || xx < 0 || xx >= g.W) return -1;
                    return ((long long)c * g.H + y) * g.W + xx;
                },
                [](float v, int) { return v; });
    }
    __syncthreads();
    {
        const float inv = 1.0f / (float)Fp;
        auto kf = [&](int i, int* f) { return small_divmod(i, Fp, inv, f); };
        gather4(wq, w, Fp * g.K,
                [&](int i) -> long long {
                    int f;
                    const int k = kf(i, &f);
                    return f < g.F ? (long long)f * g.K + k : -1;
                },
                [&](float v, int i) {
                    int f;
                    kf(i, &f);
                    return f < g.F ? (double)round_fixed(v, row_scale(S, ef[f])) : 0.0;
                });
    }
    if (t < w1 - w0) {
        const int p = w0 + t;
        const int oy = (int)fdiv((uint32_t)p, g.dOW), ox = p - oy * g.OW;
        const float* base = patch + (oy - oy_lo) * g.SY * PW + ox * g.SX;
        // Magnitude bits: a NaN in the window wins, and the window takes exponent 0.
        unsigned mb = 0;
        for (int c = 0; c < g.C; ++c)
            for (int ky = 0; ky < g.KH; ++ky) {
                const float* row = base + (c * rows + ky) * PW;
                for (int kx = 0; kx < g.KW; ++kx) mb = max(mb, __float_as_uint(row[kx]) & 0x7FFFFFFFu);
            }
        sew[t] = repro_gemm::scale_exponent(__uint_as_float(mb));
    }
    __syncthreads();
    const int wi = t % nw, gi = t / nw;
    const int p = w0 + wi;
    if (p >= w1) return;
    const int oy = (int)fdiv((uint32_t)p, g.dOW), ox = p - oy * g.OW;
    const float* base = patch + (oy - oy_lo) * g.SY * PW + ox * g.SX;
    const int se = sew[wi];
    const RowScale rs = row_scale(S, se);
    const int e0 = se - 14 * (S - 1);
    for (int f0 = gi * FC; f0 < g.F; f0 += G * FC) {
        double acc[FC];
#pragma unroll
        for (int j = 0; j < FC; ++j) acc[j] = 0.0;
        for (int c = 0; c < g.C; ++c)
            for (int ky = 0; ky < g.KH; ++ky) {
                const float* row = base + (c * rows + ky) * PW;
                const double* q = wq + ((c * g.KH + ky) * g.KW) * Fp + f0;
#pragma unroll 4
                for (int kx = 0; kx < g.KW; ++kx) {
                    const double X = (double)round_fixed(row[kx], rs);
                    const double* qk = q + kx * Fp;
#pragma unroll
                    for (int j = 0; j < FC; ++j) acc[j] = fma(X, qk[j], acc[j]);
                }
            }
        const int nf = min(FC, g.F - f0);
#pragma unroll
        for (int j = 0; j < FC; ++j)
            if (j < nf)
                out[((size_t)n * g.F + f0 + j) * g.P + p] =
                    repro_gemm::round_to_float_f64((int64_t)acc[j], e0 + ef[f0 + j]);
    }
}

// Output rows [oy_lo, oy_lo + noy) whose windows read some pixel row in [y0, y1].
__device__ __forceinline__ void dx_window_rows(const Geom& g, int y0, int y1, int* oy_lo, int* noy) {
    const int num = y0 + g.PY - g.KH + 1;
    const int lo = num <= 0 ? 0 : (int)fdiv((uint32_t)(num + g.SY - 1), g.dSY);
    const int top = y1 + g.PY;
    const int hi = min(g.OH - 1, (int)fdiv((uint32_t)top, g.dSY));
    *oy_lo = lo;
    *noy = max(0, hi - lo + 1);
}

// Input gradient (repro_conv_math.cuh:132-157). A block takes THREADS consecutive pixels of one
// (image, channel) plane: it derives the image's exponent of dY and the weights' common
// exponent, quantises the channel's weights (LDS, [ky][kx][f]) and the dY rows its pixels read
// (LDS, [f][oy][ox], one scale for the image), and each thread sums, over the windows that read
// its pixel and all filters, the products, four filters at a time into four accumulators.
// Lanes of a wavefront share the channel and walk (ky, kx, f) together, so their weight reads
// are LDS broadcasts. UNIT (stride 1): the staged dY carries zeros for the windows outside the
// output (oy from y0 + PY - KH + 1, ox from PX - KW + 1, XW = W + KW - 1 columns), so every
// (ky, kx) is read without checks; otherwise only real rows are staged and each (ky, kx) is
// tested for a window.
template <bool UNIT>
__global__ void __launch_bounds__(THREADS)
dx_direct_kernel(const float* __restrict__ dy, const float* __restrict__ w, float* __restrict__ dx,
                 Geom g, int S, FastDiv dtiles) {
    extern __shared__ float lds[];
    const int khw = g.KH * g.KW;
    float* wq = lds;                 // [KH][KW][F] of the block's channel
    float* xq = lds + g.F * khw;     // [F][noy][XW]
    __shared__ float red[THREADS / 64];
    const int t = threadIdx.x;
    const uint32_t plane = fdiv(blockIdx.x, dtiles);  // n * C + c
    const int p0 = (int)(blockIdx.x - plane * dtiles.d) * THREADS;
    const int p1 = min(g.H * g.W, p0 + THREADS);
    const uint32_t n = fdiv(plane, g.dC);
    const int c = (int)(plane - n * (uint32_t)g.C);
    const uint32_t per = (uint32_t)g.F * (uint32_t)g.P;
    const float* dyn = dy + (size_t)n * per;
    const uint32_t wn = (uint32_t)g.F * (uint32_t)g.C * khw;
    const float mi = block_max(strided_absmax(dyn, per, t, THREADS), red);
    const float mw = block_max(strided_absmax(w, wn, t, THREADS), red);
    const int se_i = repro_gemm::scale_exponent(mi), se_w = repro_gemm::scale_exponent(mw);
    const RowScale rsi = row_scale(S, se_i), rsw = row_scale(S, se_w);
    const int y0 = (int)fdiv((uint32_t)p0, g.dW), y1 = (int)fdiv((uint32_t)(p1 - 1), g.dW);
    int oy_lo, noy, ox_lo, XW;
    if (UNIT) {
        oy_lo = y0 + g.PY - g.KH + 1;
        noy = y1 - y0 + g.KH;
        ox_lo = g.PX - g.KW + 1;
        XW = g.W + g.KW - 1;
    } else {
        dx_window_rows(g, y0, y1, &oy_lo, &noy);
        ox_lo = 0;
        XW = g.OW;
    }
    {   // wq[r][f] = weight (f, c, r): destination index i = r * F + f
        const float inv = 1.0f / (float)g.F;
        gather4(wq, w + (size_t)c * khw, g.F * khw,
                [&](int i) -> long long {
                    int f;
                    const int r = small_divmod(i, g.F, inv, &f);
                    return (long long)f * g.C * khw + r;
                },
                [&](float v, int) { return (float)round_fixed(v, rsw); });
    }
    const int frows = noy * XW;
    if (frows > 0) {
        const float invf = 1.0f / (float)frows, invx = 1.0f / (float)XW;
        gather4(xq, dyn, g.F * frows,
                [&](int i) -> long long {
                    int r, col;
                    const int f = small_divmod(i, frows, invf, &r);
                    const int row = small_divmod(r, XW, invx, &col);
                    const int oy = oy_lo + row, ox = ox_lo + col;
                    if (oy < 0 || oy >= g.OH || ox < 0 || ox >= g.OW) return -1;
                    return (long long)f * g.P + oy * g.OW + ox;
                },
                [&](float v, int) { return (float)round_fixed(v, rsi); });
    }
    __syncthreads();
    const int pix = p0 + t;
    if (pix >= p1) return;
    const int y = (int)fdiv((uint32_t)pix, g.dW), xx = pix - y * g.W;
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    auto window = [&](const float* d, const float* q) {
        int f = 0;
        for (; f + 4 <= g.F; f += 4) {
            a0 = fma((double)d[f * frows], (double)q[f], a0);
            a1 = fma((double)d[(f + 1) * frows], (double)q[f + 1], a1);
            a2 = fma((double)d[(f + 2) * frows], (double)q[f + 2], a2);
            a3 = fma((double)d[(f + 3) * frows], (double)q[f + 3], a3);
        }
        for (; f < g.F; ++f) a0 = fma((double)d[f * frows], (double)q[f], a0);
    };
    if (UNIT) {
        // Window (oy, ox) = (y + PY - ky, x + PX - kx) sits at staged row y - y0 + KH - 1 - ky,
        // column x + KW - 1 - kx.
        const float* base = xq + (y - y0 + g.KH - 1) * XW + xx + g.KW - 1;
        for (int ky = 0; ky < g.KH; ++ky)
            for (int kx = 0; kx < g.KW; ++kx)
                window(base - ky * XW - kx, wq + (ky * g.KW + kx) * g.F);
    } else {
        for (int ky = 0; ky < g.KH; ++ky) {
            const int oy = window_at(y, g.PY, ky, g.dSY, g.SY, g.OH);
            if (oy < 0) continue;
            for (int kx = 0; kx < g.KW; ++kx) {
                const int ox = window_at(xx, g.PX, kx, g.dSX, g.SX, g.OW);
                if (ox < 0) continue;
                window(xq + (oy - oy_lo) * XW + ox, wq + (ky * g.KW + kx) * g.F);
            }
        }
    }
    // Partial sums are integers below 2^53 in magnitude (their terms' magnitudes sum to less),
    // so adding them is exact too.
    const double acc = (a0 + a1) + (a2 + a3);
    dx[(size_t)plane * g.H * g.W + pix] =
        repro_gemm::round_to_float_f64((int64_t)acc, se_i + se_w - 14 * (S - 1));
}

// repro_conv_math.cuh:159-163: terms per exact sum with |X| <= 127 * 128^(S-1).
double max_terms(int S) {
    const double lim = 127.0 * std::ldexp(1.0, 7 * (S - 1));
    return 9.0e18 / (lim * lim);
}

// Shape checks of repro_conv.cu:138-149 without the reference kernels' own size limits.
bool valid(const rg_conv_shape* s, int S) {
    if (!s || S < 1 || S > 3) return false;
    if (s->N <= 0 || s->C <= 0 || s->H <= 0 || s->W <= 0 || s->F <= 0 || s->KH <= 0 || s->KW <= 0)
        return false;
    if (s->SY <= 0 || s->SX <= 0 || s->PY < 0 || s->PX < 0) return false;
    if ((long long)s->H + 2LL * s->PY < s->KH || (long long)s->W + 2LL * s->PX < s->KW) return false;
    const long long oh = ((long long)s->H + 2LL * s->PY - s->KH) / s->SY + 1;
    const long long ow = ((long long)s->W + 2LL * s->PX - s->KW) / s->SX + 1;
    if ((double)s->N * oh * ow * s->F >= 2147483648.0) return false;  // before int geometry
    const Geom g = geom(*s);
    const double in = (double)s->N * s->C * s->H * s->W;
    const double out = (double)g.windows * s->F;
    const double wsz = (double)s->F * s->C * s->KH * s->KW;
    if (in >= 2147483648.0 || out >= 2147483648.0 || wsz >= 2147483648.0) return false;
    if ((double)s->C * s->KH * s->KW >= 2147483648.0) return false;
    if ((double)g.windows * g.K >= 9.2e18) return false;
    const double mt = max_terms(S);
    return (double)g.windows <= mt && (double)s->KH * s->KW * s->F <= mt && (double)g.K <= mt;
}

enum class Kind { Forward = RG_CONV_FORWARD, GradWeight = RG_CONV_GRAD_WEIGHT,
                  GradInput = RG_CONV_GRAD_INPUT };

// The convolution's GEMMs: its own int64 bound replaces the GEMM's; raw for the input gradient.
PlanExtras conv_extras(bool raw) {
    PlanExtras ex;
    ex.raw = raw;
    ex.gemm_bound = false;
    ex.one_launch = false;  // the pipeline's options (gathering, group scales) are needed
    return ex;
}

// Direct kernels' shape limits (exactness of the binary64 sums, LDS for the weights) and the
// automatic choice: direct while the multiply-adds and the blocks' redundant reads of weights
// and maxima stay small (at most about 20 us of work on MI355X), where the GEMM pipeline's
// launches, padding of K to 64 and packed copies cost more than the arithmetic, and while one
// thread's chain of multiply-adds stays short: the direct kernels' time grows with it (MI355X,
// LeNet-5 at batch 100: forward 11 us at 200 per thread against 33 us for the GEMM pipeline,
// 28 us at 1200 against 23 us; input gradient 15 us at 150 and 26 us at 400 against 53 and
// 41 us).
constexpr double DIRECT_AUTO_MACS = 268435456.0;  // 2^28
constexpr double DIRECT_AUTO_READS = 67108864.0;  // 2^26
constexpr long long FWD_AUTO_CHAIN = 512;         // K * (padded F) / G multiply-adds per thread
constexpr long long DX_AUTO_CHAIN = 768;          // F * KH * KW

// Direct tilings (see the kernels): forward blocks of THREADS / G windows of one image, input
// gradient blocks of THREADS pixels of one plane; the LDS each needs for its staged rows is
// bounded from the largest row span of a block.
long long fwd_tiles_per_image(const Geom& g) {
    const int nw = THREADS / fwd_groups(g.F);
    return (g.P + nw - 1) / nw;
}
long long fwd_patch_floats(const Geom& g) {
    const int nw = THREADS / fwd_groups(g.F);
    const long long oy_rows = std::min<long long>(g.OH, (nw - 1) / g.OW + 2);
    const long long rows = (oy_rows - 1) * g.SY + g.KH;
    const long long pw = (long long)(g.OW - 1) * g.SX + g.KW;
    return (long long)g.C * rows * pw;
}
size_t fwd_lds_bytes(const Geom& g) {
    return (size_t)g.K * fwd_padded_filters(g.F) * sizeof(double) +
           ((size_t)g.F + THREADS / fwd_groups(g.F) + fwd_patch_floats(g)) * 4;
}
long long dx_tiles_per_plane(const Geom& g) { return ((long long)g.H * g.W + THREADS - 1) / THREADS; }
bool dx_unit_stride(const Geom& g) { return g.SY == 1 && g.SX == 1; }
long long dx_patch_floats(const Geom& g) {
    const long long rows_px = std::min<long long>(g.H, (THREADS - 1) / g.W + 2);
    if (dx_unit_stride(g))
        return (long long)g.F * (rows_px + g.KH - 1) * (g.W + g.KW - 1);
    const long long noy = std::min<long long>(g.OH, (rows_px - 1 + g.KH - 1) / g.SY + 1);
    return (long long)g.F * noy * g.OW;
}
size_t dx_lds_bytes(const Geom& g) {
    return ((size_t)g.F * g.KH * g.KW + dx_patch_floats(g)) * 4;
}

bool direct_possible(Kind kind, const Geom& g) {
    if (kind == Kind::Forward)
        return g.K <= DIRECT_MAX_TERMS &&
               (long long)fwd_padded_filters(g.F) * g.K <= FWD_DIRECT_MAX_WEIGHTS &&
               fwd_patch_floats(g) <= DIRECT_PATCH_FLOATS &&
               (long long)g.N * fwd_tiles_per_image(g) <= INT_MAX;
    if (kind == Kind::GradInput)
        return (long long)g.F * g.KH * g.KW <= DIRECT_MAX_TERMS &&
               dx_patch_floats(g) <= DIRECT_PATCH_FLOATS &&
               (long long)g.N * g.C * dx_tiles_per_plane(g) <= INT_MAX;
    return false;
}

bool direct_preferred(Kind kind, const Geom& g) {
    if (!direct_possible(kind, g)) return false;
    double macs, reads;
    if (kind == Kind::Forward) {
        if ((long long)g.K * fwd_padded_filters(g.F) / fwd_groups(g.F) > FWD_AUTO_CHAIN) return false;
        const double blocks = (double)g.N * fwd_tiles_per_image(g);
        macs = (double)g.windows * g.F * g.K;
        reads = blocks * ((double)g.F * g.K + (double)fwd_patch_floats(g));
    } else {
        if ((long long)g.F * g.KH * g.KW > DX_AUTO_CHAIN) return false;
        const double blocks = (double)g.N * g.C * dx_tiles_per_plane(g);
        macs = (double)g.N * g.C * g.H * g.W * g.F * g.KH * g.KW;
        reads = blocks * ((double)g.F * g.P + (double)g.F * g.C * g.KH * g.KW);
    }
    return macs <= DIRECT_AUTO_MACS && reads <= DIRECT_AUTO_READS;
}

struct ConvPlan {
    Geom g;
    bool direct;
    bool implicit;   // forward GEMM reads the im2col matrix through Im2col (no cols buffer)
    Layout L;        // the GEMM (GEMM algorithm only)
    size_t buf0, buf1, gemm, total;
    size_t flags;    // NaN flags of the packed cols' windows (forward) or positions (weight
    long long nflags;  // gradient), one per padded row of that GEMM operand; 0 if none
};

int conv_plan(Kind kind, const rg_conv_shape* s, int S, int algo, ConvPlan* P) {
    if (!valid(s, S)) return hipErrorInvalidValue;
    if (algo != RG_CONV_ALGO_AUTO && algo != RG_CONV_ALGO_GEMM && algo != RG_CONV_ALGO_DIRECT)
        return hipErrorInvalidValue;
    ConvPlan p;
    std::memset(&p, 0, sizeof p);
    p.g = geom(*s);
    const Geom& g = p.g;
    p.direct = algo == RG_CONV_ALGO_DIRECT ||
               (algo == RG_CONV_ALGO_AUTO && direct_preferred(kind, g));
    if (p.direct) {
        if (!direct_possible(kind, g)) return hipErrorNotSupported;
        DeviceInfo dev;
        const int e = query_device(&dev);
        if (e != hipSuccess) return e;
        if (!dev.gfx950) return hipErrorNotSupported;
        p.total = CONV_ALIGN;  // no scratch; kept non-zero so that every pass takes a buffer
        *P = p;
        return hipSuccess;
    }
    rg_config cfg;
    rg_config_init(&cfg);
    cfg.slices = S;
    const int W = (int)g.windows;
    int e = hipSuccess;
    size_t b0 = 0, b1 = 0;
    switch (kind) {
        case Kind::Forward:       // C[W][F] = cols[W][K] * weight[F][K]^T
            cfg.trans_b = 1;
            e = layout_for_current_device(W, g.F, g.K, &cfg, &p.L, conv_extras(false));
            // The one-pass slicing gathers cols from x itself (implicit im2col); longer
            // windows take the two passes over a packed cols matrix.
            p.implicit = e == hipSuccess && p.L.Kp <= ONEPASS_MAX_K;
            b0 = p.implicit ? 0 : (size_t)W * g.K * sizeof(float);   // cols
            b1 = (size_t)W * g.F * sizeof(float);                     // Y rows
            if (e == hipSuccess && !p.implicit) p.nflags = p.L.Mp;    // windows
            break;
        case Kind::GradWeight:    // dW[F][K] = (dY rows[W][F])^T * cols[W][K]
            cfg.trans_a = 1;
            e = layout_for_current_device(g.F, g.K, W, &cfg, &p.L, conv_extras(false));
            b0 = (size_t)W * g.F * sizeof(float);   // dY rows
            b1 = (size_t)W * g.K * sizeof(float);   // cols
            if (e == hipSuccess) p.nflags = p.L.Np;  // positions
            break;
        case Kind::GradInput:     // T^T[K][W] = weight^T[K][F] * (dY rows[W][F])^T, exact int64
            // Transposed, so that the pixels of one row read neighbouring windows of one
            // position k in col2im_round (consecutive addresses).
            cfg.trans_a = 1;
            cfg.trans_b = 1;
            e = layout_for_current_device(g.K, W, g.F, &cfg, &p.L, conv_extras(true));
            b0 = (size_t)W * g.F * sizeof(float);   // dY rows
            break;
    }
    if (e != hipSuccess) return e;
    p.buf0 = 0;
    p.buf1 = align_up(b0);
    p.flags = p.buf1 + align_up(b1);
    p.gemm = p.flags + align_up((size_t)p.nflags * sizeof(unsigned));
    p.total = p.gemm + p.L.total;
    *P = p;
    return hipSuccess;
}

// Zeroes the plan's NaN flags (a kernel rather than a memset node, so that a captured graph
// replays it correctly).
unsigned* zero_flags(const ConvPlan& p, char* base, hipStream_t stream) {
    unsigned* f = reinterpret_cast<unsigned*>(base + p.flags);
    hipLaunchKernelGGL(zero_flags_kernel, dim3((unsigned)grid_for((size_t)p.nflags)), dim3(THREADS),
                       0, stream, f, (long long)p.nflags);
    return f;
}

// cols for every window. Consecutive blocks take the position tiles of one window tile (grid
// x), so a row of cols is completed, and its patch of x read, by neighbouring blocks; launches
// of at most 65535 window tiles (grid y).
void launch_im2col(const float* x, float* cols, const Geom& g, unsigned* nanw, unsigned* nank,
                   hipStream_t stream) {
    const long long per = 65535LL * IM2COL_TILE;
    const unsigned ktiles = (unsigned)((g.K + IM2COL_TILE - 1) / IM2COL_TILE);
    for (long long w0 = 0; w0 < g.windows; w0 += per) {
        const long long nw = std::min<long long>(per, g.windows - w0);
        const unsigned wtiles = (unsigned)((nw + IM2COL_TILE - 1) / IM2COL_TILE);
        hipLaunchKernelGGL(im2col_kernel, dim3(ktiles, wtiles), dim3(THREADS), 0, stream, x, cols,
                           g, (uint32_t)w0, (uint32_t)nw, nanw, nank);
    }
}

// [N][F][P] -> [N * P][F] (to_rows) or back, as N transposes of F x P matrices; the element-
// wise kernels when N exceeds the grid's y range.
void launch_nfp_rows(const float* src, float* dst, const Geom& g, bool to_rows, hipStream_t stream) {
    const int rows = to_rows ? g.F : g.P, cols = to_rows ? g.P : g.F;
    if (g.N <= 65535) {
        const int tiles_r = (rows + 31) / 32, tiles_c = (cols + 31) / 32;
        hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)(tiles_r * tiles_c), (unsigned)g.N),
                           dim3(THREADS), 0, stream, src, dst, rows, cols, tiles_c);
        return;
    }
    const size_t outn = (size_t)g.windows * g.F;
    if (to_rows)
        hipLaunchKernelGGL(nfp_to_rows_kernel, dim3((unsigned)grid_for(outn)), dim3(THREADS), 0,
                           stream, src, dst, g);
    else
        hipLaunchKernelGGL(rows_to_nfp_kernel, dim3((unsigned)grid_for(outn)), dim3(THREADS), 0,
                           stream, src, dst, g);
}

int run_pass(Kind kind, const float* a, const float* b, float* out, const rg_conv_shape* s, int S,
             int algo, void* workspace, size_t workspace_bytes, void* stream_) {
    if (!a || !b || !out) return hipErrorInvalidValue;
    ConvPlan p;
    int e = conv_plan(kind, s, S, algo, &p);
    if (e != hipSuccess) return e;
    if (!workspace || workspace_bytes < p.total) return hipErrorInvalidValue;
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    const Geom& g = p.g;
    if (p.direct) {
        if (kind == Kind::Forward) {
            const long long tiles = fwd_tiles_per_image(g);
            const dim3 grid((unsigned)(g.N * tiles));
            const FastDiv dt = make_fastdiv((uint32_t)tiles);
            const int G = fwd_groups(g.F), Fp = fwd_padded_filters(g.F);
            const size_t lds = fwd_lds_bytes(g);
            switch (fwd_pass_width(g.F)) {
                case 1: fwd_direct_kernel<1><<<grid, THREADS, lds, stream>>>(a, b, out, g, S, dt, G, Fp); break;
                case 2: fwd_direct_kernel<2><<<grid, THREADS, lds, stream>>>(a, b, out, g, S, dt, G, Fp); break;
                case 4: fwd_direct_kernel<4><<<grid, THREADS, lds, stream>>>(a, b, out, g, S, dt, G, Fp); break;
                default: fwd_direct_kernel<8><<<grid, THREADS, lds, stream>>>(a, b, out, g, S, dt, G, Fp); break;
            }
        } else {
            const long long tiles = dx_tiles_per_plane(g);
            const dim3 grid((unsigned)(g.N * g.C * tiles));
            const FastDiv dt = make_fastdiv((uint32_t)tiles);
            if (dx_unit_stride(g))
                dx_direct_kernel<true><<<grid, THREADS, dx_lds_bytes(g), stream>>>(a, b, out, g, S, dt);
            else
                dx_direct_kernel<false><<<grid, THREADS, dx_lds_bytes(g), stream>>>(a, b, out, g, S, dt);
        }
        return hipGetLastError();
    }
    char* base = static_cast<char*>(workspace);
    char* gws = base + p.gemm;
    switch (kind) {
        case Kind::Forward: {
            float* yrows = reinterpret_cast<float*>(base + p.buf1);
            if (p.implicit) {
                Im2col ic;
                ic.x = a;
                ic.C = g.C; ic.H = g.H; ic.W = g.W; ic.KH = g.KH; ic.KW = g.KW;
                ic.SY = g.SY; ic.SX = g.SX; ic.PY = g.PY; ic.PX = g.PX; ic.OW = g.OW; ic.P = g.P;
                ic.dP = g.dP; ic.dOW = g.dOW; ic.dKHW = g.dKHW; ic.dKW = g.dKW;
                GemmOptions opt;
                opt.im2col_a = &ic;
                e = gemm_launch(nullptr, b, yrows, p.L, gws, stream, nullptr, opt,
                                dense_addressing(p.L));
            } else {
                // Windows holding a NaN take exponent 0 (their maximum compares raw bits).
                float* cols = reinterpret_cast<float*>(base + p.buf0);
                GemmOptions opt;
                unsigned* nanw = zero_flags(p, base, stream);
                opt.nanrows_a = nanw;
                launch_im2col(a, cols, g, nanw, nullptr, stream);
                e = gemm_launch(cols, b, yrows, p.L, gws, stream, nullptr, opt,
                                dense_addressing(p.L));
            }
            if (e != hipSuccess) return e;
            launch_nfp_rows(yrows, out, g, false, stream);
            break;
        }
        case Kind::GradWeight: {
            float* dyrows = reinterpret_cast<float*>(base + p.buf0);
            float* cols = reinterpret_cast<float*>(base + p.buf1);
            launch_nfp_rows(a, dyrows, g, true, stream);
            // Positions holding a NaN in some window take exponent 0 (raw-bit maxima).
            GemmOptions opt;
            unsigned* nank = zero_flags(p, base, stream);
            opt.nanrows_b = nank;
            launch_im2col(b, cols, g, nullptr, nank, stream);
            e = gemm_launch(dyrows, cols, out, p.L, gws, stream, nullptr, opt,
                            dense_addressing(p.L));
            if (e != hipSuccess) return e;
            break;
        }
        case Kind::GradInput: {
            float* dyrows = reinterpret_cast<float*>(base + p.buf0);
            launch_nfp_rows(a, dyrows, g, true, stream);
            GemmOptions opt;
            opt.group_a = g.K;   // rows of op(A) are the positions: one scale for all weights
            opt.group_b = g.P;   // rows of op(B)^T are the windows: one scale per image
            opt.raw = true;
            e = gemm_launch(b, dyrows, nullptr, p.L, gws, stream, nullptr, opt,
                            dense_addressing(p.L));
            if (e != hipSuccess) return e;
            const size_t pixels = (size_t)g.N * g.C * g.H * g.W;
            const auto col2im = g.KH == 3 && g.KW == 3   ? col2im_round_kernel<3, 3>
                                : g.KH == 5 && g.KW == 5 ? col2im_round_kernel<5, 5>
                                : g.KH == 1 && g.KW == 1 ? col2im_round_kernel<1, 1>
                                                         : col2im_round_kernel<0, 0>;
            hipLaunchKernelGGL(col2im, dim3((unsigned)grid_for(pixels)), dim3(THREADS), 0, stream, reinterpret_cast<const int64_t*>(gws + p.L.part),
                               p.L.split, reinterpret_cast<const int*>(gws + p.L.ea),
                               reinterpret_cast<const int*>(gws + p.L.eb), out, g, -14 * (S - 1));
            break;
        }
    }
    return hipGetLastError();
}

int workspace_bytes_for(Kind kind, const rg_conv_shape* s, int S, int algo, size_t* bytes) {
    if (!bytes) return hipErrorInvalidValue;
    ConvPlan p;
    const int e = conv_plan(kind, s, S, algo, &p);
    if (e != hipSuccess) return e;
    *bytes = p.total;
    return hipSuccess;
}

bool valid_pass(int pass) {
    return pass == RG_CONV_FORWARD || pass == RG_CONV_GRAD_WEIGHT || pass == RG_CONV_GRAD_INPUT;
}

}  // namespace
}  // namespace rg

extern "C" {

void rg_conv_shape_init(rg_conv_shape* g) {
    if (!g) return;
    std::memset(g, 0, sizeof *g);
    g->SY = g->SX = 1;
}

int rg_conv2d_workspace(const rg_conv_shape* g, int S, size_t* bytes) {
    return rg::workspace_bytes_for(rg::Kind::Forward, g, S, RG_CONV_ALGO_AUTO, bytes);
}

int rg_conv2d_grad_weight_workspace(const rg_conv_shape* g, int S, size_t* bytes) {
    return rg::workspace_bytes_for(rg::Kind::GradWeight, g, S, RG_CONV_ALGO_AUTO, bytes);
}

int rg_conv2d_grad_input_workspace(const rg_conv_shape* g, int S, size_t* bytes) {
    return rg::workspace_bytes_for(rg::Kind::GradInput, g, S, RG_CONV_ALGO_AUTO, bytes);
}

int rg_conv2d_ws(const float* x, const float* weight, float* out, const rg_conv_shape* s, int S,
                 void* workspace, size_t workspace_bytes, void* stream) {
    return rg::run_pass(rg::Kind::Forward, x, weight, out, s, S, RG_CONV_ALGO_AUTO, workspace,
                        workspace_bytes, stream);
}

int rg_conv2d_grad_weight_ws(const float* dy, const float* x, float* dw, const rg_conv_shape* s,
                             int S, void* workspace, size_t workspace_bytes, void* stream) {
    return rg::run_pass(rg::Kind::GradWeight, dy, x, dw, s, S, RG_CONV_ALGO_AUTO, workspace,
                        workspace_bytes, stream);
}

int rg_conv2d_grad_input_ws(const float* dy, const float* weight, float* dx,
                            const rg_conv_shape* s, int S, void* workspace,
                            size_t workspace_bytes, void* stream) {
    return rg::run_pass(rg::Kind::GradInput, dy, weight, dx, s, S, RG_CONV_ALGO_AUTO, workspace,
                        workspace_bytes, stream);
}

int rg_conv2d_algo(int pass, const rg_conv_shape* g, int S, int* algo) {
    if (!algo || !rg::valid_pass(pass)) return hipErrorInvalidValue;
    rg::ConvPlan p;
    const int e = rg::conv_plan(static_cast<rg::Kind>(pass), g, S, RG_CONV_ALGO_AUTO, &p);
    if (e != hipSuccess) return e;
    *algo = p.direct ? RG_CONV_ALGO_DIRECT : RG_CONV_ALGO_GEMM;
    return hipSuccess;
}

int rg_conv2d_algo_workspace(int pass, const rg_conv_shape* g, int S, int algo, size_t* bytes) {
    if (!rg::valid_pass(pass)) return hipErrorInvalidValue;
    return rg::workspace_bytes_for(static_cast<rg::Kind>(pass), g, S, algo, bytes);
}

int rg_conv2d_algo_ws(int pass, const float* a, const float* b, float* out, const rg_conv_shape* g,
                      int S, int algo, void* workspace, size_t workspace_bytes, void* stream) {
    if (!rg::valid_pass(pass)) return hipErrorInvalidValue;
    return rg::run_pass(static_cast<rg::Kind>(pass), a, b, out, g, S, algo, workspace,
                        workspace_bytes, stream);
}

}  // extern "C"
