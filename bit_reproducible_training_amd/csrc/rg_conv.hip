// Reproducible 2D convolution and its two gradients on the int8 MFMA contraction.
//
// Definition: repro_conv_cuda/repro_conv_math.cuh:1-18. With W = N*OH*OW windows and
// Kc = C*KH*KW positions per window:
//   forward      Y = im2col(x)[W][Kc] * weight[F][Kc]^T       scales per window, per filter
//   weight grad  dW = dY^T[F][W] * im2col(x)[W][Kc]           scales per filter, per position
//   input grad   dX[pixel] = sum over the (window, position) pairs that read the pixel of
//                T[w][k] = sum_f D[w][f] * Wq[f][k]            one scale per image of dY,
//                                                              one for all weights
// The first two are exactly the reproducible GEMM on the im2col matrix, so they run the GEMM
// pipeline on packed operands. The input gradient runs the same slicing and contraction with
// group scales (every window of an image shares the image's scale; all positions share the
// weights' scale) and keeps the exact int64 T; col2im_round then adds each pixel's terms in
// int64 (exact, order-free) and rounds once with E = e_image + e_weights - 14 (S - 1).
//
// The packing kernels move fp32 values only (HBM-bound): im2col with zero padding, and the
// [N][F][OH*OW] <-> [W][F] transposes of dY and Y.
#include "rg_internal.h"
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

struct Geom {
    int N, C, H, W, F, KH, KW, SY, SX, PY, PX;
    int OH, OW, P;      // output size, P = OH * OW windows per image
    int K;              // C * KH * KW positions per window
    long long windows;  // N * P
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
    return g;
}

size_t grid_for(size_t n) { return std::min<size_t>((n + THREADS - 1) / THREADS, 65536); }

// cols[w][k] = x at position k = (c, ky, kx) of window w = (n, oy, ox), zero in the padding.
__global__ void __launch_bounds__(THREADS)
im2col_kernel(const float* __restrict__ x, float* __restrict__ cols, Geom g) {
    const size_t total = (size_t)g.windows * g.K;
    for (size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x; i < total;
         i += (size_t)gridDim.x * THREADS) {
        const long long w = (long long)(i / g.K);
        const int k = (int)(i - (size_t)w * g.K);
        const int n = (int)(w / g.P), p = (int)(w - (long long)n * g.P);
        const int oy = p / g.OW, ox = p - oy * g.OW;
        const int c = k / (g.KH * g.KW), r = k - c * (g.KH * g.KW);
        const int ky = r / g.KW, kx = r - ky * g.KW;
        const int y = oy * g.SY - g.PY + ky, xx = ox * g.SX - g.PX + kx;
        float v = 0.0f;
        if (y >= 0 && y < g.H && xx >= 0 && xx < g.W)
            v = x[(((size_t)n * g.C + c) * g.H + y) * g.W + xx];
        cols[i] = v;
    }
}

// rows[w][f] = t[n][f][p] for w = n * P + p (dY to one row per window).
__global__ void __launch_bounds__(THREADS)
nfp_to_rows_kernel(const float* __restrict__ t, float* __restrict__ rows, Geom g) {
    const size_t total = (size_t)g.windows * g.F;
    for (size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x; i < total;
         i += (size_t)gridDim.x * THREADS) {
        const long long w = (long long)(i / g.F);
        const int f = (int)(i - (size_t)w * g.F);
        const int n = (int)(w / g.P), p = (int)(w - (long long)n * g.P);
        rows[i] = t[((size_t)n * g.F + f) * g.P + p];
    }
}

// t[n][f][p] = rows[n * P + p][f] (GEMM output to NCHW).
__global__ void __launch_bounds__(THREADS)
rows_to_nfp_kernel(const float* __restrict__ rows, float* __restrict__ t, Geom g) {
    const size_t total = (size_t)g.windows * g.F;
    const size_t per_image = (size_t)g.F * g.P;
    for (size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x; i < total;
         i += (size_t)gridDim.x * THREADS) {
        const int n = (int)(i / per_image);
        const size_t r = i - (size_t)n * per_image;
        const int f = (int)(r / g.P), p = (int)(r - (size_t)f * g.P);
        t[i] = rows[((size_t)n * g.P + p) * g.F + f];
    }
}

// dX[n][c][y][x]: the exact int64 sum of T[w][k] (summed over the split parts) over every
// window w that reads pixel (y, x) at position k = (c, ky, kx), rounded once.
__global__ void __launch_bounds__(THREADS)
col2im_round_kernel(const int64_t* __restrict__ part, int split, const int* __restrict__ ea,
                    const int* __restrict__ eb, float* __restrict__ dx, Geom g, int e0) {
    const size_t total = (size_t)g.N * g.C * g.H * g.W;
    const size_t MN = (size_t)g.windows * g.K;
    const int eW = eb[0];
    for (size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x; i < total;
         i += (size_t)gridDim.x * THREADS) {
        const int xx = (int)(i % g.W);
        const int y = (int)((i / g.W) % g.H);
        const int c = (int)((i / ((size_t)g.W * g.H)) % g.C);
        const int n = (int)(i / ((size_t)g.W * g.H * g.C));
        int64_t t = 0;
        for (int ky = 0; ky < g.KH; ++ky) {
            const int ry = y + g.PY - ky;
            if (ry < 0 || ry % g.SY != 0) continue;
            const int oy = ry / g.SY;
            if (oy >= g.OH) continue;
            for (int kx = 0; kx < g.KW; ++kx) {
                const int rx = xx + g.PX - kx;
                if (rx < 0 || rx % g.SX != 0) continue;
                const int ox = rx / g.SX;
                if (ox >= g.OW) continue;
                const size_t w = (size_t)n * g.P + (size_t)oy * g.OW + ox;
                const size_t at = w * g.K + ((size_t)c * g.KH + ky) * g.KW + kx;
                for (int s = 0; s < split; ++s) t += part[(size_t)s * MN + at];
            }
        }
        dx[i] = repro_gemm::round_to_float_fast(t, ea[(size_t)n * g.P] + eW + e0);
    }
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

enum class Kind { Forward, GradWeight, GradInput };

// The convolution's GEMMs: its own int64 bound replaces the GEMM's; raw for the input gradient.
PlanExtras conv_extras(bool raw) {
    PlanExtras ex;
    ex.raw = raw;
    ex.gemm_bound = false;
    return ex;
}

struct ConvPlan {
    Geom g;
    Layout L;        // the GEMM
    size_t buf0, buf1, gemm, total;
};

int conv_plan(Kind kind, const rg_conv_shape* s, int S, ConvPlan* P) {
    if (!valid(s, S)) return hipErrorInvalidValue;
    ConvPlan p;
    std::memset(&p, 0, sizeof p);
    p.g = geom(*s);
    const Geom& g = p.g;
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
            b0 = (size_t)W * g.K * sizeof(float);   // cols
            b1 = (size_t)W * g.F * sizeof(float);   // Y rows
            break;
        case Kind::GradWeight:    // dW[F][K] = (dY rows[W][F])^T * cols[W][K]
            cfg.trans_a = 1;
            e = layout_for_current_device(g.F, g.K, W, &cfg, &p.L, conv_extras(false));
            b0 = (size_t)W * g.F * sizeof(float);   // dY rows
            b1 = (size_t)W * g.K * sizeof(float);   // cols
            break;
        case Kind::GradInput:     // T[W][K] = dY rows[W][F] * weight[F][K], exact int64
            e = layout_for_current_device(W, g.K, g.F, &cfg, &p.L, conv_extras(true));
            b0 = (size_t)W * g.F * sizeof(float);   // dY rows
            break;
    }
    if (e != hipSuccess) return e;
    p.buf0 = 0;
    p.buf1 = align_up(b0);
    p.gemm = p.buf1 + align_up(b1);
    p.total = p.gemm + p.L.total;
    *P = p;
    return hipSuccess;
}

int workspace_bytes_for(Kind kind, const rg_conv_shape* s, int S, size_t* bytes) {
    if (!bytes) return hipErrorInvalidValue;
    ConvPlan p;
    const int e = conv_plan(kind, s, S, &p);
    if (e != hipSuccess) return e;
    *bytes = p.total;
    return hipSuccess;
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
    return rg::workspace_bytes_for(rg::Kind::Forward, g, S, bytes);
}

int rg_conv2d_grad_weight_workspace(const rg_conv_shape* g, int S, size_t* bytes) {
    return rg::workspace_bytes_for(rg::Kind::GradWeight, g, S, bytes);
}

int rg_conv2d_grad_input_workspace(const rg_conv_shape* g, int S, size_t* bytes) {
    return rg::workspace_bytes_for(rg::Kind::GradInput, g, S, bytes);
}

int rg_conv2d_ws(const float* x, const float* weight, float* out, const rg_conv_shape* s, int S,
                 void* workspace, size_t workspace_bytes, void* stream_) {
    if (!x || !weight || !out) return hipErrorInvalidValue;
    rg::ConvPlan p;
    int e = rg::conv_plan(rg::Kind::Forward, s, S, &p);
    if (e != hipSuccess) return e;
    if (!workspace || workspace_bytes < p.total) return hipErrorInvalidValue;
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    char* base = static_cast<char*>(workspace);
    float* cols = reinterpret_cast<float*>(base + p.buf0);
    float* yrows = reinterpret_cast<float*>(base + p.buf1);
    const size_t packed = (size_t)p.g.windows * p.g.K, outn = (size_t)p.g.windows * p.g.F;
    hipLaunchKernelGGL(rg::im2col_kernel, dim3((unsigned)rg::grid_for(packed)), dim3(rg::THREADS),
                       0, stream, x, cols, p.g);
    e = rg::gemm_launch(cols, weight, yrows, p.L, base + p.gemm, stream, nullptr, rg::GemmOptions(),
                        rg::dense_addressing(p.L));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(rg::rows_to_nfp_kernel, dim3((unsigned)rg::grid_for(outn)),
                       dim3(rg::THREADS), 0, stream, yrows, out, p.g);
    return hipGetLastError();
}

int rg_conv2d_grad_weight_ws(const float* dy, const float* x, float* dw, const rg_conv_shape* s,
                             int S, void* workspace, size_t workspace_bytes, void* stream_) {
    if (!dy || !x || !dw) return hipErrorInvalidValue;
    rg::ConvPlan p;
    int e = rg::conv_plan(rg::Kind::GradWeight, s, S, &p);
    if (e != hipSuccess) return e;
    if (!workspace || workspace_bytes < p.total) return hipErrorInvalidValue;
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    char* base = static_cast<char*>(workspace);
    float* dyrows = reinterpret_cast<float*>(base + p.buf0);
    float* cols = reinterpret_cast<float*>(base + p.buf1);
    const size_t packed = (size_t)p.g.windows * p.g.K, outn = (size_t)p.g.windows * p.g.F;
    hipLaunchKernelGGL(rg::nfp_to_rows_kernel, dim3((unsigned)rg::grid_for(outn)),
                       dim3(rg::THREADS), 0, stream, dy, dyrows, p.g);
    hipLaunchKernelGGL(rg::im2col_kernel, dim3((unsigned)rg::grid_for(packed)), dim3(rg::THREADS),
                       0, stream, x, cols, p.g);
    e = rg::gemm_launch(dyrows, cols, dw, p.L, base + p.gemm, stream, nullptr, rg::GemmOptions(),
                        rg::dense_addressing(p.L));
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

int rg_conv2d_grad_input_ws(const float* dy, const float* weight, float* dx,
                            const rg_conv_shape* s, int S, void* workspace,
                            size_t workspace_bytes, void* stream_) {
    if (!dy || !weight || !dx) return hipErrorInvalidValue;
    rg::ConvPlan p;
    int e = rg::conv_plan(rg::Kind::GradInput, s, S, &p);
    if (e != hipSuccess) return e;
    if (!workspace || workspace_bytes < p.total) return hipErrorInvalidValue;
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    char* base = static_cast<char*>(workspace);
    float* dyrows = reinterpret_cast<float*>(base + p.buf0);
    char* gws = base + p.gemm;
    const size_t outn = (size_t)p.g.windows * p.g.F;
    hipLaunchKernelGGL(rg::nfp_to_rows_kernel, dim3((unsigned)rg::grid_for(outn)),
                       dim3(rg::THREADS), 0, stream, dy, dyrows, p.g);
    rg::GemmOptions opt;
    opt.group_a = p.g.P;   // one scale per image
    opt.group_b = p.g.K;   // one scale for all weights
    opt.raw = true;
    e = rg::gemm_launch(dyrows, weight, nullptr, p.L, gws, stream, nullptr, opt,
                        rg::dense_addressing(p.L));
    if (e != hipSuccess) return e;
    const size_t pixels = (size_t)p.g.N * p.g.C * p.g.H * p.g.W;
    hipLaunchKernelGGL(rg::col2im_round_kernel, dim3((unsigned)rg::grid_for(pixels)),
                       dim3(rg::THREADS), 0, stream,
                       reinterpret_cast<const int64_t*>(gws + p.L.part), p.L.split,
                       reinterpret_cast<const int*>(gws + p.L.ea),
                       reinterpret_cast<const int*>(gws + p.L.eb), dx, p.g, -14 * (S - 1));
    return hipGetLastError();
}

}  // extern "C"
