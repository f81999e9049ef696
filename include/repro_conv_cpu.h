#pragma once
// repro_conv_cpu.h -- the reproducible 2D convolution and its two gradients on the host CPU
// (header-only C++17; no GPU needed), bit-identical to rg_conv2d_ws,
// rg_conv2d_grad_weight_ws and rg_conv2d_grad_input_ws (include/repro_conv.h) for every input.
// Replaces repro_conv_cuda/repro_conv_cpu.h for the PyTorch binding's CPU branch
// (repro_torch/src/bindings.cpp:6,128,149,172): same namespace, names and arguments.
//
// The definition (repro_conv_cuda/repro_conv_math.cuh:1-18), with e0 = -14 (S - 1):
//   forward      Y[n,f,oy,ox] = round(sum_k X[w,k] Wf[f,k],  e_window(w) + e_filter(f) + e0)
//   weight grad  dW[f,k]      = round(sum_w D[w,f] X[w,k],   e_dY_filter(f) + e_position(k) + e0)
//   input grad   dX[n,c,y,x]  = round(sum D[n,f,oy,ox] Wq[f,c,ky,kx] over the windows (oy, ox)
//                               that cover the pixel and all filters,  e_image(n) + e_weights + e0)
// where X[w,k] is the window's value at position k (zero in the padding). Every scale is
// scale_exponent of the largest magnitude it covers, every value becomes fixed_point with its
// scale, every sum is exact in int64 and is rounded once. The forward pass and the weight
// gradient are therefore the reproducible GEMM on the im2col matrix; the input gradient's terms
// share one scale per image of dY and one for all weights.
//
// Each entry point throws std::invalid_argument for a null pointer or a shape the GPU entry
// points reject (cpu_shape_valid). Inputs are meant to be finite; a NaN or an infinity still
// gives the reference's CPU bits (see conv_detail::raw_magnitude_bits).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <vector>

#include "repro_conv_shape.h"
#include "repro_gemm_cpu.h"

namespace repro_conv {

// The GPU entry points' shape checks: positive sizes and strides, non-negative padding, a
// kernel no larger than the padded image, every tensor below 2^31 elements, and no exact sum
// with more terms than int64 holds at this S (9e18 / (127 * 128^(S-1))^2 terms).
inline bool cpu_shape_valid(const ConvShape& g, int S) {
    if (S < 1 || S > repro_gemm::MAX_SLICES) return false;
    if (g.N <= 0 || g.C <= 0 || g.H <= 0 || g.W <= 0 || g.F <= 0 || g.KH <= 0 || g.KW <= 0) return false;
    if (g.SY <= 0 || g.SX <= 0 || g.PY < 0 || g.PX < 0) return false;
    if ((long long)g.H + 2LL * g.PY < g.KH || (long long)g.W + 2LL * g.PX < g.KW) return false;
    const double oh = (double)(((long long)g.H + 2LL * g.PY - g.KH) / g.SY + 1);
    const double ow = (double)(((long long)g.W + 2LL * g.PX - g.KW) / g.SX + 1);
    const double limit = 2147483648.0;
    const double windows = (double)g.N * oh * ow, K = (double)g.C * g.KH * g.KW;
    if (windows * g.F >= limit || (double)g.N * g.C * g.H * g.W >= limit || K * g.F >= limit ||
        K >= limit)
        return false;
    const double top = 127.0 * std::ldexp(1.0, 7 * (S - 1));
    const double terms = 9.0e18 / (top * top);
    return windows <= terms && (double)g.KH * g.KW * g.F <= terms && K <= terms;
}

namespace conv_detail {

inline void require(bool ok, const char* what) {
    if (!ok) throw std::invalid_argument(what);
}

// The reference takes two kinds of maxima. The window maxima of the forward pass and the
// position maxima of the weight gradient compare the raw bits of |v|, so a NaN (bits above
// +inf) wins and its scale exponent is 0 (repro_conv_math.cuh:73-86, 121-130). The filter,
// dY and weight maxima use std::max on floats, which skips a NaN (repro_conv_cpu.h:29,48,77,82).
// For finite inputs both give the same maximum.
inline uint32_t raw_magnitude_bits(float v) { return repro_gemm::float_to_bits(v) & 0x7FFFFFFFu; }
inline uint32_t magnitude_bits(float v) { return repro_gemm::magnitude_key(v); }

// Values of window w (= (n, oy, ox)) at every position k, zero in the padding.
inline void gather_window(const float* x, const ConvShape& g, int w, float* vals) {
    const int P = g.OH() * g.OW(), n = w / P, p = w % P;
    const int y0 = (p / g.OW()) * g.SY - g.PY, x0 = (p % g.OW()) * g.SX - g.PX;
    int k = 0;
    for (int c = 0; c < g.C; ++c) {
        const float* plane = x + ((size_t)n * g.C + c) * g.H * g.W;
        for (int ky = 0; ky < g.KH; ++ky) {
            const int y = y0 + ky;
            for (int kx = 0; kx < g.KW; ++kx, ++k) {
                const int xx = x0 + kx;
                vals[k] = (y >= 0 && y < g.H && xx >= 0 && xx < g.W) ? plane[(size_t)y * g.W + xx] : 0.0f;
            }
        }
    }
}

}  // namespace conv_detail

inline void cpu_conv2d(const float* x, const float* w, float* out, const ConvShape& g, int S) {
    using namespace repro_gemm;
    conv_detail::require(x && w && out, "cpu_conv2d: null tensor");
    conv_detail::require(cpu_shape_valid(g, S), "cpu_conv2d: invalid shape");
    const int K = g.K(), P = g.OH() * g.OW(), e0 = -14 * (S - 1);
    std::vector<int32_t> Wq((size_t)g.F * K);
    std::vector<int> eF(g.F);
    repro_gemm::cpu_detail::fixed_point_rows(w, g.F, K, false, S, Wq.data(), eF.data());
    cpu_for(g.windows(), [&](int win) {
        std::vector<float> vals(K);
        std::vector<int32_t> q(K);
        conv_detail::gather_window(x, g, win, vals.data());
        uint32_t top = 0;
        for (int k = 0; k < K; ++k) top = std::max(top, conv_detail::raw_magnitude_bits(vals[k]));
        const int e = scale_exponent(bits_to_float(top));
        for (int k = 0; k < K; ++k) q[k] = fixed_point(vals[k], e, S);
        const int n = win / P, p = win % P;
        for (int f = 0; f < g.F; ++f) {
            const int32_t* wf = Wq.data() + (size_t)f * K;
            int64_t t = 0;
            for (int k = 0; k < K; ++k) t += (int64_t)q[k] * wf[k];
            out[((size_t)n * g.F + f) * P + p] = round_to_float(t, e + eF[f] + e0);
        }
    });
}

inline void cpu_conv2d_grad_weight(const float* dy, const float* x, float* dw, const ConvShape& g,
                                   int S) {
    using namespace repro_gemm;
    conv_detail::require(dy && x && dw, "cpu_conv2d_grad_weight: null tensor");
    conv_detail::require(cpu_shape_valid(g, S), "cpu_conv2d_grad_weight: invalid shape");
    const int K = g.K(), P = g.OH() * g.OW(), Wn = g.windows(), e0 = -14 * (S - 1);
    // dY per filter: D[f][w] with w = n * P + p, one scale per filter over all images.
    std::vector<int32_t> D((size_t)g.F * Wn);
    std::vector<int> eF(g.F);
    cpu_for(g.F, [&](int f) {
        uint32_t top = 0;
        for (int n = 0; n < g.N; ++n) {
            const float* run = dy + ((size_t)n * g.F + f) * P;
            for (int p = 0; p < P; ++p) top = std::max(top, conv_detail::magnitude_bits(run[p]));
        }
        const int e = eF[f] = scale_exponent(bits_to_float(top));
        int32_t* d = D.data() + (size_t)f * Wn;
        for (int n = 0; n < g.N; ++n) {
            const float* run = dy + ((size_t)n * g.F + f) * P;
            for (int p = 0; p < P; ++p) d[(size_t)n * P + p] = fixed_point(run[p], e, S);
        }
    });
    // One position k at a time: its im2col column over every window, scaled by its maximum.
    cpu_for(K, [&](int k) {
        const int c = k / (g.KH * g.KW), ky = (k / g.KW) % g.KH, kx = k % g.KW;
        std::vector<float> col(Wn);
        uint32_t top = 0;
        for (int win = 0; win < Wn; ++win) {
            const int n = win / P, p = win % P;
            const int y = (p / g.OW()) * g.SY - g.PY + ky, xx = (p % g.OW()) * g.SX - g.PX + kx;
            const float v = (y >= 0 && y < g.H && xx >= 0 && xx < g.W)
                                ? x[(((size_t)n * g.C + c) * g.H + y) * g.W + xx] : 0.0f;
            col[win] = v;
            top = std::max(top, conv_detail::raw_magnitude_bits(v));
        }
        const int e = scale_exponent(bits_to_float(top));
        std::vector<int32_t> q(Wn);
        for (int win = 0; win < Wn; ++win) q[win] = fixed_point(col[win], e, S);
        for (int f = 0; f < g.F; ++f) {
            const int32_t* d = D.data() + (size_t)f * Wn;
            int64_t t = 0;
            for (int win = 0; win < Wn; ++win) t += (int64_t)d[win] * q[win];
            dw[(size_t)f * K + k] = round_to_float(t, eF[f] + e + e0);
        }
    });
}

inline void cpu_conv2d_grad_input(const float* dy, const float* w, float* dx, const ConvShape& g,
                                  int S) {
    using namespace repro_gemm;
    conv_detail::require(dy && w && dx, "cpu_conv2d_grad_input: null tensor");
    conv_detail::require(cpu_shape_valid(g, S), "cpu_conv2d_grad_input: invalid shape");
    const int OH = g.OH(), OW = g.OW(), P = OH * OW, e0 = -14 * (S - 1);
    // dY per image, stored window-major ([n][p][f]) so the filter loop below reads one run.
    std::vector<int32_t> D((size_t)g.N * P * g.F);
    std::vector<int> eI(g.N);
    cpu_for(g.N, [&](int n) {
        const float* img = dy + (size_t)n * g.F * P;
        uint32_t top = 0;
        for (size_t i = 0; i < (size_t)g.F * P; ++i) top = std::max(top, conv_detail::magnitude_bits(img[i]));
        const int e = eI[n] = scale_exponent(bits_to_float(top));
        int32_t* d = D.data() + (size_t)n * P * g.F;
        for (int f = 0; f < g.F; ++f)
            for (int p = 0; p < P; ++p) d[(size_t)p * g.F + f] = fixed_point(img[(size_t)f * P + p], e, S);
    });
    // All weights with one scale, stored [c][ky][kx][f].
    const size_t nw = g.weight_size();
    uint32_t wtop = 0;
    for (size_t i = 0; i < nw; ++i) wtop = std::max(wtop, conv_detail::magnitude_bits(w[i]));
    const int eW = scale_exponent(bits_to_float(wtop));
    const int K = g.K();
    std::vector<int32_t> Wt(nw);
    for (int f = 0; f < g.F; ++f)
        for (int k = 0; k < K; ++k) Wt[(size_t)k * g.F + f] = fixed_point(w[(size_t)f * K + k], eW, S);
    // One (image, channel) plane per item; each pixel gathers the windows that cover it.
    cpu_for(g.N * g.C, [&](int plane) {
        const int n = plane / g.C, c = plane % g.C;
        const int E = eI[n] + eW + e0;
        const int32_t* dn = D.data() + (size_t)n * P * g.F;
        for (int y = 0; y < g.H; ++y) {
            for (int xx = 0; xx < g.W; ++xx) {
                int64_t t = 0;
                for (int ky = 0; ky < g.KH; ++ky) {
                    const int ry = y + g.PY - ky;
                    if (ry < 0 || ry % g.SY != 0 || ry / g.SY >= OH) continue;
                    for (int kx = 0; kx < g.KW; ++kx) {
                        const int rx = xx + g.PX - kx;
                        if (rx < 0 || rx % g.SX != 0 || rx / g.SX >= OW) continue;
                        const int32_t* d = dn + (size_t)((ry / g.SY) * OW + rx / g.SX) * g.F;
                        const int32_t* wk = Wt.data() + ((size_t)(c * g.KH + ky) * g.KW + kx) * g.F;
                        for (int f = 0; f < g.F; ++f) t += (int64_t)d[f] * wk[f];
                    }
                }
                dx[((size_t)plane * g.H + y) * g.W + xx] = round_to_float(t, E);
            }
        }
    });
}

}  // namespace repro_conv
