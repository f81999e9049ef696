/*
 * repro_conv.h -- flat C ABI of the reproducible 2D convolution and its two gradients on
 * MI355X (gfx950), in PyTorch layouts:
 *
 *   rg_conv2d_ws:             out[N][F][OH][OW] from x[N][C][H][W], weight[F][C][KH][KW]
 *   rg_conv2d_grad_weight_ws: dW[F][C][KH][KW] from dY[N][F][OH][OW], x
 *   rg_conv2d_grad_input_ws:  dX[N][C][H][W]   from dY[N][F][OH][OW], weight
 *
 * Definition (repro_conv_cuda/repro_conv_math.cuh:1-18): every input gets a power-of-two
 * scale, is rounded once to a 7*S-bit integer, products are summed exactly and the sum is
 * rounded once to FP32. The forward pass and the weight gradient are the reproducible GEMM
 * on the im2col matrix (scales per window and per filter, per filter and per window
 * position); the input gradient uses one scale per image for dY and one for all weights, so
 * each pixel's terms (several windows, all filters) share a scale. Here all three run on the
 * int8 MFMA contraction of librepro_gemm.so. Output bits depend only on the inputs, the
 * shape and S. Bias is not included (add it; its gradient is rg_sum_fp32_ws). Small filters
 * take direct kernels instead (forward and input gradient, at most 2048 products per sum):
 * one launch, binary64 sums that are exact integers at that length, the same bits.
 *
 * Plain C types only; the stream is a hipStream_t passed as void*. Return values are
 * hipError_t codes (0 success, 1 invalid value, 801 not supported, others from HIP).
 */
#ifndef REPRO_CONV_H
#define REPRO_CONV_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* repro_conv_cuda/repro_conv_math.cuh:29-42 (same fields; stride defaults 1, padding 0). */
typedef struct rg_conv_shape {
    int N, C, H, W; /* input [N][C][H][W] */
    int F, KH, KW;  /* weight [F][C][KH][KW] */
    int SY, SX;     /* stride */
    int PY, PX;     /* zero padding */
} rg_conv_shape;

/* Zeroes the shape and sets the stride to 1. */
void rg_conv_shape_init(rg_conv_shape* g);

/* Replace conv2d_workspace / conv2d_grad_weight_workspace / conv2d_grad_input_workspace
 * (repro_conv_cuda/repro_conv.cuh:21-23, repro_conv.cu:171-187). 1 (invalid value) for a null
 * argument, S outside 1..3, non-positive sizes or stride, negative padding, a kernel larger
 * than the padded image, tensors of 2^31 or more elements, or more terms in one exact sum than
 * int64 holds at this S (windows, KH*KW*F or C*KH*KW above 9e18 / (127*128^(S-1))^2; the
 * reference's same bound, repro_conv_math.cuh:159-163). The reference's kernel-specific limits
 * (C*KH*KW <= 1024, F <= 256, N <= 65535) do not apply here. 801 on a device that is not
 * gfx950. The size depends on the shape, S and the current device. */
int rg_conv2d_workspace(const rg_conv_shape* g, int S, size_t* bytes);
int rg_conv2d_grad_weight_workspace(const rg_conv_shape* g, int S, size_t* bytes);
int rg_conv2d_grad_input_workspace(const rg_conv_shape* g, int S, size_t* bytes);

/* Replace repro_conv2d_ws / repro_conv2d_grad_weight_ws / repro_conv2d_grad_input_ws
 * (repro_conv_cuda/repro_conv.cuh:26-31, repro_conv.cu:189-241). Asynchronous on `stream`,
 * allocation-free. Errors as the workspace functions, plus 1 for null tensors or a workspace
 * that is null or too small, and any launch error. Inputs are meant to be finite; a NaN or an
 * infinity gives the bits of the reference's CPU convolution (a NaN wins a window's or a
 * position's maximum, which then takes exponent 0). */
int rg_conv2d_ws(const float* x, const float* weight, float* out, const rg_conv_shape* g, int S,
                 void* workspace, size_t workspace_bytes, void* stream);
int rg_conv2d_grad_weight_ws(const float* dy, const float* x, float* dw, const rg_conv_shape* g,
                             int S, void* workspace, size_t workspace_bytes, void* stream);
int rg_conv2d_grad_input_ws(const float* dy, const float* weight, float* dx,
                            const rg_conv_shape* g, int S, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Diagnostic hooks, with no counterpart in the reference: a pass run with its algorithm
 * forced, for tests and benchmarks. pass: RG_CONV_FORWARD (a = x, b = weight),
 * RG_CONV_GRAD_WEIGHT (a = dy, b = x) or RG_CONV_GRAD_INPUT (a = dy, b = weight). algo:
 * RG_CONV_ALGO_AUTO (the choice of the entry points above), RG_CONV_ALGO_GEMM (im2col and the
 * int8 MFMA GEMM pipeline) or RG_CONV_ALGO_DIRECT (forward and input gradient only, while one
 * sum has at most 2048 products and, forward, F*C*KH*KW <= 4096; else 801). Both algorithms
 * give the same bits. rg_conv2d_algo reports what AUTO resolves to; errors as above, plus 1 for
 * an unknown pass or algo. */
enum { RG_CONV_FORWARD = 0, RG_CONV_GRAD_WEIGHT = 1, RG_CONV_GRAD_INPUT = 2 };
enum { RG_CONV_ALGO_AUTO = 0, RG_CONV_ALGO_GEMM = 1, RG_CONV_ALGO_DIRECT = 2 };
int rg_conv2d_algo(int pass, const rg_conv_shape* g, int S, int* algo);
int rg_conv2d_algo_workspace(int pass, const rg_conv_shape* g, int S, int algo, size_t* bytes);
int rg_conv2d_algo_ws(int pass, const float* a, const float* b, float* out, const rg_conv_shape* g,
                      int S, int algo, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
