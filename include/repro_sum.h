/*
 * repro_sum.h -- flat C ABI of the exact, order-independent float32 sum on MI355X (gfx950),
 * and of the non-finite scan the layers use to stop on NaN/Inf.
 *
 * x is viewed as a row-major [A][B][C] tensor. For every b,
 *   out[b] = round_to_float32(exact sum over a, c of x[a][b][c])          (mean = 0)
 *   out[b] = round_to_float32(exact sum over a, c of x[a][b][c] / (A*C))  (mean = 1)
 * rounded once, nearest-even. The exact sum is held in a 320-bit integer accumulator, so the
 * bits never depend on data order, chunking, launch configuration or the GPU. An exactly zero
 * result is +0.0; NaN or infinity among the summands gives NaN. Requires A*C <= 2^31 - 1.
 * The scalar arithmetic is include/repro_sum_math.h.
 *
 * Plain C types only; the stream is a hipStream_t passed as void*. Return values are
 * hipError_t codes (0 success, 1 invalid value, others from the HIP runtime).
 */
#ifndef REPRO_SUM_H
#define REPRO_SUM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* repro_sum_cuda/repro_sum.cuh:27-30 (same fields and defaults). chunks: work split along
 * the A*C summands of each output, 0 = chosen for the shape and device. */
typedef struct rg_sum_config {
    int chunks;
    int mean;
} rg_sum_config;

/* repro_sum_cuda/repro_sum.cuh:32-35. */
typedef struct rg_sum_plan {
    int chunks;
    size_t workspace_bytes; /* 0 when one chunk per output (then no workspace is needed) */
} rg_sum_plan;

void rg_sum_config_init(rg_sum_config* cfg);

/* Replaces repro_sum::make_sum_plan (repro_sum_cuda/repro_sum.cuh:37,
 * repro_sum.cu:183-230). 1 (invalid value): null cfg/plan, A/B/C <= 0, chunks < 0, or
 * A*C > 2^31 - 1. Queries the current device's compute-unit count when chunks == 0. */
int rg_make_sum_plan(int A, int B, int C, const rg_sum_config* cfg, rg_sum_plan* plan);

/* The planner with an explicit compute-unit count (no device query), for host code without a
 * GPU. No counterpart in the reference. */
int rg_sum_plan_for_device(int A, int B, int C, const rg_sum_config* cfg, int num_cus,
                           rg_sum_plan* plan);

/* Replaces repro_sum::repro_sum_fp32_ws (repro_sum_cuda/repro_sum.cuh:39-41,
 * repro_sum.cu:232-259). Asynchronous on `stream`, allocation-free. Errors as
 * rg_make_sum_plan, plus 1 for null x/out or a workspace that is needed and null or too
 * small, and any launch error. */
int rg_sum_fp32_ws(const float* x, float* out, int A, int B, int C, const rg_sum_config* cfg,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Replaces repro_sum::repro_sum_fp32 (repro_sum_cuda/repro_sum.cuh:43-45,
 * repro_sum.cu:261-271): allocates the workspace, runs, synchronises the stream, frees. */
int rg_sum_fp32(const float* x, float* out, int A, int B, int C, const rg_sum_config* cfg,
                void* stream);

/* Replaces repro_scan_finite (repro_torch/src/kernels.cu:8-20): lowers the device int
 * *flag to op_id if x[0..n) holds a NaN or infinity; stream-ordered, never synchronises.
 * n == 0 launches nothing. 1 (invalid value): null x or flag with n > 0. */
int rg_scan_finite(const float* x, int* flag, size_t n, int op_id, void* stream);

#ifdef __cplusplus
}
#endif
#endif
