/*
 * repro_oracle.h -- CPU restatement of the reproducible FP32 GEMM definition.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library under
 * bit_reproducible_training_amd/) links, loads or calls this code. Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker (or as the timed CPU baseline), never as the thing shipped.
 *
 * Every function restates the scalar definition of the reference from the
 * mathematics it documents; each cites the reference file:line it follows.
 * Built with -O2 -std=c11 -pthread -fno-fast-math -ffp-contract=off, the
 * same floating-point flags the reference uses for its CPU build
 * (gpt2_ops_suite/run_suite.sh:17-18).
 *
 * Pinning (how each function is checked by tests/, independently of itself):
 *   oracle_scale_exponent  exhaustive over every non-negative finite float against an
 *                          integer formulation (correctly rounded division done in
 *                          integers), and against oracle/_ref (the reference header
 *                          compiled here) where that builds.
 *   oracle_fixed_point     exact rational arithmetic (Python fractions) on random and
 *                          edge inputs; oracle/_ref. NaN and infinite inputs (the x86
 *                          conversion, -127 * 2^(7(S-1))): whole GEMMs against oracle/_ref
 *                          and two GEMMs worked out by hand (tests/test_nonfinite.py).
 *   oracle_round_to_float  exact rational rounding to binary32 (Python ints) on
 *                          random, tie, subnormal-boundary and overflow inputs; _ref.
 *   oracle_cpu_gemm        the 21 GEMM output hashes the reference records for its
 *                          GPT-2 operation suite (gpt2_ops_suite/results/mac/cpu.txt:2-22),
 *                          brute force with Python integers on tiny shapes, and _ref.
 *   oracle_gen_normal      the 21 recorded input hashes (same lines, in= column).
 *   oracle_fnv1a64         the FNV-1a-64 published test vectors.
 *   oracle_exact_sum       exact rational sums (Python fractions) rounded to binary32 by an
 *                          integer-only rounding, on random, cancelling, tie, subnormal,
 *                          overflow and non-finite inputs, sum and mean; oracle/_ref (the
 *                          reference's repro_sum_math.cuh compiled here).
 *   oracle_has_nonfinite   numpy.isfinite on the same arrays.
 *   oracle_conv2d*         the five LeNet convolution hashes the reference records
 *                          (gpt2_ops_suite/results/mac/cpu.txt:35-39); forward and weight
 *                          gradient against oracle_cpu_gemm on the im2col matrix (an
 *                          independent path); the input gradient against brute force with
 *                          Python integers on small shapes; all three against oracle/_ref
 *                          (the reference's repro_conv_cpu.h compiled here), on finite
 *                          inputs and on inputs with NaN and infinities; a hand case
 *                          whose window holds a NaN (exponent 0).
 */
#ifndef REPRO_ORACLE_H
#define REPRO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* repro_gemm_cuda/repro_gemm_math.cuh:57-69 */
int oracle_scale_exponent(float m);
/* repro_gemm_cuda/repro_gemm_math.cuh:44-55 */
float oracle_scale_by_pow2(float x, int n);
/* repro_gemm_cuda/repro_gemm_math.cuh:71-83 */
int oracle_fixed_point(float x, int se, int S);
/* repro_gemm_cuda/repro_gemm_math.cuh:93-119 */
float oracle_round_to_float(int64_t T, int E);

/* Vectorised forms of the three scalars above (n elements), for tests. */
void oracle_scale_exponent_n(const float* m, int* e, size_t n);
void oracle_fixed_point_n(const float* x, const int* se, int S, int* X, size_t n);
void oracle_round_to_float_n(const int64_t* T, const int* E, float* out, size_t n);

/* Checks oracle_scale_exponent against an integer formulation for every float
 * whose bit pattern lies in [lo, hi) (non-negative finite range is [0, 0x7F800000)).
 * Returns the number of mismatches; *first gets the first mismatching bit pattern. */
uint64_t oracle_check_scale_exponent_range(uint32_t lo, uint32_t hi, uint32_t* first);

/* Row/column quantisation of op(A) and op(B), as the reference's CPU path does
 * (repro_gemm_cuda/repro_gemm_cpu.h:29-41): X[M][K], Y[N][K] (Y is op(B)
 * transposed), eA[M], eB[N]. ta: A stored KxM. tb: B stored NxK. */
void oracle_quantize(const float* A, const float* B, int M, int N, int K, int ta, int tb, int S,
                     int32_t* X, int32_t* Y, int* eA, int* eB, int nthreads);

/* Exact integer products T[M][N] = sum_k X[r][k] * Y[c][k] (int64). */
void oracle_exact_products(const int32_t* X, const int32_t* Y, int64_t* T, int M, int N, int K,
                           int nthreads);

/* C[M][N] = op(A) op(B), the whole definition (repro_gemm_cuda/repro_gemm_cpu.h:25-51):
 * quantise rows, quantise columns, int64 dot products, one rounding per output.
 * nthreads <= 0: hardware concurrency, or $REPRO_CPU_THREADS (repro_gemm_cpu.h:16-17).
 * Returns the thread count used. */
int oracle_cpu_gemm(const float* A, const float* B, float* C, int M, int N, int K, int ta, int tb,
                    int S, int nthreads);

/* Same as oracle_cpu_gemm, but computes only output rows [r0, r1) of C (C points at
 * row r0), still quantising op(B) over all N columns. Used to time a bounded sample. */
int oracle_cpu_gemm_rows(const float* A, const float* B, float* C, int M, int N, int K, int ta,
                         int tb, int S, int r0, int r1, int nthreads);

/* SplitMix64 + Irwin-Hall generators (repro_gemm_cuda/repro_test_util.h:30-48,
 * gpt2_ops_suite/gpt2_ops_suite.cu:59-82). out[i] = (float)(scale * draw). */
void oracle_gen_normal(float* out, size_t n, double scale, uint64_t seed);
/* The same stream, starting at element first_elem (each normal element uses 12 draws),
 * so A then B drawn from one seed is gen_normal_at(A, nA, s, 0) + gen_normal_at(B, nB, s, nA). */
void oracle_gen_normal_at(float* out, size_t n, double scale, uint64_t seed, uint64_t first_elem);
void oracle_gen_uniform(float* out, size_t n, double scale, uint64_t seed);
/* float32 U[-bound, bound) exactly as repro_torch/utils.py:23-29 (one draw per element). */
void oracle_gen_uniform_pm(float* out, size_t n, float bound, uint64_t seed, uint64_t first_elem);
/* rows x cols adversarial dynamic range: random signs, |x| = 2^e with e ~ U[-60, 60],
 * 5% exact zeros, 1% subnormals. Elements come in pairs (columns c, c^1, or rows r, r^1
 * when pair_rows): the second is the first times (1 + 2^-20 t), t in {-1,0,1}, negated
 * when negate is set, so negated pairs in op(A) against plain pairs in op(B) cancel
 * almost exactly in every dot product. */
void oracle_gen_adversarial(float* out, int rows, int cols, uint64_t seed, int pair_rows, int negate);
/* hash_repro_gemm.cu:20-56 input distributions (0 uniform, 1 normal, 2 weights, 3 wide, 4 stress)
 * from one sequential stream; returns 1 for a bad argument. */
int oracle_gen_hash_inputs(float* A, float* B, int M, int N, int K, uint64_t seed, int dist);
/* Raw stream: n successive SplitMix64 outputs. */
void oracle_splitmix64(uint64_t* out, size_t n, uint64_t seed);

/* out[b] = exact sum over a, c of x[a][b][c] (x is [A][B][C] row-major), rounded once to
 * float32 nearest-even, or the exact sum / (A*C) when mean; NaN if any summand is NaN or
 * infinite; an exactly zero sum is +0.0 (repro_sum_cuda/repro_sum_math.cuh:66-157,
 * repro_torch/src/bindings.cpp:69-91). */
void oracle_exact_sum(const float* x, float* out, int A, int B, int C, int mean);
/* 1 if x[0..n) holds a NaN or infinity (repro_torch/src/kernels.cu:10-14). */
int oracle_has_nonfinite(const float* x, size_t n);

/* Convolution geometry (repro_conv_cuda/repro_conv_math.cuh:29-42): input [N][C][H][W],
 * weight [F][C][KH][KW], stride SY, SX, zero padding PY, PX. */
typedef struct oracle_conv_shape {
    int N, C, H, W, F, KH, KW, SY, SX, PY, PX;
} oracle_conv_shape;
/* out[N][F][OH][OW] (repro_conv_cuda/repro_conv_cpu.h:23-38). */
void oracle_conv2d(const float* x, const float* w, float* out, const oracle_conv_shape* g, int S);
/* dW[F][C][KH][KW] from dY[N][F][OH][OW] and x (repro_conv_cpu.h:40-70). */
void oracle_conv2d_grad_weight(const float* dy, const float* x, float* dw,
                               const oracle_conv_shape* g, int S);
/* dX[N][C][H][W] from dY and the weights (repro_conv_cpu.h:72-91). */
void oracle_conv2d_grad_input(const float* dy, const float* w, float* dx,
                              const oracle_conv_shape* g, int S);

/* FNV-1a 64 over raw bytes, chained from h (repro_gemm_cuda/repro_test_util.h:20-24). */
uint64_t oracle_fnv1a64(const void* data, size_t n, uint64_t h);

#ifdef __cplusplus
}
#endif
#endif
