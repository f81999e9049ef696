/*
 * repro_gemm.h -- flat C ABI of the MI355X (gfx950) reproducible FP32 GEMM.
 *
 * C[M,N] = op(A)[M,K] * op(B)[K,N], FP32 in and out, row-major, where every row of
 * op(A) and column of op(B) gets a power-of-two scale, every input is rounded once
 * to a 7*S-bit integer split into S int8 digits, the digit products are contracted
 * exactly on CDNA4 int8 MFMA (int32 inside overflow-safe K chunks, int64 across
 * chunks and split-K), and the exact integer result is rounded once to FP32.
 * Output bits depend only on the input bits, M, N, K, S and the transposes: never on
 * tiling, split-K, launch configuration or the GPU.
 *
 * Plain C types only (no HIP or torch types): the stream is a hipStream_t passed as
 * void*, stage events are hipEvent_t passed as void*. Return values are hipError_t
 * codes: 0 success, 1 invalid value, 801 not supported, others from the HIP runtime.
 * The C++ interface with the reference's names is repro_gemm.hpp (inline over this).
 */
#ifndef REPRO_GEMM_H
#define REPRO_GEMM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Algorithm selector; values follow repro_gemm_cuda/repro_gemm.cuh:25-30.
 * AUTO and TENSOR_CORE run the int8 MFMA contraction with the block tile chosen for
 * the shape; TILED forces the 64x64 MFMA block tile; REFERENCE is the one-thread-
 * per-output int64 kernel, kept for verification. */
enum {
    RG_ALGO_AUTO = 0,
    RG_ALGO_REFERENCE = 1,
    RG_ALGO_TILED = 2,
    RG_ALGO_TENSOR_CORE = 3
};

/* repro_gemm_cuda/repro_gemm.cuh:32-41 (same fields, order and defaults).
 * tile_m/tile_n: the reference ignores them; here a pair naming an MFMA block tile
 * (128x128, 128x64, 64x128, 64x64, and at slices = 3 64x192 or 192x64) forces that tile;
 * 32x32 asks for the one-launch small-GEMM kernel (K <= 512, default split_k, plain GEMMs);
 * 32xW (W >= 64, a multiple of 32) asks for the band kernel with blocks of 32 rows of op(A)
 * by W columns (op(A) not transposed, K <= 1024, default split_k, plain GEMMs);
 * anything else lets the planner choose. tile_k is ignored. */
typedef struct rg_config {
    int split_k;  /* >= 1; raised when needed for exact int32 sums, and from the default 1
                     when the output tiles alone cannot occupy the GPU */
    int tile_m;   /* default 16 */
    int tile_n;   /* default 16 */
    int tile_k;   /* default 32, ignored */
    int algo;     /* RG_ALGO_*, default RG_ALGO_AUTO */
    int slices;   /* S in 1..3, default 3 */
    int trans_a;  /* 0: A is MxK row-major. 1: A is KxM row-major (use A^T) */
    int trans_b;  /* 0: B is KxN row-major. 1: B is NxK row-major (use B^T) */
} rg_config;

/* repro_gemm_cuda/repro_gemm.cuh:44-48, plus the block tile actually used. */
typedef struct rg_plan {
    int algo;               /* resolved, never RG_ALGO_AUTO */
    int split_k;            /* effective split count */
    size_t workspace_bytes; /* size needed by rg_gemm_fp32_ws */
    int tile_m;             /* block tile rows (MFMA algorithms; 32: one-launch or band kernel), 0 for REFERENCE */
    int tile_n;             /* block tile columns */
} rg_plan;

/* Fills *cfg with the defaults of repro_gemm::Config. */
void rg_config_init(rg_config* cfg);

/* Replaces repro_gemm::make_plan (repro_gemm_cuda/repro_gemm.cuh:53, repro_gemm.cu:503-509).
 * 1 (invalid value): cfg or plan null, M/N/K <= 0, split_k <= 0, slices outside 1..3,
 *   or K too large for exact int64 at this S (S=3 allows K up to about 1,000,000).
 * 801 (not supported): an MFMA algorithm on a device that is not gfx950.
 * Queries the current device for its architecture and compute-unit count. */
int rg_make_plan(int M, int N, int K, const rg_config* cfg, rg_plan* plan);

/* Replaces repro_gemm::repro_gemm_fp32_ws (repro_gemm_cuda/repro_gemm.cuh:60-66,
 * repro_gemm.cu:511-528). Asynchronous on `stream` (a hipStream_t; NULL = default
 * stream), allocates nothing and synchronises nothing. workspace must hold at least
 * plan.workspace_bytes (hipMalloc alignment); its size depends only on (M, N, K, cfg)
 * and the device. stage_events, if not NULL, points to 4 hipEvent_t recorded on
 * `stream` before slicing, after slicing, after the contraction and after the
 * final rounding. Errors as rg_make_plan, plus 1 for null A/B/C or a workspace that is
 * null or too small, and any launch error. */
int rg_gemm_fp32_ws(const float* A, const float* B, float* C, int M, int N, int K,
                    const rg_config* cfg, void* workspace, size_t workspace_bytes, void* stream,
                    void* const* stage_events);

/* Replaces repro_gemm::repro_gemm_fp32 (repro_gemm_cuda/repro_gemm.cuh:69-73,
 * repro_gemm.cu:530-542): allocates the workspace, runs, synchronises the stream to
 * surface asynchronous errors, frees. */
int rg_gemm_fp32(const float* A, const float* B, float* C, int M, int N, int K,
                 const rg_config* cfg, void* stream);

/* Replaces repro_gemm::algo_name (repro_gemm_cuda/repro_gemm.cuh:75, repro_gemm.cu:493-501):
 * "auto", "ref", "tiled", "tc". */
const char* rg_algo_name(int algo);

/* Text of a returned error code (hipGetErrorString). */
const char* rg_error_string(int code);

/* Byte offsets of the internal workspace regions for (M, N, K, cfg) on the current
 * device, for tests that inspect the sliced operands. No counterpart in the
 * reference (its layout is private). qa/qb: digit panels of op(A)/op(B); ea/eb:
 * int32 exponents; part: int64 split-K partials [split][M][N] (or -1 if unused).
 * Panel layout: [row/32][k/32][digit][1024 bytes], byte (lane*16 + j) of a panel holding
 * element (row%32 = lane%32, k%32 = 16*(lane/32) + j). Kp (padded K), Mp, Np returned.
 * REFERENCE stores int32 fixed-point values [Rp][Kp] row-major instead of digits. */
typedef struct rg_layout_info {
    size_t qa, qb, ea, eb;
    long long part;
    int Mp, Np, Kp;
    int split_k;
} rg_layout_info;
int rg_workspace_layout(int M, int N, int K, const rg_config* cfg, rg_layout_info* info);

/* The planner with an explicit device description instead of a query of the current
 * device (is_gfx950: 1 if the device is gfx950; num_cus: its compute units), so host
 * code can plan without a GPU. No counterpart in the reference (its planner always
 * queries the device, repro_gemm_cuda/repro_gemm.cu:398-408). info may be NULL. */
int rg_plan_for_device(int M, int N, int K, const rg_config* cfg, int is_gfx950, int num_cus,
                       rg_plan* plan, rg_layout_info* info);

/* Test hook, no counterpart in the reference: which output tile each workgroup of the MFMA
 * contraction computes, for the plan rg_plan_for_device makes (same arguments, batch items).
 * *blocks receives the contraction's workgroup count (0 when the plan has no MFMA contraction:
 * the reference algorithm or the one-launch small kernel). If coords is non-NULL and capacity
 * >= 4 * *blocks, coords[4 i .. 4 i + 3] receives (item, split part, tile row, tile column)
 * of the workgroup with linear id i (tiles of plan->tile_m x plan->tile_n); the hardware
 * deals workgroup i to XCD i mod 8. Host only; 1 (invalid value) as rg_plan_for_device, or
 * for batch outside 1..65535. */
int rg_test_block_order(int M, int N, int K, const rg_config* cfg, int is_gfx950, int num_cus,
                        int batch, int* coords, long long capacity, long long* blocks);

/* Test hook, no counterpart in the reference: where the one-read slicing (operands whose padded
 * K is past the one-pass limit) places its blocks, for the plan rg_test_block_order makes (same
 * arguments). *blocks receives the one-read blocks of both operands (0 when neither takes that
 * route) and *split_panels the number of row panels (strips of 8 rows for row access) whose
 * parts along K run on more than one XCD (workgroup i on XCD i mod 8); such parts cannot see
 * each other's partial maxima through their L2 and each waits out its bound. Host only;
 * 1 (invalid value) as rg_test_block_order. */
int rg_test_pslice_placement(int M, int N, int K, const rg_config* cfg, int num_cus, int batch,
                             long long* blocks, long long* split_panels);

/* Test hook, no counterpart in the reference: the GPU epilogue's final rounding on arrays,
 * so tests can compare it with round_to_float on chosen inputs. Exactly one of levels and T
 * is non-NULL. levels: n x (2S-1) int32 level sums per output, most significant first, rounded
 * as the contraction's epilogue rounds T = sum_l levels[l] * 2^(7 (2S-2-l)); T: n int64
 * values rounded as the split-K reduction does. out[i] = round_to_float(T_i, E[i]).
 * Device pointers; asynchronous on stream; 1 (invalid value) for bad arguments or
 * n > 2^30. */
int rg_test_round(const int* levels, const long long* T, const int* E, float* out, long long n,
                  int S, void* stream);

/* Test hook, no counterpart in the reference: the bound on a slicing block's wait for the
 * other k ranges of its row panel (long column-access operands, whose blocks exchange partial
 * maxima), in polls; past it the block reads the panel's whole K itself, which gives the same
 * bits. Applies to launches made after the call. polls = 0 makes every such block take the
 * fallback (tests of that path); a negative value restores the default. Returns the previous
 * bound. Host only, process-wide. */
int rg_test_set_spin_limit(int polls);

/* Strided-batched GEMM, no counterpart in the reference (which lists it as still needed for
 * attention: README.md:29, repro_gemm_cuda/README.md:106). batch independent GEMMs
 *   C_b[M,N] = op(A_b) op(B_b),  A_b = A + b*stride_a, B_b = B + b*stride_b, C_b = C + b*stride_c
 * with leading dimensions (elements between rows of the stored matrices): A_b is MxK with
 * row stride lda (KxM if trans_a), B_b is KxN with row stride ldb (NxK if trans_b), C_b is MxN
 * with row stride ldc. Every item is bit-identical to rg_gemm_fp32_ws on that item alone
 * (its own row and column scales). Items of C must not overlap. 1 (invalid value) as
 * rg_make_plan, plus batch outside 1..65535, lda < (trans_a ? M : K), ldb < (trans_b ? K : N),
 * ldc < N, or a negative stride. Asynchronous, allocation-free. */
int rg_make_plan_strided_batched(int M, int N, int K, int batch, const rg_config* cfg,
                                 rg_plan* plan);
int rg_gemm_strided_batched_fp32_ws(const float* A, long long lda, long long stride_a,
                                    const float* B, long long ldb, long long stride_b, float* C,
                                    long long ldc, long long stride_c, int M, int N, int K,
                                    int batch, const rg_config* cfg, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* No counterpart in the reference: rg_gemm_fp32_ws for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is a fixed device array inside the library, RG_NOALLOC_SCRATCH_BYTES (128 MiB)
 * on each GPU, held from the first call on that GPU until the process ends (the array sits in
 * a code object of its own, loaded on that first call: loading the library or running the
 * other entry points reserves none of it); this entry point
 * calls no hipMalloc/hipFree and no allocating library routine. The caller passes A, B, C as
 * for rg_gemm_fp32_ws. Returns 1 (invalid value) when the plan's workspace_bytes
 * (rg_make_plan) exceeds RG_NOALLOC_SCRATCH_BYTES (4096^3 at S = 3 needs about 96 MiB), or
 * for the arguments rg_gemm_fp32_ws rejects. Every call on one GPU uses that GPU's array:
 * calls that overlap on one GPU (two streams, two host threads) race and must be ordered on
 * one stream. Same bits as rg_gemm_fp32_ws. Asynchronous on `stream`. */
#define RG_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int rg_gemm_fp32_noalloc(const float* A, const float* B, float* C, int M, int N, int K,
                         const rg_config* cfg, void* stream);

/* Diagnostic, no counterpart in the reference: the sustained int8 MFMA rate of the current
 * (gfx950) device in TOP/s, measured with a kernel that keeps its operands in registers
 * (no memory traffic) for about a millisecond. dense = 1: random operand bytes; dense = 2:
 * random bytes in [0, 127] (as the contraction's lower digit planes); dense = 0: zero
 * operands. The first two are practical ceilings of the contraction under the device's
 * power limit. 1 (invalid value) for another dense. Allocates a few KiB of device memory and
 * synchronises its own stream. */
int rg_measure_mfma_int8_rate(int dense, double* tops);

#ifdef __cplusplus
}
#endif
#endif
