#pragma once
// C++ interface of the reproducible GEMM with the names and signatures of
// repro_gemm_cuda/repro_gemm.cuh:25-75, on HIP types. Header-only: every function is an
// inline wrapper over the flat C ABI in repro_gemm.h, so C++ callers (a Conv2d layer,
// a framework binding, the tests) link only against C symbols of librepro_gemm.so.
//
// C[M,N] = op(A)[M,K] * op(B)[K,N], FP32, row-major. The result is bit-identical across
// runs, split_k values, tile sizes and GPUs, and equal to a CPU implementation of the same
// definition. S=1: 7-bit inputs, 1 int8 product; S=2: 14-bit, 4; S=3: 21-bit, 9 (default).
// Inputs are meant to be finite; a NaN or an infinity still gives the bits of the reference's
// CPU path (see fixed_point in repro_gemm_math.h). Do not build with -ffast-math or denormal
// flushing.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "repro_gemm.h"
#include "repro_gemm_math.h"

namespace repro_gemm {

enum class Algo {
    Auto = RG_ALGO_AUTO,             // MFMA contraction, block tile chosen for the shape
    Reference = RG_ALGO_REFERENCE,   // one thread per output, int64; slow, for verification
    Tiled = RG_ALGO_TILED,           // MFMA contraction, 64x64 block tile
    TensorCore = RG_ALGO_TENSOR_CORE // MFMA contraction, block tile chosen for the shape
};

// Field names, order and defaults are the reference's (repro_gemm.cuh:32-41); the meaning of
// each field on this GPU:
struct Config {
    int split_k = 1;        // K-parts summed in int64; the planner may use more (int32 chunk
                            // limit, or to fill the GPU); never changes a bit of C
    int tile_m = 16;        // 64 or 128 (with tile_n; 64x192 / 192x64 at S = 3) pins that MFMA
    int tile_n = 16;        //   block tile, 32x32 the one-launch kernel for K <= 512, 32xW
                            //   (W >= 64) the band kernel for K <= 1024; other values leave
                            //   the choice to the planner
    int tile_k = 32;        // not used
    Algo algo = Algo::Auto;
    int slices = 3;         // S in 1..MAX_SLICES: inputs rounded to 7*S-bit integers
    bool trans_a = false;   // A stored K rows of M (op(A) = A^T) instead of M rows of K
    bool trans_b = false;   // B stored N rows of K (op(B) = B^T) instead of K rows of N
};

// The planner's decision for one shape and Config on the current device.
struct Plan {
    Algo algo;               // the algorithm that runs: TensorCore, Tiled or Reference
    int split_k;             // K-parts the launch sums (the request, raised or clamped)
    size_t workspace_bytes;  // the smallest workspace repro_gemm_fp32_ws accepts for it
};

inline rg_config to_c(const Config& c) {
    rg_config r;
    r.split_k = c.split_k;
    r.tile_m = c.tile_m;
    r.tile_n = c.tile_n;
    r.tile_k = c.tile_k;
    r.algo = static_cast<int>(c.algo);
    r.slices = c.slices;
    r.trans_a = c.trans_a ? 1 : 0;
    r.trans_b = c.trans_b ? 1 : 0;
    return r;
}

// Errors: hipErrorNotSupported when the device is not gfx950 and cfg.algo needs the MFMA
// contraction; hipErrorInvalidValue for sizes <= 0, S outside 1..3, a split_k <= 0, or a K
// whose exact int64 sums could overflow at this S.
inline hipError_t make_plan(int M, int N, int K, Config cfg, Plan* plan) {
    if (!plan) return hipErrorInvalidValue;
    rg_config c = to_c(cfg);
    rg_plan p;
    int e = rg_make_plan(M, N, K, &c, &p);
    if (e == 0) {
        plan->algo = static_cast<Algo>(p.algo);
        plan->split_k = p.split_k;
        plan->workspace_bytes = p.workspace_bytes;
    }
    return static_cast<hipError_t>(e);
}

// The GEMM queued on `stream` with the caller's workspace (plan.workspace_bytes or more);
// nothing is allocated and nothing waits, so a training loop calls this one. stage_events,
// if non-null, are 4 events this call records on `stream`: before the slicing, after it,
// after the contraction and after the final rounding.
inline hipError_t repro_gemm_fp32_ws(const float* A, const float* B, float* C, int M, int N,
                                     int K, Config cfg, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream = nullptr,
                                     const hipEvent_t* stage_events = nullptr) {
    rg_config c = to_c(cfg);
    return static_cast<hipError_t>(rg_gemm_fp32_ws(
        A, B, C, M, N, K, &c, workspace, workspace_bytes, static_cast<void*>(stream),
        reinterpret_cast<void* const*>(stage_events)));
}

// One-shot form: takes a workspace of its own with hipMalloc, runs repro_gemm_fp32_ws, waits
// for the stream and releases the workspace (returning the first error met).
inline hipError_t repro_gemm_fp32(const float* A, const float* B, float* C, int M, int N, int K,
                                  Config cfg = Config(), hipStream_t stream = nullptr) {
    rg_config c = to_c(cfg);
    return static_cast<hipError_t>(
        rg_gemm_fp32(A, B, C, M, N, K, &c, static_cast<void*>(stream)));
}

inline const char* algo_name(Algo a) { return rg_algo_name(static_cast<int>(a)); }

}  // namespace repro_gemm
