// Exact, order-independent float32 sums (bias gradients, loss means) and the non-finite
// scan, for the layers built on the reproducible GEMM.
//
// Accumulation: every thread owns a 10-limb superaccumulator in LDS (limb l of thread t at
// acc[l][t], radix 2^32, limb l weighing 2^(32 l - 149)). A finite float is one wide term
// v < 2^55 at limb idx = (biased exponent - 1) / 32 (repro_sum::wide_term), added with a
// single 64-bit LDS read-modify-write; nobody else touches that address, so no atomics are
// needed. At most 252 wide adds land between carry resolutions, which keeps every limb below
// 2^32 + 252 * 2^55 < 2^63. Threads, waves, blocks and chunks are then merged by integer
// addition of normalised limbs (exact and associative), and one thread per output divides
// exactly (for a mean) and rounds once (repro_sum::finalize).
//
// Kernels by layout of x = [A][B][C]:
//   C == 1   columns: a 256-thread block covers 64 outputs x 4 row phases; a wave reads
//            64 consecutive floats of one row (bias gradient of a Linear layer).
//   C >  1   segments: one wave per (output, chunk) walks contiguous runs of C floats
//            (conv bias gradient, loss mean, row sums).
// With more than one chunk per output, the chunks' limbs go to the workspace and a third
// kernel merges and rounds them.
#include "rg_internal.h"
#include "repro_sum.h"
#include "repro_sum_math.h"

#include <algorithm>
#include <climits>

namespace rg {
namespace {

using repro_sum::LIMBS;

constexpr int SUM_THREADS = 256;
constexpr int GROUP = 4;          // loads issued together per thread
constexpr int FLUSH_AT = 252;     // wide adds per limb between carry resolutions
constexpr size_t SUM_ALIGN = 256;

size_t align_up(size_t x) { return (x + SUM_ALIGN - 1) / SUM_ALIGN * SUM_ALIGN; }

// Thread-private accumulator in LDS: limb l at p[l * SUM_THREADS].
struct LdsAcc {
    int64_t* p;

    __device__ void clear() {
#pragma unroll
        for (int l = 0; l < LIMBS; ++l) p[l * SUM_THREADS] = 0;
    }
    __device__ void add(float x, int& nonfinite) {
        int idx;
        uint64_t v;
        bool neg;
        if (!repro_sum::wide_term(x, idx, v, neg)) {
            nonfinite = 1;
            return;
        }
        p[idx * SUM_THREADS] += neg ? -(int64_t)v : (int64_t)v;
    }
    // Carries: limbs 0..LIMBS-2 into [0, 2^32), the top limb keeps the sign.
    __device__ void carry() {
        int64_t c = 0;
#pragma unroll
        for (int l = 0; l < LIMBS; ++l) {
            int64_t t = p[l * SUM_THREADS] + c;
            if (l + 1 < LIMBS) {
                c = t >> 32;
                t -= c * ((int64_t)1 << 32);
            }
            p[l * SUM_THREADS] = t;
        }
    }
};

// Writes one output's merged limbs: rounds them when this is the only chunk, else stores them
// as chunk `chunk` of output b.
__device__ void emit(const int64_t* limbs, int stride, int nonfinite, int b, int B, int chunk,
                     int chunks, uint32_t divisor, float* out, int64_t* part, int* part_nf) {
    if (chunks == 1) {
        out[b] = repro_sum::finalize(limbs, stride, divisor, nonfinite);
    } else {
#pragma unroll
        for (int l = 0; l < LIMBS; ++l)
            part[((size_t)chunk * LIMBS + l) * B + b] = limbs[l * stride];
        part_nf[(size_t)chunk * B + b] = nonfinite;
    }
}

// C == 1. Block = 64 outputs (lanes) x 4 row phases (waves); chunk = blockIdx.y covers rows
// [a0, a1), phase w takes rows a0 + w, a0 + w + 4, ...
__global__ void __launch_bounds__(SUM_THREADS)
sum_columns(const float* __restrict__ x, int A, int B, int rows_per_chunk, int chunks,
            uint32_t divisor, float* __restrict__ out, int64_t* __restrict__ part,
            int* __restrict__ part_nf) {
    __shared__ int64_t acc[LIMBS * SUM_THREADS];
    __shared__ int nf_sh[SUM_THREADS];
    const int t = threadIdx.x, col = t & 63, phase = t >> 6;
    const int b = blockIdx.x * 64 + col;
    const int chunk = blockIdx.y;
    const int a0 = chunk * rows_per_chunk;
    const int a1 = min(A, a0 + rows_per_chunk);
    LdsAcc acc_t{acc + t};
    acc_t.clear();
    int nf = 0;
    if (b < B) {
        int since = 0;
        for (int a = a0 + phase; a < a1; a += 4 * GROUP) {
            float v[GROUP];
#pragma unroll
            for (int g = 0; g < GROUP; ++g) {
                const int r = a + 4 * g;
                v[g] = r < a1 ? x[(size_t)r * B + b] : 0.0f;
            }
#pragma unroll
            for (int g = 0; g < GROUP; ++g) acc_t.add(v[g], nf);
            since += GROUP;
            if (since >= FLUSH_AT) {
                acc_t.carry();
                since = 0;
            }
        }
    }
    acc_t.carry();
    nf_sh[t] = nf;
    __syncthreads();
    if (phase == 0 && b < B) {
#pragma unroll
        for (int l = 0; l < LIMBS; ++l) {
            int64_t s = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) s += acc[l * SUM_THREADS + t + 64 * w];
            acc[l * SUM_THREADS + t] = s;
        }
        const int nfb = nf_sh[t] | nf_sh[t + 64] | nf_sh[t + 128] | nf_sh[t + 192];
        emit(acc + t, SUM_THREADS, nfb, b, B, chunk, chunks, divisor, out, part, part_nf);
    }
}

// C > 1. Wave w of block x handles item 4 x + w of the B * chunks (output, chunk) items,
// output b = item / chunks, chunk item % chunks: summands [i0, i1) of the A*C values of b, in
// order a-major, walked as contiguous runs of x. Every wave of a block has work when
// B * chunks fills the grid, however small B is.
__global__ void __launch_bounds__(SUM_THREADS)
sum_segments(const float* __restrict__ x, int A, int B, int C, int chunks, uint32_t divisor,
             float* __restrict__ out, int64_t* __restrict__ part, int* __restrict__ part_nf) {
    __shared__ int64_t acc[LIMBS * SUM_THREADS];
    __shared__ int64_t merged[4][LIMBS];
    __shared__ int nf_sh[SUM_THREADS];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const long long item = (long long)blockIdx.x * 4 + w;
    const int b = item < (long long)B * chunks ? (int)(item / chunks) : B;  // B: no work
    const int chunk = b < B ? (int)(item - (long long)b * chunks) : 0;
    LdsAcc acc_t{acc + t};
    acc_t.clear();
    int nf = 0;
    if (b < B) {
        const long long count = (long long)A * C;
        const long long i0 = count * chunk / chunks, i1 = count * (chunk + 1) / chunks;
        int a = (int)(i0 / C);
        int c = (int)(i0 - (long long)a * C);
        long long left = i1 - i0;
        int since = 0;
        while (left > 0) {
            const int len = (int)std::min<long long>(C - c, left);
            const float* p = x + ((size_t)a * B + b) * C + c;
            for (int j = lane; j < len; j += 64 * GROUP) {
                float v[GROUP];
#pragma unroll
                for (int g = 0; g < GROUP; ++g) {
                    const int k = j + 64 * g;
                    v[g] = k < len ? p[k] : 0.0f;
                }
#pragma unroll
                for (int g = 0; g < GROUP; ++g) acc_t.add(v[g], nf);
                since += GROUP;
                if (since >= FLUSH_AT) {
                    acc_t.carry();
                    since = 0;
                }
            }
            left -= len;
            ++a;
            c = 0;
        }
    }
    acc_t.carry();
    nf_sh[t] = nf;
    __syncthreads();
    if (b < B && lane < LIMBS) {
        int64_t s = 0;
        for (int j = 0; j < 64; ++j) s += acc[lane * SUM_THREADS + 64 * w + j];  // < 2^38
        merged[w][lane] = s;
    }
    if (b < B && lane == LIMBS) {
        int any = 0;
        for (int j = 0; j < 64; ++j) any |= nf_sh[64 * w + j];
        nf_sh[64 * w] = any;  // read back by lane 0 of this wave after the barrier
    }
    __syncthreads();
    if (b < B && lane == 0)
        emit(merged[w], 1, nf_sh[64 * w], b, B, chunk, chunks, divisor, out, part, part_nf);
}

// Merges the chunks of each output and rounds once. Few chunks: a thread per output adds
// them; many: a block per output, thread t adding chunks t, t + 256, ... and the block
// reducing its threads' sums. Either way the normalised limbs (each < 2^32) of at most 65535
// chunks sum below 2^48 in int64.
constexpr int MERGE_BLOCK_FROM = 32;

__global__ void __launch_bounds__(SUM_THREADS)
sum_merge_threads(const int64_t* __restrict__ part, const int* __restrict__ part_nf, int B,
                  int chunks, uint32_t divisor, float* __restrict__ out) {
    const int b = blockIdx.x * SUM_THREADS + threadIdx.x;
    if (b >= B) return;
    int64_t tot[LIMBS];
#pragma unroll
    for (int l = 0; l < LIMBS; ++l) tot[l] = 0;
    int nf = 0;
    for (int k = 0; k < chunks; ++k) {
#pragma unroll
        for (int l = 0; l < LIMBS; ++l) tot[l] += part[((size_t)k * LIMBS + l) * B + b];
        nf |= part_nf[(size_t)k * B + b];
    }
    out[b] = repro_sum::finalize(tot, 1, divisor, nf);
}

__global__ void __launch_bounds__(SUM_THREADS)
sum_merge(const int64_t* __restrict__ part, const int* __restrict__ part_nf, int B, int chunks,
          uint32_t divisor, float* __restrict__ out) {
    __shared__ int64_t red[LIMBS][SUM_THREADS];
    __shared__ int nf_sh[SUM_THREADS];
    const int b = blockIdx.x, t = threadIdx.x;
    int64_t tot[LIMBS];
#pragma unroll
    for (int l = 0; l < LIMBS; ++l) tot[l] = 0;
    int nf = 0;
    for (int k = t; k < chunks; k += SUM_THREADS) {
#pragma unroll
        for (int l = 0; l < LIMBS; ++l) tot[l] += part[((size_t)k * LIMBS + l) * B + b];
        nf |= part_nf[(size_t)k * B + b];
    }
#pragma unroll
    for (int l = 0; l < LIMBS; ++l) red[l][t] = tot[l];
    nf_sh[t] = nf;
    __syncthreads();
    for (int s = SUM_THREADS / 2; s > 0; s >>= 1) {
        if (t < s) {
#pragma unroll
            for (int l = 0; l < LIMBS; ++l) red[l][t] += red[l][t + s];
            nf_sh[t] |= nf_sh[t + s];
        }
        __syncthreads();
    }
    if (t == 0) {
        int64_t lim[LIMBS];
#pragma unroll
        for (int l = 0; l < LIMBS; ++l) lim[l] = red[l][0];
        out[b] = repro_sum::finalize(lim, 1, divisor, nf_sh[0]);
    }
}

// Non-finite scan (repro_torch/src/kernels.cu:8-20): one vote per wave, one atomic min per
// wave that saw a NaN or infinity. Grid-stride over 16-byte vectors when x is aligned.
__device__ inline bool is_nonfinite(float v) {
    return (repro_gemm::float_to_bits(v) & 0x7F800000u) == 0x7F800000u;
}

__global__ void __launch_bounds__(SUM_THREADS)
scan_nonfinite(const float* __restrict__ x, size_t n, int vec, int* flag, int op_id) {
    const size_t tid = (size_t)blockIdx.x * SUM_THREADS + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * SUM_THREADS;
    bool bad = false;
    size_t tail = 0;
    if (vec) {
        const size_t n4 = n / 4;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        for (size_t i = tid; i < n4; i += stride) {
            const float4 v = x4[i];
            bad = bad || is_nonfinite(v.x) || is_nonfinite(v.y) || is_nonfinite(v.z) ||
                  is_nonfinite(v.w);
        }
        tail = 4 * n4;
    }
    for (size_t i = tail + tid; i < n; i += stride) bad = bad || is_nonfinite(x[i]);
    const unsigned long long votes = __ballot(bad);
    if (votes != 0 && (threadIdx.x & 63) == (unsigned)(__ffsll((long long)votes) - 1))
        atomicMin(flag, op_id);
}

struct SumLayout {
    bool columns;
    int chunks;
    int rows_per_chunk;   // columns kind
    size_t nf_offset, total;
};

int sum_layout(int A, int B, int C, const rg_sum_config* cfg, int num_cus, SumLayout* Lp) {
    if (!cfg || A <= 0 || B <= 0 || C <= 0 || cfg->chunks < 0) return hipErrorInvalidValue;
    if ((long long)A * C > INT_MAX) return hipErrorInvalidValue;
    SumLayout L{};
    L.columns = C == 1;
    const long long count = (long long)A * C;
    const int max_chunks = (int)std::min<long long>(65535, L.columns ? A : count);
    int chunks = cfg->chunks;
    if (chunks == 0) {
        const int target_blocks = 2 * std::max(1, num_cus);
        if (L.columns) {
            const int bx = (B + 63) / 64;
            chunks = (target_blocks + bx - 1) / bx;
            chunks = std::min(chunks, std::max(1, A / 64));     // >= 64 rows per chunk
        } else {
            const long long target_waves = 4LL * target_blocks;      // (output, chunk) items
            chunks = (int)std::min<long long>((target_waves + B - 1) / B, 65535);
            chunks = (int)std::min<long long>(chunks, std::max(1LL, count / 2048));
        }
    }
    chunks = std::max(1, std::min(chunks, max_chunks));
    if (L.columns) {
        L.rows_per_chunk = (A + chunks - 1) / chunks;
        chunks = (A + L.rows_per_chunk - 1) / L.rows_per_chunk;  // no empty chunk
    }
    L.chunks = chunks;
    const size_t slots = chunks > 1 ? (size_t)chunks * B : 0;
    L.nf_offset = align_up(slots * LIMBS * sizeof(int64_t));
    L.total = slots ? L.nf_offset + align_up(slots * sizeof(int)) : 0;
    *Lp = L;
    return hipSuccess;
}

int sum_layout_current(int A, int B, int C, const rg_sum_config* cfg, SumLayout* L) {
    if (!cfg) return hipErrorInvalidValue;
    DeviceInfo dev{false, 1};
    if (cfg->chunks == 0) {
        const int e = query_device(&dev);
        if (e != hipSuccess) return e;
    }
    return sum_layout(A, B, C, cfg, dev.num_cus, L);
}

}  // namespace
}  // namespace rg

extern "C" {

void rg_sum_config_init(rg_sum_config* cfg) {
    if (!cfg) return;
    cfg->chunks = 0;
    cfg->mean = 0;
}

int rg_make_sum_plan(int A, int B, int C, const rg_sum_config* cfg, rg_sum_plan* plan) {
    if (!plan) return hipErrorInvalidValue;
    rg::SumLayout L;
    const int e = rg::sum_layout_current(A, B, C, cfg, &L);
    if (e != hipSuccess) return e;
    plan->chunks = L.chunks;
    plan->workspace_bytes = L.total;
    return hipSuccess;
}

int rg_sum_plan_for_device(int A, int B, int C, const rg_sum_config* cfg, int num_cus,
                           rg_sum_plan* plan) {
    if (!plan) return hipErrorInvalidValue;
    rg::SumLayout L;
    const int e = rg::sum_layout(A, B, C, cfg, num_cus, &L);
    if (e != hipSuccess) return e;
    plan->chunks = L.chunks;
    plan->workspace_bytes = L.total;
    return hipSuccess;
}

int rg_sum_fp32_ws(const float* x, float* out, int A, int B, int C, const rg_sum_config* cfg,
                   void* workspace, size_t workspace_bytes, void* stream_) {
    if (!x || !out) return hipErrorInvalidValue;
    rg::SumLayout L;
    const int e = rg::sum_layout_current(A, B, C, cfg, &L);
    if (e != hipSuccess) return e;
    if (L.total && (!workspace || workspace_bytes < L.total)) return hipErrorInvalidValue;
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    const uint32_t divisor = cfg->mean ? (uint32_t)((long long)A * C) : 1u;
    int64_t* part = L.total ? static_cast<int64_t*>(workspace) : nullptr;
    int* part_nf = L.total ? reinterpret_cast<int*>(static_cast<char*>(workspace) + L.nf_offset)
                           : nullptr;
    if (L.columns) {
        dim3 grid((B + 63) / 64, L.chunks);
        hipLaunchKernelGGL(rg::sum_columns, grid, dim3(rg::SUM_THREADS), 0, stream, x, A, B,
                           L.rows_per_chunk, L.chunks, divisor, out, part, part_nf);
    } else {
        const long long items = (long long)B * L.chunks;
        if ((items + 3) / 4 > INT_MAX) return hipErrorInvalidValue;
        hipLaunchKernelGGL(rg::sum_segments, dim3((unsigned)((items + 3) / 4)), dim3(rg::SUM_THREADS),
                           0, stream, x, A, B, C, L.chunks, divisor, out, part, part_nf);
    }
    if (L.chunks > 1) {
        if (L.chunks < rg::MERGE_BLOCK_FROM)
            hipLaunchKernelGGL(rg::sum_merge_threads, dim3((B + rg::SUM_THREADS - 1) / rg::SUM_THREADS),
                               dim3(rg::SUM_THREADS), 0, stream, part, part_nf, B, L.chunks,
                               divisor, out);
        else
            hipLaunchKernelGGL(rg::sum_merge, dim3((unsigned)B), dim3(rg::SUM_THREADS), 0, stream,
                               part, part_nf, B, L.chunks, divisor, out);
    }
    return hipGetLastError();
}

int rg_sum_fp32(const float* x, float* out, int A, int B, int C, const rg_sum_config* cfg,
                void* stream) {
    rg_sum_plan plan;
    int e = rg_make_sum_plan(A, B, C, cfg, &plan);
    if (e != hipSuccess) return e;
    void* ws = nullptr;
    if (plan.workspace_bytes && (e = hipMalloc(&ws, plan.workspace_bytes)) != hipSuccess) return e;
    e = rg_sum_fp32_ws(x, out, A, B, C, cfg, ws, plan.workspace_bytes, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (ws) (void)hipFree(ws);
    return e;
}

int rg_scan_finite(const float* x, int* flag, size_t n, int op_id, void* stream_) {
    if (n == 0) return hipSuccess;
    if (!x || !flag) return hipErrorInvalidValue;
    const int vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const size_t per_block = (size_t)rg::SUM_THREADS * (vec ? 16 : 4);
    const size_t blocks = std::min<size_t>((n + per_block - 1) / per_block, 4096);
    hipLaunchKernelGGL(rg::scan_nonfinite, dim3((unsigned)blocks), dim3(rg::SUM_THREADS), 0,
                       static_cast<hipStream_t>(stream_), x, n, vec, flag, op_id);
    return hipGetLastError();
}

}  // extern "C"
