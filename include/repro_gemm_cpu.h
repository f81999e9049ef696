#pragma once
// repro_gemm_cpu.h -- the reproducible FP32 GEMM on the host CPU. Header-only C++17 with
// std::thread; needs no GPU and no HIP runtime. Its output is bit-identical to the GPU library
// (librepro_gemm.so) for every input, because both compute the same exact integer sums from
// the scalar definition in repro_gemm_math.h and round them once.
//
// Replaces repro_gemm_cuda/repro_gemm_cpu.h:14-51 for its callers (the PyTorch binding's CPU
// branch, repro_torch/src/bindings.cpp:7,40,64; gpt2_ops_suite.cu:17): same namespace,
// names, signatures and results.
//
//   cpu_thread_count()   workers used by cpu_for: $REPRO_CPU_THREADS when it is a positive
//                        integer, else std::thread::hardware_concurrency() (at least 1).
//   cpu_for(n, f)        calls f(i) exactly once for every i in [0, n), spread over the
//                        workers; returns when all calls have returned. Results never depend
//                        on the worker count, only on what f(i) writes.
//   cpu_gemm(A, B, C, M, N, K, ta, tb, S)
//                        C[M][N] = op(A) op(B), all row-major: A is MxK (KxM when ta), B is
//                        KxN (NxK when tb). Throws std::invalid_argument for a null pointer,
//                        a size <= 0, S outside 1..MAX_SLICES, or K beyond the exact-int64
//                        bound K * d^2 <= 2^62 (d = the largest digit-split value, as the GPU
//                        planner checks).
//
// The computation, in three passes over the data:
//   1. op(A) row r: e_r = scale_exponent(max_k |op(A)[r][k]|), X[r][k] = fixed_point(., e_r, S);
//      op(B) column c: f_c and Y[c][k] likewise (the operand is read once per pass, along its
//      rows in memory, whichever way it is transposed).
//   2. T[r][c] = sum_k X[r][k] * Y[c][k] in int64 -- exact, so the order of k, the blocking
//      and the threading cannot change it.
//   3. C[r][c] = round_to_float(T[r][c], e_r + f_c - 14 (S - 1)).
// Inputs are meant to be finite. For a NaN or an infinity the maxima skip NaN and fixed_point
// gives -127 * 2^(7(S-1)), as the reference's CPU path does on x86; the GPU path gives the same
// bits.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <thread>
#include <vector>

#include "repro_gemm_math.h"

namespace repro_gemm {

inline int cpu_thread_count() {
    if (const char* env = std::getenv("REPRO_CPU_THREADS")) {
        char* end = nullptr;
        const long v = std::strtol(env, &end, 10);
        if (end != env && *end == '\0' && v > 0 && v <= 4096) return (int)v;
    }
    const unsigned hw = std::thread::hardware_concurrency();
    return hw > 0 ? (int)hw : 1;
}

// Work is handed out in runs of consecutive indices from one atomic cursor, about eight runs
// per worker, so uneven items still balance; the calling thread is one of the workers.
template <class F>
void cpu_for(int n, F f) {
    if (n <= 0) return;
    const int workers = std::min(cpu_thread_count(), n);
    if (workers == 1) {
        for (int i = 0; i < n; ++i) f(i);
        return;
    }
    const int run = std::max(1, n / (8 * workers));
    std::atomic<int> cursor{0};
    auto drain = [&]() {
        for (;;) {
            const int first = cursor.fetch_add(run, std::memory_order_relaxed);
            if (first >= n) return;
            const int last = std::min(n, first + run);
            for (int i = first; i < last; ++i) f(i);
        }
    };
    std::vector<std::thread> helpers;
    helpers.reserve((size_t)workers - 1);
    for (int t = 1; t < workers; ++t) helpers.emplace_back(drain);
    drain();
    for (auto& h : helpers) h.join();
}

namespace cpu_detail {

// Largest |X| of the digit split (127 * 128^(S-1) plus the balanced lower digits' 64s),
// the bound the GPU planner applies to K.
inline double largest_fixed_point(int S) {
    double d = 127.0 * std::ldexp(1.0, 7 * (S - 1));
    for (int t = 0; t + 1 < S; ++t) d += 64.0 * std::ldexp(1.0, 7 * t);
    return d;
}

// Fixed-point rows of an operand: R rows of K values, row r element k at
// src[r * K + k] (row access) or src[k * R + r] (column access). Writes q[r * K + k] and
// e[r]. Magnitudes are compared as magnitude_key(x) (the bits of |x|, NaN skipped), which is
// the maximum the definition asks for.
inline void fixed_point_rows(const float* src, int R, int K, bool column_access, int S,
                             int32_t* q, int* e) {
    if (!column_access) {
        cpu_for(R, [&](int r) {
            const float* row = src + (size_t)r * K;
            uint32_t top = 0;
            for (int k = 0; k < K; ++k) top = std::max(top, magnitude_key(row[k]));
            const int ex = scale_exponent(bits_to_float(top));
            e[r] = ex;
            int32_t* out = q + (size_t)r * K;
            for (int k = 0; k < K; ++k) out[k] = fixed_point(row[k], ex, S);
        });
        return;
    }
    // Column access: blocks of 64 columns, each walked k by k over contiguous 256-byte runs.
    constexpr int CB = 64;
    const int blocks = (R + CB - 1) / CB;
    cpu_for(blocks, [&](int blk) {
        const int r0 = blk * CB, r1 = std::min(R, r0 + CB);
        uint32_t top[CB] = {};
        for (int k = 0; k < K; ++k) {
            const float* line = src + (size_t)k * R;
            for (int r = r0; r < r1; ++r)
                top[r - r0] = std::max(top[r - r0], magnitude_key(line[r]));
        }
        int ex[CB];
        for (int r = r0; r < r1; ++r) e[r] = ex[r - r0] = scale_exponent(bits_to_float(top[r - r0]));
        for (int k = 0; k < K; ++k) {
            const float* line = src + (size_t)k * R;
            for (int r = r0; r < r1; ++r) q[(size_t)r * K + k] = fixed_point(line[r], ex[r - r0], S);
        }
    });
}

// T for a 4x4 block of outputs: 16 independent int64 chains over k (rows past the matrix
// repeat the last one; their results are not stored).
inline void dot_4x4(const int32_t* const* x, const int32_t* const* y, int K, int64_t (*t)[4]) {
    int64_t s[4][4] = {};
    for (int k = 0; k < K; ++k) {
        const int64_t a0 = x[0][k], a1 = x[1][k], a2 = x[2][k], a3 = x[3][k];
        const int64_t b0 = y[0][k], b1 = y[1][k], b2 = y[2][k], b3 = y[3][k];
        s[0][0] += a0 * b0; s[0][1] += a0 * b1; s[0][2] += a0 * b2; s[0][3] += a0 * b3;
        s[1][0] += a1 * b0; s[1][1] += a1 * b1; s[1][2] += a1 * b2; s[1][3] += a1 * b3;
        s[2][0] += a2 * b0; s[2][1] += a2 * b1; s[2][2] += a2 * b2; s[2][3] += a2 * b3;
        s[3][0] += a3 * b0; s[3][1] += a3 * b1; s[3][2] += a3 * b2; s[3][3] += a3 * b3;
    }
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) t[i][j] = s[i][j];
}

}  // namespace cpu_detail

inline void cpu_gemm(const float* A, const float* B, float* C, int M, int N, int K, bool ta,
                     bool tb, int S) {
    if (!A || !B || !C) throw std::invalid_argument("cpu_gemm: null matrix");
    if (M <= 0 || N <= 0 || K <= 0) throw std::invalid_argument("cpu_gemm: sizes must be positive");
    if (S < 1 || S > MAX_SLICES) throw std::invalid_argument("cpu_gemm: slices must be 1..3");
    const double d = cpu_detail::largest_fixed_point(S);
    if ((double)K * d * d > std::ldexp(1.0, 62))
        throw std::invalid_argument("cpu_gemm: K too large for exact int64 sums at this S");

    std::vector<int32_t> X((size_t)M * K), Y((size_t)N * K);
    std::vector<int> ex(M), ey(N);
    // op(A) rows are A's rows unless ta; op(B) columns are B's rows only when tb.
    cpu_detail::fixed_point_rows(A, M, K, ta, S, X.data(), ex.data());
    cpu_detail::fixed_point_rows(B, N, K, !tb, S, Y.data(), ey.data());

    // Tiles of 16 rows x 64 columns; inside a tile, 4x4 blocks of outputs share each loaded
    // row of X and Y four times.
    constexpr int TR = 16, TC = 64;
    const int tiles_r = (M + TR - 1) / TR, tiles_c = (N + TC - 1) / TC;
    const int e0 = -14 * (S - 1);
    cpu_for(tiles_r * tiles_c, [&](int tile) {
        const int r0 = (tile / tiles_c) * TR, c0 = (tile % tiles_c) * TC;
        const int r1 = std::min(M, r0 + TR), c1 = std::min(N, c0 + TC);
        for (int r = r0; r < r1; r += 4) {
            const int32_t* xr[4];
            for (int i = 0; i < 4; ++i) xr[i] = X.data() + (size_t)std::min(r + i, r1 - 1) * K;
            for (int c = c0; c < c1; c += 4) {
                const int32_t* yc[4];
                for (int j = 0; j < 4; ++j) yc[j] = Y.data() + (size_t)std::min(c + j, c1 - 1) * K;
                int64_t t[4][4];
                cpu_detail::dot_4x4(xr, yc, K, t);
                for (int i = 0; i < 4 && r + i < r1; ++i)
                    for (int j = 0; j < 4 && c + j < c1; ++j)
                        C[(size_t)(r + i) * N + c + j] = round_to_float(t[i][j], ex[r + i] + ey[c + j] + e0);
            }
        }
    });
}

}  // namespace repro_gemm
