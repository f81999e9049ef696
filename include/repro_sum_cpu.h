#pragma once
// repro_sum_cpu.h -- the exact, order-independent float32 sum on the host CPU (header-only
// C++17; no GPU needed), bit-identical to rg_sum_fp32_ws (include/repro_sum.h) for every
// input. It is the CPU branch of the PyTorch binding's exact_sum
// (repro_torch/src/bindings.cpp:69-91, which inlines the same loop over repro_sum::acc_add).
//
//   cpu_sum(x, out, A, B, C, mean)   x viewed as row-major [A][B][C]; for every b,
//       out[b] = the exact sum over a, c of x[a][b][c] (divided exactly by A*C when mean),
//       rounded once to float32 by repro_sum::finalize. Throws std::invalid_argument for a
//       null pointer, a size <= 0 or A*C > 2^31 - 1 (the GPU path's limits).
//
// Each output owns a LIMBS-limb accumulator (repro_sum_math.h). A summand |x| = v * 2^(32 idx
// - 149) with v < 2^55 (wide_term) is added to limb idx as one signed 64-bit term; carries are
// resolved every 252 additions, before any limb can reach 2^63 (2^32 + 252 * 2^55 < 2^63).
// Integer addition is exact, so the grouping over threads and the summation order cannot change
// a bit.
#include <cstdint>
#include <stdexcept>

#include "repro_gemm_cpu.h"
#include "repro_sum_math.h"

namespace repro_sum {

namespace cpu_detail {

struct WideAccumulator {
    int64_t limb[LIMBS] = {};
    int pending = 0;
    int nonfinite = 0;

    void add(float x) {
        int idx;
        uint64_t v;
        bool negative;
        if (!wide_term(x, idx, v, negative)) {
            nonfinite = 1;
            return;
        }
        limb[idx] += negative ? -(int64_t)v : (int64_t)v;
        if (++pending == 252) {
            normalize(limb);
            pending = 0;
        }
    }
};

}  // namespace cpu_detail

inline void cpu_sum(const float* x, float* out, int A, int B, int C, bool mean) {
    if (!x || !out) throw std::invalid_argument("cpu_sum: null pointer");
    if (A <= 0 || B <= 0 || C <= 0) throw std::invalid_argument("cpu_sum: sizes must be positive");
    if ((int64_t)A * C > 2147483647LL) throw std::invalid_argument("cpu_sum: A*C must be below 2^31");
    const uint32_t divisor = mean ? (uint32_t)((int64_t)A * C) : 1u;
    repro_gemm::cpu_for(B, [&](int b) {
        cpu_detail::WideAccumulator acc;
        for (int a = 0; a < A; ++a) {
            const float* run = x + ((size_t)a * B + b) * C;
            for (int c = 0; c < C; ++c) acc.add(run[c]);
        }
        out[b] = finalize(acc.limb, 1, divisor, acc.nonfinite);
    });
}

}  // namespace repro_sum
