// Host build of the product's exact-sum header (include/repro_sum_math.h), so CPU tests can
// compare it with the oracle, and replay the GPU kernels' accumulation schedule (wide terms,
// carry resolution every `flush` adds, lanes merged by limb addition) on the CPU.
#include <cstddef>
#include <cstdint>
#include <vector>

#include "repro_sum_math.h"

extern "C" {

// out[b] = finalize of the plain two-addend accumulator over x[a][b][c].
void hs_exact_sum(const float* x, float* out, int A, int B, int C, int mean) {
    const uint32_t divisor = mean ? (uint32_t)((int64_t)A * C) : 1u;
    for (int b = 0; b < B; ++b) {
        int64_t acc[repro_sum::LIMBS] = {};
        int nf = 0;
        for (int a = 0; a < A; ++a)
            for (int c = 0; c < C; ++c) repro_sum::acc_add(acc, 1, x[((size_t)a * B + b) * C + c], nf);
        out[b] = repro_sum::finalize(acc, 1, divisor, nf);
    }
}

// The GPU schedule for one output: the n summands v[order[i]] are dealt to `lanes` lanes in
// turn; each lane adds wide terms to its limbs and resolves carries after every `flush` adds
// (as the kernels do after at most 252); the lanes' normalised limbs are summed in `groups`
// partial sums (chunks) which are summed again before one finalize.
float hs_wide_schedule(const float* v, const int* order, int n, int lanes, int flush, int groups,
                       uint32_t divisor) {
    using repro_sum::LIMBS;
    std::vector<int64_t> acc((size_t)lanes * LIMBS, 0);
    std::vector<int> since(lanes, 0), nf(lanes, 0);
    auto carry = [&](int64_t* p) {
        int64_t c = 0;
        for (int l = 0; l < LIMBS; ++l) {
            int64_t t = p[l] + c;
            if (l + 1 < LIMBS) {
                c = t >> 32;
                t -= c * ((int64_t)1 << 32);
            }
            p[l] = t;
        }
    };
    for (int i = 0; i < n; ++i) {
        const int lane = i % lanes;
        int idx;
        uint64_t w;
        bool neg;
        if (!repro_sum::wide_term(v[order[i]], idx, w, neg)) {
            nf[lane] = 1;
            continue;
        }
        acc[(size_t)lane * LIMBS + idx] += neg ? -(int64_t)w : (int64_t)w;
        if (++since[lane] == flush) {
            carry(&acc[(size_t)lane * LIMBS]);
            since[lane] = 0;
        }
    }
    std::vector<int64_t> part((size_t)groups * LIMBS, 0);
    int any = 0;
    for (int lane = 0; lane < lanes; ++lane) {
        carry(&acc[(size_t)lane * LIMBS]);
        for (int l = 0; l < LIMBS; ++l) part[(size_t)(lane % groups) * LIMBS + l] += acc[(size_t)lane * LIMBS + l];
        any |= nf[lane];
    }
    int64_t tot[LIMBS] = {};
    for (int g = groups - 1; g >= 0; --g)
        for (int l = 0; l < LIMBS; ++l) tot[l] += part[(size_t)g * LIMBS + l];
    return repro_sum::finalize(tot, 1, divisor, any);
}

}  // extern "C"
