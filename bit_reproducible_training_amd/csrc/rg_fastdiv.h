#pragma once
// Division of integers in [0, 2^31) by a divisor fixed before a launch, as a multiply-high,
// an add and a shift: the round-up multiplier of Granlund and Montgomery ("Division by
// invariant integers using multiplication", PLDI 1994, section 4). With l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1 (below 2^32 for every d >= 1),
//     n / d = (mulhi32(n, m) + n) >> l      for 0 <= n < 2^31,
// where the sum stays below 2^32. Used for the index arithmetic of the convolution's packing
// kernels, whose tensors hold fewer than 2^31 elements.
#include <cstdint>

#include "repro_gemm_math.h"  // RG_HD

namespace rg {

struct FastDiv {
    uint32_t d, m;
    int l;
};

inline FastDiv make_fastdiv(uint32_t d) {  // d >= 1
    int l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = (((1ull << 32) * ((1ull << l) - d)) / d) + 1;
    return FastDiv{d, (uint32_t)m, l};
}

RG_HD inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
    const uint32_t t = (uint32_t)(((uint64_t)n * f.m) >> 32);
    return (t + n) >> f.l;
}

}  // namespace rg
