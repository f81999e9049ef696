#pragma once
// repro_sum_math.h -- host/device scalar arithmetic of the exact float32 sum (namespace
// repro_sum; the names LIMBS, split_float, acc_add, normalize and finalize are those of
// repro_sum_cuda/repro_sum_math.cuh, so callers of that header compile against this one).
//
// Representation: the sum is an integer count of the smallest subnormal, 2^-149. A float32
// below 2^128 is a whole number of those units below 2^277, and the int64 limbs below hold it
// in radix 2^32 (limb l weighs 2^(32 l - 149)); with LIMBS = 10 there is room for the carries
// of 2^31 - 1 summands. Limbs are signed and may run ahead of their radix between
// normalisations, so the additions can be done in any order, split and merged freely: the
// value is a plain integer sum.
//
// Rounding (finalize): the integer, or the integer divided by a count for a mean, is rounded
// to float32 once, nearest-even. Conventions: a zero result is +0.0; a nonzero result that
// rounds to zero keeps its sign; a result beyond the float32 range is an infinity of its sign;
// any NaN or infinity among the summands makes the result NaN.
#include <cstdint>

#include "repro_gemm_math.h"

namespace repro_sum {

constexpr int LIMBS = 10;

// Finite x as (idx, v, negative) with |x| = v * 2^(32 idx - 149), idx in 0..7 and
// v = significand << (biased exponent - 1 mod 32) < 2^55. Returns false for NaN/Inf.
RG_HD inline bool wide_term(float x, int& idx, uint64_t& v, bool& negative) {
    const uint32_t b = repro_gemm::float_to_bits(x);
    const uint32_t e = (b >> 23) & 0xFFu;
    if (e == 0xFFu) return false;
    const uint32_t f = b & 0x7FFFFFu;
    const uint32_t sig = e ? (f | 0x800000u) : f;
    const int sh = e ? (int)e - 1 : 0;          // |x| = sig * 2^(sh - 149)
    idx = sh >> 5;
    v = (uint64_t)sig << (sh & 31);
    negative = (b >> 31) != 0;
    return true;
}

// repro_sum_math.cuh:66-82: x = (lo * 2^(32 idx) + hi * 2^(32 (idx + 1))) * 2^-149 with
// |lo| < 2^32 and |hi| < 2^23. Returns false for NaN/Inf (addends zero, idx 0).
RG_HD inline bool split_float(float x, int& idx, int64_t& lo, int64_t& hi) {
    uint64_t v;
    bool neg;
    if (!wide_term(x, idx, v, neg)) {
        idx = 0;
        lo = hi = 0;
        return false;
    }
    lo = (int64_t)(v & 0xFFFFFFFFull);
    hi = (int64_t)(v >> 32);
    if (neg) {
        lo = -lo;
        hi = -hi;
    }
    return true;
}

// repro_sum_math.cuh:84-91: adds x to an accumulator whose limb l is acc[l * stride];
// sets nonfinite for NaN/Inf.
RG_HD inline void acc_add(int64_t* acc, int stride, float x, int& nonfinite) {
    int idx;
    int64_t lo, hi;
    if (!split_float(x, idx, lo, hi)) {
        nonfinite = 1;
        return;
    }
    acc[idx * stride] += lo;
    acc[(idx + 1) * stride] += hi;
}

// Carry propagation (repro_sum_math.cuh:93-100): afterwards limbs 0..LIMBS-2 lie in
// [0, 2^32) and the top limb carries the sign. The value is unchanged.
RG_HD inline void normalize(int64_t* t) {
    for (int l = 0; l + 1 < LIMBS; ++l) {
        const int64_t carry = t[l] >> 32;       // floor(t / 2^32)
        t[l] -= carry * ((int64_t)1 << 32);
        t[l + 1] += carry;
    }
}

// Exact value of the accumulator divided by `divisor` (1 <= divisor < 2^31), rounded once
// to float32 nearest-even (repro_sum_math.cuh:102-157 states the same result).
//
// The magnitude is extended by two fractional radix-2^32 digits and divided exactly, so
// the quotient q = floor(|value| * 2^64 / divisor) carries at least 33 bits whenever the
// value is nonzero. The 62 bits below q's leading bit, with every lower bit and the
// division remainder folded into the last one (a sticky bit), are rounded by
// repro_gemm::round_to_float, which then sees the same rounding decision as the full
// quotient.
RG_HD inline float finalize(const int64_t* acc, int stride, uint32_t divisor, int nonfinite) {
    if (nonfinite) return repro_gemm::bits_to_float(0x7FC00000u);
    int64_t t[LIMBS];
    for (int l = 0; l < LIMBS; ++l) t[l] = acc[l * stride];
    normalize(t);
    const bool neg = t[LIMBS - 1] < 0;
    if (neg) {
        for (int l = 0; l < LIMBS; ++l) t[l] = -t[l];
        normalize(t);
    }
    constexpr int D = LIMBS + 2;                // digits of |value| * 2^64
    uint32_t q[D];
    uint64_t rem = 0;
    for (int i = D - 1; i >= 0; --i) {
        const uint64_t digit = i >= 2 ? (uint64_t)(uint32_t)t[i - 2] : 0u;
        const uint64_t cur = (rem << 32) | digit;   // < divisor * 2^32 <= 2^63
        q[i] = (uint32_t)(cur / divisor);
        rem = cur % divisor;
    }
    int top = D - 1;
    while (top >= 0 && q[top] == 0) --top;
    if (top < 0) return 0.0f;                   // the exact value is zero
    const int lead = 32 * top + 31 - __builtin_clz(q[top]);
    const int low = lead > 61 ? lead - 61 : 0;  // lowest bit kept in the 62-bit window
    const int d = low >> 5, s = low & 31;
    const uint64_t w0 = (uint64_t)q[d] | ((d + 1 < D ? (uint64_t)q[d + 1] : 0u) << 32);
    const uint64_t w1 = d + 2 < D ? (uint64_t)q[d + 2] : 0u;
    uint64_t T = (w0 >> s) | (s ? w1 << (64 - s) : 0u);
    T &= (lead - low + 1 >= 64) ? ~0ull : ((1ull << (lead - low + 1)) - 1);
    bool sticky = rem != 0;
    for (int i = 0; i < d; ++i) sticky = sticky || q[i] != 0;
    if (s) sticky = sticky || (q[d] & ((1u << s) - 1u)) != 0;
    if (sticky) T |= 1u;
    const int64_t signed_T = neg ? -(int64_t)T : (int64_t)T;
    return repro_gemm::round_to_float(signed_T, low - 149 - 64);
}

}  // namespace repro_sum
