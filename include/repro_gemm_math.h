#pragma once
// Scalar arithmetic that defines the reproducible GEMM's output, callable from host
// and device code. Replaces repro_gemm_cuda/repro_gemm_math.cuh:20-121 (same namespace
// and names, so repro_conv_math.cuh:20-26 and repro_conv_cpu.h:63 can use it).
//
// Every function is either exact or performs one IEEE rounding with a fixed mode.
// fixed_point and round_to_float are written with integer operations only, so their
// results do not depend on the floating-point environment (denormal flushing, FMA
// contraction) of the compiler or the GPU. scale_exponent needs one correctly rounded
// binary32 division; HIP's default (-fhip-fp32-correctly-rounded-divide-sqrt) and any
// IEEE host compiler provide it. round_to_float_f64, the faster equivalent of round_to_float
// used by the GPU epilogues, relies on exact binary64 arithmetic and one IEEE conversion to
// binary32. Do not build with -ffast-math or denormal flushing.
#include <cmath>
#include <cstdint>
#include <cstring>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define RG_HD __host__ __device__
#else
#define RG_HD
// Host-only builds of code written for both sides (repro_conv_math.cuh marks its functions
// __host__ __device__) see the qualifiers as nothing, as under the reference's header.
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif

namespace repro_gemm {

// Slices S per operand element: S int8 digits give a 7*S-bit fixed-point value.
constexpr int MAX_SLICES = 3;

RG_HD inline uint32_t float_to_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
RG_HD inline float bits_to_float(uint32_t b) { return __builtin_bit_cast(float, b); }

RG_HD inline int clz64(uint64_t x) { return __builtin_clzll(x); }

// x * 2^n for |n| <= 252 as two multiplications by normal powers of two
// (repro_gemm_math.cuh:44-55). Exact unless the result is subnormal, where it rounds once.
RG_HD inline float scale_by_pow2(float x, int n) {
    int n1 = n >> 1, n2 = n - n1;
    float p1 = bits_to_float((uint32_t)(n1 + 127) << 23);
    float p2 = bits_to_float((uint32_t)(n2 + 127) << 23);
    return (x * p1) * p2;
}

// Exponent e of the row/column scale 2^e: the smallest power of two >= fl32(m / 127),
// or 0 when m is not positive or m / 127 rounds to zero (repro_gemm_math.cuh:57-69).
RG_HD inline int scale_exponent(float m) {
    if (!(m > 0.0f)) return 0;
    uint32_t b = float_to_bits(m / 127.0f);
    uint32_t E = (b >> 23) & 0xFFu, f = b & 0x7FFFFFu;
    if (E != 0) return f == 0 ? (int)E - 127 : (int)E - 126;
    if (f == 0) return 0;                       // quotient underflowed to zero
    int pf = 31 - __builtin_clz(f);             // subnormal quotient f * 2^-149
    return (f & (f - 1)) == 0 ? pf - 149 : pf - 148;
}

// Bits of |x|, ordered like the values for every non-NaN float, and 0 for a NaN: the largest
// key of a row is the bit pattern of the maximum the reference takes with std::fmax, which
// skips NaN (repro_gemm_cpu.h:30-31, 36-37).
RG_HD inline uint32_t magnitude_key(float x) {
    const uint32_t a = float_to_bits(x) & 0x7FFFFFFFu;
    return a > 0x7F800000u ? 0u : a;
}

// X = round-to-nearest-even(x * 2^(7(S-1) - se)), clamped to |X| <= 127 * 2^(7(S-1))
// (repro_gemm_math.cuh:71-83), computed on the integer significand of x.
// A NaN or infinite x gives -127 * 2^(7(S-1)). The definition is meant for finite inputs (the
// reference's hash tool refuses others), but its CPU path still computes one: it converts
// with (int)nearbyintf, which gives INT_MIN for a NaN or an infinity on x86, and then clamps.
// Every path here gives that value, so the CPU and the GPU agree bit for bit on such inputs too.
RG_HD inline int fixed_point(float x, int se, int S) {
    uint32_t b = float_to_bits(x);
    uint32_t be = (b >> 23) & 0xFFu, fr = b & 0x7FFFFFu;
    int64_t lim = (int64_t)127 << (7 * (S - 1));
    if (be == 0xFFu) return (int)-lim;
    uint64_t mant = be ? (uint64_t)(fr | 0x800000u) : (uint64_t)fr;  // |x| = mant * 2^e2
    int e2 = be ? (int)be - 150 : -149;
    int up = e2 + 7 * (S - 1) - se;             // |x| * 2^(7(S-1)-se) = mant * 2^up
    int64_t q;
    if (mant == 0) {
        q = 0;
    } else if (up >= 0) {
        q = up > 40 ? lim + 1 : (int64_t)(mant << up);
    } else if (up <= -25) {
        q = 0;                                  // mant * 2^up < 1/2
    } else {
        int sh = -up;
        uint64_t t = mant >> sh, rem = mant & ((1ull << sh) - 1), half = 1ull << (sh - 1);
        if (rem > half || (rem == half && (t & 1))) ++t;
        q = (int64_t)t;
    }
    if (q > lim) q = lim;
    return (int)((b >> 31) ? -q : q);
}

// Correctly rounded (nearest-even) binary32 value of T * 2^E, including subnormal
// results, -0.0 for negative T that rounds to zero, and overflow to infinity
// (repro_gemm_math.cuh:93-119). The float is assembled from its bit fields.
RG_HD inline float round_to_float(int64_t T, int E) {
    if (T == 0) return 0.0f;
    uint32_t sign = T < 0 ? 0x80000000u : 0u;
    uint64_t m = T < 0 ? (uint64_t)0 - (uint64_t)T : (uint64_t)T;
    int p = 63 - clz64(m);                      // leading bit of T * 2^E at 2^(p+E)
    // Bits of m to drop: enough to leave a binary32 significand (p - 23), or more when the
    // result lies in the subnormal range, whose last bit has the weight 2^-149.
    int shift = p - 23;
    if (-149 - E > shift) shift = -149 - E;
    uint64_t q;
    int ex;
    if (shift <= 0) {
        q = m;
        ex = E;
    } else if (shift >= 64) {
        return bits_to_float(sign);
    } else {
        q = m >> shift;
        uint64_t rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        ex = E + shift;
    }
    if (q == 0) return bits_to_float(sign);
    int pq = 63 - clz64(q);                     // q <= 2^24, ex >= -149
    int top = ex + pq;
    if (top > 127) return bits_to_float(sign | 0x7F800000u);
    if (top >= -126) {
        uint64_t mant = pq >= 23 ? q >> (pq - 23) : q << (23 - pq);
        return bits_to_float(sign | ((uint32_t)(top + 127) << 23) | ((uint32_t)mant & 0x7FFFFFu));
    }
    return bits_to_float(sign | (uint32_t)(q << (ex + 149)));
}

// round_to_float(T, E) for the common case of a GEMM epilogue, without branches: when the
// result's exponent before rounding is a normal one (*normal = true), q = the 24 leading bits
// of |T| rounded to nearest-even and the float's bits are ((biased exponent - 1) << 23) + q,
// where a rounding carry (q == 2^24) moves into the exponent field by itself and a carry out of
// the largest binade gives exactly +-inf. Otherwise (zero, subnormal or out-of-range results)
// *normal = false and the returned value is meaningless: use round_to_float.
RG_HD inline float round_to_float_normal(int64_t T, int E, bool* normal) {
    const uint64_t neg = (uint64_t)(T >> 63);           // all ones when T < 0
    const uint64_t m = ((uint64_t)T ^ neg) - neg;       // |T|
    const int p = 63 - clz64(m | 1);                    // leading bit of |T|
    const int e = p + E + 127;                          // biased exponent before rounding
    *normal = m != 0 && e >= 1 && e <= 254;
    const int sh = p - 23;                              // bits below the 24-bit significand
    const int down = sh > 0 ? sh : 0, up = sh < 0 ? -sh : 0;
    const uint64_t top = m >> down;
    const uint64_t rem = m & ((1ull << down) - 1);      // 0 when nothing is dropped
    const uint64_t half = (1ull << down) >> 1;          // 0 when nothing is dropped
    const uint32_t carry = (uint32_t)(down > 0) & (uint32_t)((rem > half) | ((rem == half) & (top & 1)));
    const uint32_t q = ((uint32_t)top << up) + carry;
    return bits_to_float((((uint32_t)(e - 1) << 23) + q) | ((uint32_t)neg & 0x80000000u));
}

// The same value as round_to_float(T, E) for every input; branch-free in the common case.
RG_HD inline float round_to_float_fast(int64_t T, int E) {
    bool normal;
    const float r = round_to_float_normal(T, E, &normal);
    return normal ? r : round_to_float(T, E);
}

// Exponents E for which T * 2^E is exact in binary64 for every |T| <= 2^53: no overflow
// (2^53 * 2^E < 2^1024) and no underflow below the smallest normal (2^E >= 2^-1022).
RG_HD inline bool f64_scale_exact(int E) { return (uint32_t)(E + 1022) <= 1022u + 970u; }

// round_to_float(T, E) through binary64 when |T| <= 2^53: T is exact in a double (its two
// 32-bit halves are, and hi * 2^32 + lo is representable, so the fused multiply-add does not
// round), the scaling by 2^E is exact for f64_scale_exact(E), and the conversion to binary32
// is the one rounding: nearest-even, with subnormal results, -0.0 for negative T that rounds
// to zero and overflow to infinity, all by IEEE 754. Needs binary32 denormals (no flushing)
// and the default rounding mode. Other inputs take round_to_float.
// round_to_float_f64_try gives that value and *ok = true when -2^53 <= T < 2^53 and
// f64_scale_exact(E); otherwise *ok = false and the returned value is meaningless.
RG_HD inline float round_to_float_f64_try(int64_t T, int E, bool* ok) {
    const int32_t hi = (int32_t)(T >> 32);
    *ok = (uint32_t)(hi + (1 << 21)) < (1u << 22) && f64_scale_exact(E);
    const double d = __builtin_fma((double)hi, 4294967296.0, (double)(uint32_t)T);
    return (float)__builtin_ldexp(d, E);
}

RG_HD inline float round_to_float_f64(int64_t T, int E) {
    bool ok;
    const float r = round_to_float_f64_try(T, E, &ok);
    return ok ? r : round_to_float(T, E);
}

}  // namespace repro_gemm
