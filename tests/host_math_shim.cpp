// Host build of the product's scalar header (include/repro_gemm_math.h), so CPU tests can
// compare its integer formulations with the oracle on every input they choose. The GPU
// tests then compare the device build of the same header with this host build.
#include <cstdint>

#include "repro_gemm_math.h"
#include "rg_fastdiv.h"

extern "C" {

void hm_scale_exponent_n(const float* m, int* e, long long n) {
    for (long long i = 0; i < n; ++i) e[i] = repro_gemm::scale_exponent(m[i]);
}

// Every float with bit pattern in [lo, hi): number whose exponent differs from `want_fn`'s.
long long hm_scale_exponent_count_range(uint32_t lo, uint32_t hi, int (*want_fn)(float)) {
    long long bad = 0;
    for (uint32_t b = lo; b < hi; ++b) {
        float x = repro_gemm::bits_to_float(b);
        if (repro_gemm::scale_exponent(x) != want_fn(x)) ++bad;
    }
    return bad;
}

void hm_fixed_point_n(const float* x, const int* se, int S, int* out, long long n) {
    for (long long i = 0; i < n; ++i) out[i] = repro_gemm::fixed_point(x[i], se[i], S);
}

void hm_round_to_float_n(const int64_t* T, const int* E, float* out, long long n) {
    for (long long i = 0; i < n; ++i) out[i] = repro_gemm::round_to_float(T[i], E[i]);
}

void hm_round_to_float_fast_n(const int64_t* T, const int* E, float* out, long long n) {
    for (long long i = 0; i < n; ++i) out[i] = repro_gemm::round_to_float_fast(T[i], E[i]);
}

void hm_round_to_float_f64_n(const int64_t* T, const int* E, float* out, long long n) {
    for (long long i = 0; i < n; ++i) out[i] = repro_gemm::round_to_float_f64(T[i], E[i]);
}


// Pairs (d[i], n[j]) for which the fast divider of the packing kernels differs from n / d, for
// every i and j; and for one divisor, every n in [n0, n1).
long long hm_fastdiv_mismatches(const uint32_t* d, long long nd, const uint32_t* n, long long nn) {
    long long bad = 0;
    for (long long i = 0; i < nd; ++i) {
        const rg::FastDiv f = rg::make_fastdiv(d[i]);
        for (long long j = 0; j < nn; ++j) bad += rg::fdiv(n[j], f) != n[j] / d[i];
    }
    return bad;
}

long long hm_fastdiv_range(uint32_t d, uint32_t n0, uint32_t n1) {
    const rg::FastDiv f = rg::make_fastdiv(d);
    long long bad = 0;
    for (uint32_t n = n0; n < n1; ++n) bad += rg::fdiv(n, f) != n / d;
    return bad;
}

}  // extern "C"
