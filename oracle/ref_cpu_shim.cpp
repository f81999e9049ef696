// C-linkage entry points over the reference's own CPU implementation, compiled from the
// reference headers where they lie (-I <reference>/repro_gemm_cuda, repro_sum_cuda,
// repro_conv_cuda); nothing is copied.
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin oracle/repro_oracle.c against the
// reference itself, and by bench.py's cpu_baseline leg as the timed CPU path.
#include <cstdint>

#include "repro_gemm_cpu.h"  // repro_gemm_cuda/repro_gemm_cpu.h:25-51 (includes the math header)
#include "repro_sum_math.cuh"  // repro_sum_cuda/repro_sum_math.cuh (header-only superaccumulator)
#include "repro_conv_cpu.h"    // repro_conv_cuda/repro_conv_cpu.h (header-only CPU convolution)

namespace {
repro_conv::ConvShape conv_shape(const int* s) {
    repro_conv::ConvShape g;
    g.N = s[0]; g.C = s[1]; g.H = s[2]; g.W = s[3]; g.F = s[4]; g.KH = s[5]; g.KW = s[6];
    g.SY = s[7]; g.SX = s[8]; g.PY = s[9]; g.PX = s[10];
    return g;
}
}  // namespace

extern "C" {

int ref_scale_exponent(float m) { return repro_gemm::scale_exponent(m); }

int ref_fixed_point(float x, int se, int S) { return repro_gemm::fixed_point(x, se, S); }

float ref_round_to_float(int64_t T, int E) { return repro_gemm::round_to_float(T, E); }

// repro_gemm::cpu_gemm; thread count from $REPRO_CPU_THREADS or hardware_concurrency().
void ref_cpu_gemm(const float* A, const float* B, float* C, int M, int N, int K, int ta, int tb,
                  int S) {
    repro_gemm::cpu_gemm(A, B, C, M, N, K, ta != 0, tb != 0, S);
}

// The CPU branch of repro_torch/src/bindings.cpp:69-91 (exact_sum), single-threaded, on the
// reference's own accumulator functions.
void ref_exact_sum(const float* x, float* out, int A, int B, int C, int mean) {
    const uint32_t divisor = mean ? (uint32_t)((int64_t)A * C) : 1u;
    for (int b = 0; b < B; ++b) {
        int64_t acc[repro_sum::LIMBS] = {};
        int nf = 0;
        for (int a = 0; a < A; ++a)
            for (int c = 0; c < C; ++c) repro_sum::acc_add(acc, 1, x[((size_t)a * B + b) * C + c], nf);
        out[b] = repro_sum::finalize(acc, 1, divisor, nf);
    }
}

// repro_conv::cpu_conv2d, cpu_conv2d_grad_weight, cpu_conv2d_grad_input; s holds
// N, C, H, W, F, KH, KW, SY, SX, PY, PX.
void ref_conv2d(const float* x, const float* w, float* out, const int* s, int S) {
    repro_conv::cpu_conv2d(x, w, out, conv_shape(s), S);
}
void ref_conv2d_grad_weight(const float* dy, const float* x, float* dw, const int* s, int S) {
    repro_conv::cpu_conv2d_grad_weight(dy, x, dw, conv_shape(s), S);
}
void ref_conv2d_grad_input(const float* dy, const float* w, float* dx, const int* s, int S) {
    repro_conv::cpu_conv2d_grad_input(dy, w, dx, conv_shape(s), S);
}

}  // extern "C"
