// C-linkage entry points over the reference's own CPU implementation, compiled from the
// reference headers where they lie (-I <reference>/repro_gemm_cuda); nothing is copied.
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin oracle/repro_oracle.c against the
// reference itself, and by bench.py's cpu_baseline leg as the timed CPU path.
#include <cstdint>

#include "repro_gemm_cpu.h"  // repro_gemm_cuda/repro_gemm_cpu.h:25-51 (includes the math header)

extern "C" {

int ref_scale_exponent(float m) { return repro_gemm::scale_exponent(m); }

int ref_fixed_point(float x, int se, int S) { return repro_gemm::fixed_point(x, se, S); }

float ref_round_to_float(int64_t T, int E) { return repro_gemm::round_to_float(T, E); }

// repro_gemm::cpu_gemm; thread count from $REPRO_CPU_THREADS or hardware_concurrency().
void ref_cpu_gemm(const float* A, const float* B, float* C, int M, int N, int K, int ta, int tb,
                  int S) {
    repro_gemm::cpu_gemm(A, B, C, M, N, K, ta != 0, tb != 0, S);
}

}  // extern "C"
