// C entry points over the product's CPU headers (include/repro_gemm_cpu.h, repro_sum_cpu.h,
// repro_conv_cpu.h), compiled by the tests with g++ alone: no torch, no HIP runtime. Shows
// that the headers stand on their own and lets ctypes compare them with the oracle.
#include <atomic>
#include <stdexcept>

#include "repro_conv_cpu.h"
#include "repro_gemm_cpu.h"
#include "repro_sum_cpu.h"

extern "C" {

int ch_threads() { return repro_gemm::cpu_thread_count(); }

// visits[i] counts the calls cpu_for made for index i.
void ch_for_visits(int n, int* visits) {
    std::atomic<int>* v = reinterpret_cast<std::atomic<int>*>(visits);
    repro_gemm::cpu_for(n, [&](int i) { v[i].fetch_add(1, std::memory_order_relaxed); });
}

int ch_gemm(const float* A, const float* B, float* C, int M, int N, int K, int ta, int tb, int S) {
    try {
        repro_gemm::cpu_gemm(A, B, C, M, N, K, ta != 0, tb != 0, S);
        return 0;
    } catch (const std::invalid_argument&) {
        return 1;
    }
}

int ch_sum(const float* x, float* out, int A, int B, int C, int mean) {
    try {
        repro_sum::cpu_sum(x, out, A, B, C, mean != 0);
        return 0;
    } catch (const std::invalid_argument&) {
        return 1;
    }
}

// kind 0 forward (a = x, b = w), 1 weight gradient (a = dy, b = x), 2 input gradient
// (a = dy, b = w); s = N, C, H, W, F, KH, KW, SY, SX, PY, PX.
int ch_conv(int kind, const float* a, const float* b, float* out, const int* s, int S) {
    repro_conv::ConvShape g;
    g.N = s[0]; g.C = s[1]; g.H = s[2]; g.W = s[3]; g.F = s[4]; g.KH = s[5]; g.KW = s[6];
    g.SY = s[7]; g.SX = s[8]; g.PY = s[9]; g.PX = s[10];
    try {
        if (kind == 0) repro_conv::cpu_conv2d(a, b, out, g, S);
        else if (kind == 1) repro_conv::cpu_conv2d_grad_weight(a, b, out, g, S);
        else repro_conv::cpu_conv2d_grad_input(a, b, out, g, S);
        return 0;
    } catch (const std::invalid_argument&) {
        return 1;
    }
}

}  // extern "C"
