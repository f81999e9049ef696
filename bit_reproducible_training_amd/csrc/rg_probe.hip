// Diagnostic: the sustained int8 MFMA rate of the current device, with operands held in
// registers and no memory traffic in the loop. The random-byte and [0, 127]-byte figures are
// practical ceilings for the contraction kernels under the device's power limit (the lower
// digit planes are bytes in [0, 127]); zero operands show how far data-dependent power lets
// the clock rise.
#include <hip/hip_runtime.h>

#include <cstring>

#include "repro_gemm.h"

namespace rg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int PROBE_ACC = 8;   // independent accumulators per wavefront
constexpr int PROBE_WORDS = 4096;

__global__ void __launch_bounds__(256) mfma_probe(const v4i* __restrict__ in, int* __restrict__ out, int iters) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    const v4i a0 = in[(t * 4 + 0) % PROBE_WORDS], a1 = in[(t * 4 + 1) % PROBE_WORDS];
    const v4i b0 = in[(t * 4 + 2) % PROBE_WORDS], b1 = in[(t * 4 + 3) % PROBE_WORDS];
    v16i acc[PROBE_ACC];
#pragma unroll
    for (int i = 0; i < PROBE_ACC; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < PROBE_ACC; ++i)
            acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8((i & 1) ? a1 : a0, (i & 2) ? b1 : b0, acc[i], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < PROBE_ACC; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[i][e];
    out[t] = s;
}

}  // namespace
}  // namespace rg

extern "C" int rg_measure_mfma_int8_rate(int dense, double* tops) {
    if (!tops || dense < 0 || dense > 2) return hipErrorInvalidValue;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, dev)) != hipSuccess) return e;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return hipErrorNotSupported;

    const int blocks = 2 * cus;  // two wavefronts per SIMD
    const int iters = 4000;
    rg::v4i host[rg::PROBE_WORDS];
    unsigned long long x = 0x9E3779B97F4A7C15ull;
    for (int i = 0; i < rg::PROBE_WORDS; ++i)
        for (int j = 0; j < 4; ++j) {
            x = x * 6364136223846793005ull + 1442695040888963407ull;
            const uint32_t bytes = (uint32_t)(x >> 32);
            // 1: random bytes; 2: random bytes in [0, 127] (like the lower digit planes); 0: zeros
            host[i][j] = dense == 0 ? 0 : (int)(dense == 2 ? bytes & 0x7F7F7F7Fu : bytes);
        }
    rg::v4i* din = nullptr;
    int* dout = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float best = 0.0f;
    if ((e = hipMalloc(&din, sizeof host)) != hipSuccess) goto done;
    if ((e = hipMalloc(&dout, sizeof(int) * 256 * blocks)) != hipSuccess) goto done;
    if ((e = hipStreamCreate(&st)) != hipSuccess) goto done;
    if ((e = hipEventCreate(&e0)) != hipSuccess) goto done;
    if ((e = hipEventCreate(&e1)) != hipSuccess) goto done;
    if ((e = hipMemcpyAsync(din, host, sizeof host, hipMemcpyHostToDevice, st)) != hipSuccess) goto done;
    for (int rep = 0; rep < 3; ++rep) {
        (void)hipEventRecord(e0, st);
        rg::mfma_probe<<<blocks, 256, 0, st>>>(din, dout, iters);
        (void)hipEventRecord(e1, st);
        if ((e = hipEventSynchronize(e1)) != hipSuccess) goto done;
        float ms = 0.0f;
        if ((e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess) goto done;
        if (rep > 0 && (best == 0.0f || ms < best)) best = ms;
    }
    {
        const double ops = 2.0 * 32 * 32 * 32 * rg::PROBE_ACC * (double)iters * blocks * 4;
        *tops = ops / (best * 1e-3) / 1e12;
    }
    e = hipGetLastError();
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    if (din) (void)hipFree(din);
    if (dout) (void)hipFree(dout);
    return e;
}
