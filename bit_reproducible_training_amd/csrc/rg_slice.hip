// Slice-split: FP32 operand -> per-row power-of-two exponent + S int8 digit panels.
//
// Replaces quantize_kmajor / quantize_kstrided / emit (repro_gemm_cuda/repro_gemm.cu:36-121).
// Two bandwidth-bound passes:
//   absmax_*  partial max|x| of every row of op(X) over a chunk of K (one 64-lane
//             wavefront per row chunk, or per 64 columns for column access), reduced
//             across the wavefront with lane shuffles;
//   slice     one wavefront per (32-row panel, 32-k panel): reduces the partial maxima
//             of its rows, computes scale_exponent, rounds 16 elements per lane with
//             fixed_point and writes S int8 digits per element straight into the MFMA
//             operand panel (1 KiB contiguous per digit and wavefront).
// Max is exact and order-free, so the chunking never changes a bit.
#include "rg_internal.h"
#include "repro_gemm_math.h"

namespace rg {

using repro_gemm::fixed_point;
using repro_gemm::scale_exponent;

__device__ __forceinline__ float wave_max(float m) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    return m;
}

// Row access: element (r, k) at src[r*K + k]. Wavefront w handles row w / nch, chunk w % nch.
__global__ void __launch_bounds__(256) absmax_rows(const float* __restrict__ src, int R, int K,
                                                   int nch, int kch, int Rp,
                                                   float* __restrict__ pmax) {
    const int lane = threadIdx.x & 63;
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= (long long)R * nch) return;
    const int r = (int)(w / nch), c = (int)(w % nch);
    const int k0 = c * kch;
    const int k1 = min(K, k0 + kch);
    const float* row = src + (size_t)r * K;
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    int k = k0 + lane;
    for (; k + 192 < k1; k += 256) {
        m0 = fmaxf(m0, fabsf(row[k]));
        m1 = fmaxf(m1, fabsf(row[k + 64]));
        m2 = fmaxf(m2, fabsf(row[k + 128]));
        m3 = fmaxf(m3, fabsf(row[k + 192]));
    }
    for (; k < k1; k += 64) m0 = fmaxf(m0, fabsf(row[k]));
    float m = wave_max(fmaxf(fmaxf(m0, m1), fmaxf(m2, m3)));
    if (lane == 0) pmax[(size_t)c * Rp + r] = m;
}

// Column access: element (r, k) at src[k*R + r]. Wavefront w handles 64 consecutive
// columns (one per lane) of chunk w % nch.
__global__ void __launch_bounds__(256) absmax_cols(const float* __restrict__ src, int R, int K,
                                                   int nch, int kch, int Rp,
                                                   float* __restrict__ pmax) {
    const int lane = threadIdx.x & 63;
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const long long groups = (R + 63) / 64;
    if (w >= groups * nch) return;
    const int g = (int)(w / nch), c = (int)(w % nch);
    const int r = g * 64 + lane;
    if (r >= R) return;
    const int k0 = c * kch;
    const int k1 = min(K, k0 + kch);
    const float* col = src + r;
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    int k = k0;
    for (; k + 3 < k1; k += 4) {
        m0 = fmaxf(m0, fabsf(col[(size_t)k * R]));
        m1 = fmaxf(m1, fabsf(col[(size_t)(k + 1) * R]));
        m2 = fmaxf(m2, fabsf(col[(size_t)(k + 2) * R]));
        m3 = fmaxf(m3, fabsf(col[(size_t)(k + 3) * R]));
    }
    for (; k < k1; ++k) m0 = fmaxf(m0, fabsf(col[(size_t)k * R]));
    pmax[(size_t)c * Rp + r] = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
}

// Balanced base-128 digits of X, most significant first: X = sum_p d[p] * 128^(S-1-p),
// |d[0]| <= 127, d[p] in [-64, 63] for p > 0. Exact integer operations only.
template <int S>
__device__ __forceinline__ void split_digits(int X, int (&d)[S]) {
#pragma unroll
    for (int p = S - 1; p >= 1; --p) {
        int t = ((X + 64) & 127) - 64;
        d[p] = t;
        X = (X - t) >> 7;  // X - t is a multiple of 128
    }
    d[0] = X;
}

// One wavefront per (row panel rp, k panel kp). Lane l owns row rp*32 + l%32 and
// k = kp*32 + 16*(l/32) + j, j = 0..15.
template <int S, bool STRIDED, bool INT32_OUT>
__global__ void __launch_bounds__(256) slice_kernel(const float* __restrict__ src, int R, int K,
                                                    int Rp, int Kp, const float* __restrict__ pmax,
                                                    int nch, void* __restrict__ out,
                                                    int* __restrict__ expo, int vec_ok) {
    const int lane = threadIdx.x & 63;
    const int npk = Kp / PANEL_K;
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= (long long)(Rp / PANEL_ROWS) * npk) return;
    const int rp = (int)(w / npk), kp = (int)(w % npk);
    const int r = rp * PANEL_ROWS + (lane & 31);
    const int h = lane >> 5;

    float m = 0.0f;
    if (r < R)
        for (int c = 0; c < nch; ++c) m = fmaxf(m, pmax[(size_t)c * Rp + r]);
    const int se = scale_exponent(m);
    if (kp == 0 && h == 0) expo[r] = se;

    const int k0 = kp * PANEL_K + 16 * h;
    float x[16];
    if (r < R) {
        if (STRIDED) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                x[j] = (k0 + j < K) ? src[(size_t)(k0 + j) * R + r] : 0.0f;
        } else if (vec_ok && k0 + 16 <= K) {
            const float4* p = reinterpret_cast<const float4*>(src + (size_t)r * K + k0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 v = p[q];
                x[4 * q + 0] = v.x;
                x[4 * q + 1] = v.y;
                x[4 * q + 2] = v.z;
                x[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) x[j] = (k0 + j < K) ? src[(size_t)r * K + k0 + j] : 0.0f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] = 0.0f;
    }

    if (INT32_OUT) {
        int4* o = reinterpret_cast<int4*>(static_cast<int32_t*>(out) + (size_t)r * Kp + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = make_int4(fixed_point(x[4 * q], se, S), fixed_point(x[4 * q + 1], se, S),
                             fixed_point(x[4 * q + 2], se, S), fixed_point(x[4 * q + 3], se, S));
    } else {
        uint32_t word[S][4];
#pragma unroll
        for (int p = 0; p < S; ++p)
#pragma unroll
            for (int q = 0; q < 4; ++q) word[p][q] = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int d[S];
            split_digits<S>(fixed_point(x[j], se, S), d);
#pragma unroll
            for (int p = 0; p < S; ++p) word[p][j >> 2] |= ((uint32_t)d[p] & 0xFFu) << (8 * (j & 3));
        }
        uint4* o = reinterpret_cast<uint4*>(static_cast<int8_t*>(out)) +
                   ((size_t)(rp * npk + kp) * S) * (PANEL_BYTES / 16) + lane;
#pragma unroll
        for (int p = 0; p < S; ++p)
            o[(size_t)p * (PANEL_BYTES / 16)] = make_uint4(word[p][0], word[p][1], word[p][2], word[p][3]);
    }
}

void launch_absmax(const float* src, int R, int K, bool strided, int nch, int kch, int Rp,
                   float* pmax, hipStream_t stream) {
    long long waves = strided ? (long long)((R + 63) / 64) * nch : (long long)R * nch;
    unsigned blocks = (unsigned)((waves + 3) / 4);
    if (strided)
        absmax_cols<<<blocks, 256, 0, stream>>>(src, R, K, nch, kch, Rp, pmax);
    else
        absmax_rows<<<blocks, 256, 0, stream>>>(src, R, K, nch, kch, Rp, pmax);
}

template <int S, bool I32>
static void launch_slice_s(const float* src, int R, int K, int Rp, int Kp, bool strided,
                           const float* pmax, int nch, void* out, int* expo, hipStream_t stream) {
    long long waves = (long long)(Rp / PANEL_ROWS) * (Kp / PANEL_K);
    unsigned blocks = (unsigned)((waves + 3) / 4);
    int vec_ok = (K % 4 == 0) && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
    if (strided)
        slice_kernel<S, true, I32><<<blocks, 256, 0, stream>>>(src, R, K, Rp, Kp, pmax, nch, out, expo, vec_ok);
    else
        slice_kernel<S, false, I32><<<blocks, 256, 0, stream>>>(src, R, K, Rp, Kp, pmax, nch, out, expo, vec_ok);
}

void launch_slice(const float* src, int R, int K, int Rp, int Kp, bool strided, const float* pmax,
                  int nch, int S, bool int32_out, void* out, int* expo, hipStream_t stream) {
    switch (S * 2 + (int32_out ? 1 : 0)) {
        case 2: launch_slice_s<1, false>(src, R, K, Rp, Kp, strided, pmax, nch, out, expo, stream); break;
        case 3: launch_slice_s<1, true>(src, R, K, Rp, Kp, strided, pmax, nch, out, expo, stream); break;
        case 4: launch_slice_s<2, false>(src, R, K, Rp, Kp, strided, pmax, nch, out, expo, stream); break;
        case 5: launch_slice_s<2, true>(src, R, K, Rp, Kp, strided, pmax, nch, out, expo, stream); break;
        case 6: launch_slice_s<3, false>(src, R, K, Rp, Kp, strided, pmax, nch, out, expo, stream); break;
        case 7: launch_slice_s<3, true>(src, R, K, Rp, Kp, strided, pmax, nch, out, expo, stream); break;
        default: break;
    }
}

}  // namespace rg
