// Slice-split: FP32 operand -> per-row power-of-two exponent + S int8 digit panels.
//
// Replaces quantize_kmajor / quantize_kstrided / emit (repro_gemm_cuda/repro_gemm.cu:36-121).
// Both operands are handled by the same two launches (blocks [0, nA) work on op(A), the
// rest on op(B)):
//   absmax_kernel  partial max|x| of every row of op(X) over chunks of K. Row access: one
//                  64-lane wavefront per (row, chunk), float4 loads, reduced with lane
//                  shuffles. Column access: a block covers 256 columns (float4 per lane)
//                  or 64 (scalar), its 4 wavefronts split the chunk's k, reduced in LDS;
//                  an operand of at most 32 columns has each wavefront read whole rows.
//   split_kernel   a block owns one 32-row panel and 4*G consecutive 32-k panels: it
//                  reduces the rows' partial maxima once (in LDS), computes scale_exponent,
//                  and each wavefront rounds 16 elements per lane per panel to the
//                  fixed-point integer of the definition and writes its S int8 digits
//                  straight into the MFMA operand panel (1 KiB per digit and wavefront).
// Max is exact and order-free, so the chunking never changes a bit.
#include "rg_internal.h"
#include "repro_gemm_math.h"

namespace rg {

using repro_gemm::scale_exponent;

constexpr int SPLIT_G = 4;  // k panels per wavefront in split_kernel


__device__ __forceinline__ float max4(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Largest magnitude bits of v: for non-NaN values the bits of max4(v); a NaN wins.
__device__ __forceinline__ unsigned max4_bits(float4 v) {
    const unsigned a = __float_as_uint(v.x) & 0x7FFFFFFFu, b = __float_as_uint(v.y) & 0x7FFFFFFFu;
    const unsigned c = __float_as_uint(v.z) & 0x7FFFFFFFu, e = __float_as_uint(v.w) & 0x7FFFFFFFu;
    return max(max(a, b), max(c, e));
}

// The four values q[k .. k+3] of a row of K values, zero past either end of the row. q + k is
// 16-byte aligned (callers choose k so); the vector load is taken only where all four values lie
// inside the row, otherwise the values inside are read one by one.
__device__ __forceinline__ float4 load4_in_row(const float* q, int k, int K) {
    if (k >= 0 && k + 3 < K) return *reinterpret_cast<const float4*>(q + k);
    float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (k >= 0 && k < K) t.x = q[k];
    if (k + 1 >= 0 && k + 1 < K) t.y = q[k + 1];
    if (k + 2 >= 0 && k + 2 < K) t.z = q[k + 2];
    if (k + 3 >= 0 && k + 3 < K) t.w = q[k + 3];
    return t;
}

// Row access where rows are not 16-byte aligned (K or ld not a multiple of 4, or an unaligned
// base): v[i] = q[kb + 32i + 4g .. +3] (g = lane % 8, the lane's place among the eight lanes of
// its row; kb a multiple of 32), zero at k >= K, read by whole aligned 16-byte loads instead of
// four scalar loads per lane. Each lane loads the aligned vector that holds its first value
// (starting o values earlier, o = the row's misalignment in floats) and takes the values it
// lacks from the aligned vector of the next lane of its row, which for g = 7 is lane g = 0's
// vector of the next k panel (lane g = 0 loads one vector past the last panel for it). Every
// lane of the wavefront must call this (the exchange is a cross-lane read); a lane whose row
// is dead (live false) reads nothing and gets zeros. Used by the one read of row-access operands
// (8192x768x50257 NN, A's 8192 rows of 50257 values: slicing 889 -> 759 us against four scalar
// loads per lane).
template <int NF>
__device__ __forceinline__ void load_row_realigned(const float* q, int K, int kb, int lane, bool live,
                                                   float4 (&v)[NF]) {
    const int g = lane & 7;
    const int o = live ? (int)((reinterpret_cast<uintptr_t>(q) >> 2) & 3) : 0;
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < NF; ++i) v[i] = live ? load4_in_row(q, kb + 32 * i + 4 * g - o, K) : zero;
    const float4 tail = live && g == 0 ? load4_in_row(q, kb + 32 * NF - o, K) : zero;
    const int src = (lane & ~7) | ((g + 1) & 7);
#pragma unroll
    for (int i = 0; i < NF; ++i) {
        // what this lane hands to the lane before it (g = 0: to g = 7, from the next panel);
        // v[i + 1] is still the aligned vector here, v[i] is replaced below
        const float4 give = g == 0 ? (i + 1 < NF ? v[i + 1] : tail) : v[i];
        const float n0 = __shfl(give.x, src, 64), n1 = __shfl(give.y, src, 64);
        const float n2 = __shfl(give.z, src, 64);
        const float4 a = v[i];
        v[i] = o == 0 ? a
             : o == 1 ? make_float4(a.y, a.z, a.w, n0)
             : o == 2 ? make_float4(a.z, a.w, n0, n1)
                      : make_float4(a.w, n0, n1, n2);
    }
}

// Exponent of stacked row q from its maximum m (which skips NaN), or 0 where d.nanrows flags
// the row.
__device__ __forceinline__ int row_exponent(const SliceDesc& d, size_t q, float m) {
    return d.nanrows && d.nanrows[q] ? 0 : scale_exponent(m);
}

// Row access, element (r, k) of item b at src[b*bstride + r*ld + k]: wavefront w of the
// operand handles row w / nch of all items' rows (item-major), chunk w % nch.
// (row, chunk) pairs per wavefront in the row-access maxima: a lane per pair for short
// chunks (a wavefront per pair would leave most lanes idle); for 16-byte rows with chunks of
// at most 128 values, 16 or 32 lanes per pair (one float4 each per step); else the whole
// wavefront.
__host__ __device__ inline int rows_per_wave(const SliceDesc& d) {
    if (d.kch <= 32) return 64;
    if (d.vec && d.kch <= 64) return 4;
    if (d.vec && d.kch <= 128) return 2;
    return 1;
}

template <int WAVES>
__device__ void absmax_rows(const SliceDesc& d, long long blk) {
    const int lane = threadIdx.x & 63;
    if (rows_per_wave(d) == 64) {
        const long long pair = (blk * WAVES + (threadIdx.x >> 6)) * 64 + lane;
        if (pair >= (long long)d.batch * d.R * d.nch) return;
        const long long i = pair / d.nch;
        const int c = (int)(pair - i * d.nch);
        const int b = (int)(i / d.R), r = (int)(i - (long long)b * d.R);
        const int k0 = c * d.kch, k1 = min(d.K, k0 + d.kch);
        const float* row = d.src + (size_t)b * d.bstride + (size_t)r * d.ld;
        float m = 0.0f;
        for (int k = k0; k < k1; ++k) m = fmaxf(m, fabsf(row[k]));
        d.pmax[(size_t)c * d.batch * d.Rp + (size_t)b * d.Rp + r] = m;
        return;
    }
    if (rows_per_wave(d) > 1) {  // vec: lpr lanes per pair, float4 loads, shuffle reduction
        const int rpw = rows_per_wave(d), lpr = 64 / rpw;
        const long long pair = (blk * WAVES + (threadIdx.x >> 6)) * rpw + lane / lpr;
        const bool live = pair < (long long)d.batch * d.R * d.nch;
        float m = 0.0f;
        long long i = 0;
        int c = 0, b = 0, r = 0;
        if (live) {
            i = pair / d.nch;
            c = (int)(pair - i * d.nch);
            b = (int)(i / d.R);
            r = (int)(i - (long long)b * d.R);
            const float4* p =
                reinterpret_cast<const float4*>(d.src + (size_t)b * d.bstride + (size_t)r * d.ld);
            const int q1 = min(d.K, c * d.kch + d.kch) / 4;
            for (int q = c * d.kch / 4 + lane % lpr; q < q1; q += lpr) m = fmaxf(m, max4(p[q]));
        }
        for (int o = 1; o < lpr; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (live && lane % lpr == 0) d.pmax[(size_t)c * d.batch * d.Rp + (size_t)b * d.Rp + r] = m;
        return;
    }
    const long long w = blk * WAVES + (threadIdx.x >> 6);
    if (w >= (long long)d.batch * d.R * d.nch) return;
    const long long i = w / d.nch;
    const int c = (int)(w - i * d.nch);
    const int b = (int)(i / d.R), r = (int)(i - (long long)b * d.R);
    const int k0 = c * d.kch;
    const int k1 = min(d.K, k0 + d.kch);
    const float* row = d.src + (size_t)b * d.bstride + (size_t)r * d.ld;
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    int k = k0;
    if (d.vec) {  // K % 4 == 0 and 16-byte aligned rows (src, ld, bstride); kch % 4 == 0
        const float4* p = reinterpret_cast<const float4*>(row);
        int q = k0 / 4 + lane;
        const int q1 = k1 / 4;
        for (; q + 192 < q1; q += 256) {
            m0 = fmaxf(m0, max4(p[q]));
            m1 = fmaxf(m1, max4(p[q + 64]));
            m2 = fmaxf(m2, max4(p[q + 128]));
            m3 = fmaxf(m3, max4(p[q + 192]));
        }
        for (; q < q1; q += 64) m0 = fmaxf(m0, max4(p[q]));
    } else {  // unaligned rows: 16 scalar loads in flight per lane (4 KiB per wavefront)
        for (k = k0 + lane; k + 960 < k1; k += 1024) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = fabsf(row[k + 64 * j]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                m0 = fmaxf(m0, v[4 * j]);
                m1 = fmaxf(m1, v[4 * j + 1]);
                m2 = fmaxf(m2, v[4 * j + 2]);
                m3 = fmaxf(m3, v[4 * j + 3]);
            }
        }
        for (; k + 192 < k1; k += 256) {
            m0 = fmaxf(m0, fabsf(row[k]));
            m1 = fmaxf(m1, fabsf(row[k + 64]));
            m2 = fmaxf(m2, fabsf(row[k + 128]));
            m3 = fmaxf(m3, fabsf(row[k + 192]));
        }
        for (; k < k1; k += 64) m0 = fmaxf(m0, fabsf(row[k]));
    }
    float m = wave_max(fmaxf(fmaxf(m0, m1), fmaxf(m2, m3)));
    if (lane == 0) d.pmax[(size_t)c * d.batch * d.Rp + (size_t)b * d.Rp + r] = m;
}

// Column access, element (r, k) of item b at src[b*bstride + k*ld + r]: block (b, g, c)
// covers cols columns of item b, chunk c; its WAVES wavefronts take every WAVES-th k of the
// chunk and combine in LDS.
template <int WAVES>
__device__ void absmax_cols(const SliceDesc& d, long long blk) {
    __shared__ float4 part[WAVES][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int cols = d.vec ? 256 : 64;
    const long long groups = (d.R + cols - 1) / cols;
    long long gi;
    int c;
    if (!d.vec && d.R > 32) {
        // Unaligned rows: a group's 256-byte run of a k-row shares its end lines with the
        // neighbouring groups. Block blk runs on XCD blk % 8 (max_blocks is a multiple of 8
        // here); each XCD takes a contiguous range of (chunk, group) in group order, so
        // neighbouring groups of one chunk run together on one XCD and fetch those lines once.
        const long long lin = (blk & 7) * (d.max_blocks / 8) + (blk >> 3);
        const long long ng = (long long)d.batch * groups;
        if (lin >= ng * d.nch) return;
        c = (int)(lin / ng);
        gi = lin - (long long)c * ng;
    } else {
        if (blk >= (long long)d.batch * groups * d.nch) return;
        gi = blk / d.nch;
        c = (int)(blk - gi * d.nch);
    }
    const int b = (int)(gi / groups), g = (int)(gi - (long long)b * groups);
    const float* item = d.src + (size_t)b * d.bstride;
    const int k0 = c * d.kch;
    const int k1 = min(d.K, k0 + d.kch);
    float4 m = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (d.vec) {  // R, ld % 4 == 0 and 16-byte aligned: lane owns columns 4*lane .. 4*lane+3
        const int r = g * 256 + 4 * lane;
        if (r < d.R) {
            const float* base = item + r;
            int k = k0 + wv;
            for (; k + 3 * WAVES < k1; k += 4 * WAVES) {
                float4 a = *reinterpret_cast<const float4*>(base + (size_t)k * d.ld);
                float4 b = *reinterpret_cast<const float4*>(base + (size_t)(k + WAVES) * d.ld);
                float4 e = *reinterpret_cast<const float4*>(base + (size_t)(k + 2 * WAVES) * d.ld);
                float4 f = *reinterpret_cast<const float4*>(base + (size_t)(k + 3 * WAVES) * d.ld);
                m.x = fmaxf(m.x, fmaxf(fmaxf(fabsf(a.x), fabsf(b.x)), fmaxf(fabsf(e.x), fabsf(f.x))));
                m.y = fmaxf(m.y, fmaxf(fmaxf(fabsf(a.y), fabsf(b.y)), fmaxf(fabsf(e.y), fabsf(f.y))));
                m.z = fmaxf(m.z, fmaxf(fmaxf(fabsf(a.z), fabsf(b.z)), fmaxf(fabsf(e.z), fabsf(f.z))));
                m.w = fmaxf(m.w, fmaxf(fmaxf(fabsf(a.w), fabsf(b.w)), fmaxf(fabsf(e.w), fabsf(f.w))));
            }
            for (; k < k1; k += WAVES) {
                float4 a = *reinterpret_cast<const float4*>(base + (size_t)k * d.ld);
                m.x = fmaxf(m.x, fabsf(a.x));
                m.y = fmaxf(m.y, fabsf(a.y));
                m.z = fmaxf(m.z, fabsf(a.z));
                m.w = fmaxf(m.w, fabsf(a.w));
            }
        }
    } else if (d.R <= 32) {
        // Narrow operand (one group): lane L covers column L % cpr of row L / cpr of a strip of
        // 64 / cpr consecutive k (cpr: R rounded up to a power of two), so one load
        // instruction reads whole rows rather than R scalars of one row.
        int cpr = 1;
        while (cpr < d.R) cpr <<= 1;
        const int rpw = 64 / cpr, col = lane & (cpr - 1);
        const int step = WAVES * rpw;
        if (col < d.R) {
            const float* base = item + col;
            int k = k0 + wv * rpw + lane / cpr;
            for (; k + 7 * step < k1; k += 8 * step) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = fabsf(base[(size_t)(k + i * step) * d.ld]);
                m.x = fmaxf(m.x, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
                m.y = fmaxf(m.y, fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
            }
            for (; k < k1; k += step) m.x = fmaxf(m.x, fabsf(base[(size_t)k * d.ld]));
            m.x = fmaxf(m.x, m.y);
        }
        // Lanes of one column differ in the bits at and above cpr.
        for (int off = cpr; off < 64; off <<= 1) m.x = fmaxf(m.x, __shfl_xor(m.x, off));
    } else {
        const int r = g * 64 + lane;
        if (r < d.R) {
            const float* base = item + r;
            int k = k0 + wv;
            for (; k + 3 * WAVES < k1; k += 4 * WAVES) {
                m.x = fmaxf(m.x, fabsf(base[(size_t)k * d.ld]));
                m.y = fmaxf(m.y, fabsf(base[(size_t)(k + WAVES) * d.ld]));
                m.z = fmaxf(m.z, fabsf(base[(size_t)(k + 2 * WAVES) * d.ld]));
                m.w = fmaxf(m.w, fabsf(base[(size_t)(k + 3 * WAVES) * d.ld]));
            }
            for (; k < k1; k += WAVES) m.x = fmaxf(m.x, fabsf(base[(size_t)k * d.ld]));
            m.x = fmaxf(fmaxf(m.x, m.y), fmaxf(m.z, m.w));
        }
    }
    part[wv][lane] = m;
    __syncthreads();
    if (wv == 0) {
        float4 t = part[0][lane];
#pragma unroll
        for (int i = 1; i < WAVES; ++i) {
            float4 u = part[i][lane];
            t.x = fmaxf(t.x, u.x);
            t.y = fmaxf(t.y, u.y);
            t.z = fmaxf(t.z, u.z);
            t.w = fmaxf(t.w, u.w);
        }
        float* out = d.pmax + (size_t)c * d.batch * d.Rp + (size_t)b * d.Rp;
        if (d.vec) {
            const int r = g * 256 + 4 * lane;
            if (r < d.R) *reinterpret_cast<float4*>(out + r) = t;  // Rp % 32 == 0: in range
        } else {
            const int r = g * 64 + lane;
            if (r < d.R) out[r] = t.x;
        }
    }
}

__global__ void __launch_bounds__(256) absmax_kernel(SliceDesc a, SliceDesc b) {
    const long long blk = blockIdx.x;
    if (blk < a.max_blocks) {
        if (a.strided) absmax_cols<4>(a, blk); else absmax_rows<4>(a, blk);
    } else {
        if (b.strided) absmax_cols<4>(b, blk - a.max_blocks); else absmax_rows<4>(b, blk - a.max_blocks);
    }
}

// Rounds 16 values and writes them: S digit planes of 16 bytes (base 128, most significant
// first, digits_of: X = sum_p d_p 128^(S-1-p), |d_0| <= 127, d_p in [0, 127] for p > 0), or
// 16 int32 fixed-point values for INT32_OUT.
template <int S, bool INT32_OUT>
__device__ __forceinline__ void emit_panel(const SliceDesc& d, const float (&x)[16], const RowScale& rs,
                                           int rp, int kp, int q, int h, int lane) {
    int X[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) X[j] = round_fixed(x[j], rs);
    if (INT32_OUT) {
        int4* o = reinterpret_cast<int4*>(static_cast<int32_t*>(d.out) + (size_t)q * d.Kp + kp * PANEL_K + 16 * h);
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = make_int4(X[4 * q], X[4 * q + 1], X[4 * q + 2], X[4 * q + 3]);
        return;
    }
    int dg[S][16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        int d[S];
        digits_of<S>(X[j], d);
#pragma unroll
        for (int p = 0; p < S; ++p) dg[p][j] = d[p];
    }
    const int npk = d.Kp / PANEL_K;
    uint4* o = reinterpret_cast<uint4*>(d.out) + ((size_t)rp * npk + kp) * S * (PANEL_BYTES / 16) + lane;
#pragma unroll
    for (int p = 0; p < S; ++p)
        o[(size_t)p * (PANEL_BYTES / 16)] =
            make_uint4(pack4(dg[p][0], dg[p][1], dg[p][2], dg[p][3]), pack4(dg[p][4], dg[p][5], dg[p][6], dg[p][7]),
                       pack4(dg[p][8], dg[p][9], dg[p][10], dg[p][11]), pack4(dg[p][12], dg[p][13], dg[p][14], dg[p][15]));
}

// The 16 values of lane (half h) of panel kp in the row whose element k = 0 is at rowp (null
// for a padding row); zero outside the matrix.
__device__ __forceinline__ void load_panel(const SliceDesc& d, int kp, const float* rowp, int h,
                                           bool checked, float (&x)[16]) {
    const int k0 = kp * PANEL_K + 16 * h;
    if (rowp == nullptr) {
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] = 0.0f;
        return;
    }
    if (d.strided) {
        const float* p = rowp + (size_t)k0 * d.ld;
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] = (!checked || k0 + j < d.K) ? p[(size_t)j * d.ld] : 0.0f;
    } else if (d.vec && (!checked || k0 + 16 <= d.K)) {
        const float4* p = reinterpret_cast<const float4*>(rowp + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float4 v = p[q];
            x[4 * q + 0] = v.x;
            x[4 * q + 1] = v.y;
            x[4 * q + 2] = v.z;
            x[4 * q + 3] = v.w;
        }
    } else {
        const float* p = rowp + k0;
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] = (!checked || k0 + j < d.K) ? p[j] : 0.0f;
    }
}

// Row access, one wavefront's SPLIT_G panels (32 rows x 32*SPLIT_G k) read through LDS: a
// lane of the panel layout needs 16 consecutive k of one row, and loading that directly makes
// every load instruction touch 32 rows 16 bytes at a time. Here instruction i loads whole
// 512-byte row segments instead (lane L: row 2i + L/32, float4 L%32), the wavefront writes them
// to its padded LDS tile and reads back in the panel layout. The row pitch of 132 floats puts
// the 8 rows a ds_read_b128 phase reads in distinct banks.
constexpr int STAGE_PITCH = 32 * SPLIT_G + 4;

__device__ __forceinline__ void load_panels_staged(const SliceDesc& d, float* tile, int item, int r0,
                                                   int kpb, int lane, float (&x)[SPLIT_G][16]) {
    const int c4 = lane & 31;
    float4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = 2 * i + (lane >> 5);
        v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r0 + row < d.R)
            v[i] = *reinterpret_cast<const float4*>(d.src + (size_t)item * d.bstride +
                                                    (size_t)(r0 + row) * d.ld + kpb * PANEL_K + 4 * c4);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
        *reinterpret_cast<float4*>(tile + (2 * i + (lane >> 5)) * STAGE_PITCH + 4 * c4) = v[i];
    // The tile is this wavefront's alone: order its LDS writes before the reads of other lanes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float* src = tile + (lane & 31) * STAGE_PITCH + 16 * (lane >> 5);
#pragma unroll
    for (int g = 0; g < SPLIT_G; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 t = *reinterpret_cast<const float4*>(src + g * PANEL_K + 4 * q);
            x[g][4 * q + 0] = t.x;
            x[g][4 * q + 1] = t.y;
            x[g][4 * q + 2] = t.z;
            x[g][4 * q + 3] = t.w;
        }
}

// The same staging for rows that are not 16-byte aligned (or K % 4 != 0): instruction i loads
// 128 contiguous bytes of each of 2 rows (lane L: row 2(i/4) + L/32, k = 32(i%4) + L%32), 64
// scalar loads per lane in all, written to the tile one value at a time.
__device__ __forceinline__ void load_panels_staged_scalar(const SliceDesc& d, float* tile, int item, int r0,
                                                          int kpb, int lane, float (&x)[SPLIT_G][16]) {
    const int kl = lane & 31;
    float v[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        const int row = 2 * (i >> 2) + (lane >> 5);
        v[i] = 0.0f;
        if (r0 + row < d.R)
            v[i] = d.src[(size_t)item * d.bstride + (size_t)(r0 + row) * d.ld + kpb * PANEL_K + 32 * (i & 3) + kl];
    }
#pragma unroll
    for (int i = 0; i < 64; ++i)
        tile[(2 * (i >> 2) + (lane >> 5)) * STAGE_PITCH + 32 * (i & 3) + kl] = v[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float* src = tile + (lane & 31) * STAGE_PITCH + 16 * (lane >> 5);
#pragma unroll
    for (int g = 0; g < SPLIT_G; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 t = *reinterpret_cast<const float4*>(src + g * PANEL_K + 4 * q);
            x[g][4 * q + 0] = t.x;
            x[g][4 * q + 1] = t.y;
            x[g][4 * q + 2] = t.z;
            x[g][4 * q + 3] = t.w;
        }
}

template <int S, bool INT32_OUT>
__device__ void split_operand(const SliceDesc& d, long long blk) {
    __shared__ float smax[8][32];
    __shared__ int sse[32];
    // Staging tiles of the row path, one per wavefront; allocated at launch (dynamic LDS) only
    // when an operand of the launch takes that path, so column-access launches keep occupancy.
    extern __shared__ float stage[];
    const int npk = d.Kp / PANEL_K;
    const int rpanels = d.batch * (d.Rp / PANEL_ROWS);   // stacked over the items
    const int kgroups = (npk + 4 * SPLIT_G - 1) / (4 * SPLIT_G);
    // Column access: neighbouring blocks take neighbouring row panels of the same k rows;
    // row access: neighbouring blocks continue along k of the same rows.
    int rp, kg;
    if (d.strided && !d.vec) {
        // Unaligned rows: a panel's 128-byte run of a k-row straddles two lines, each shared
        // with a neighbouring row panel. Block blk runs on XCD blk % 8 (the dispatcher's round
        // robin; split_blocks is a multiple of 8 here). Each XCD takes a contiguous range of
        // (k group, row panel) in panel order, so neighbouring panels run together on one XCD
        // and fetch the shared lines into its L2 once.
        const long long per_xcd = d.split_blocks / 8;
        const long long lin = (blk & 7) * per_xcd + (blk >> 3);
        if (lin >= (long long)rpanels * kgroups) return;  // padding block (whole block)
        rp = (int)(lin % rpanels);
        kg = (int)(lin / rpanels);
    } else if (d.strided) {
        rp = (int)(blk % rpanels);
        kg = (int)(blk / rpanels);
    } else {
        rp = (int)(blk / kgroups);
        kg = (int)(blk % kgroups);
    }
    const int t = threadIdx.x;
    // A panel never straddles two items (Rp is a multiple of the panel height).
    const int item = (rp * PANEL_ROWS) / d.Rp;
    const int r0 = rp * PANEL_ROWS - item * d.Rp;  // the panel's first row within its item
    const size_t rows_total = (size_t)d.batch * d.Rp;
    {   // row maxima of this panel's 32 rows, reduced once for the whole block
        const int rr = t & 31, c0 = t >> 5;
        float m = 0.0f;
        if (r0 + rr < d.R) {
            const float* pm = d.pmax + rp * PANEL_ROWS + rr;
            int c = c0;
            for (; c + 24 < d.nch; c += 32)  // four independent loads in flight
                m = fmaxf(m, fmaxf(fmaxf(pm[(size_t)c * rows_total], pm[(size_t)(c + 8) * rows_total]),
                                   fmaxf(pm[(size_t)(c + 16) * rows_total], pm[(size_t)(c + 24) * rows_total])));
            for (; c < d.nch; c += 8) m = fmaxf(m, pm[(size_t)c * rows_total]);
        }
        smax[c0][rr] = m;
    }
    __syncthreads();
    if (t < 32) {
        float m = smax[0][t];
#pragma unroll
        for (int i = 1; i < 8; ++i) m = fmaxf(m, smax[i][t]);
        const int se = row_exponent(d, rp * PANEL_ROWS + t, m);  // rows >= R: m == 0, se == 0
        sse[t] = se;
        if (kg == 0) d.expo[rp * PANEL_ROWS + t] = se;
    }
    __syncthreads();
    const int lane = t & 63, wv = t >> 6;
    const int r = r0 + (lane & 31), h = lane >> 5;       // row within the item
    const int q = rp * PANEL_ROWS + (lane & 31);         // stacked row
    const float* rowp = r < d.R ? d.src + (size_t)item * d.bstride +
                                      (d.strided ? (size_t)r : (size_t)r * d.ld)
                                : nullptr;
    const RowScale rs = row_scale<S>(sse[lane & 31]);
    const int kpb = kg * 4 * SPLIT_G + wv * SPLIT_G;
    if (kpb + SPLIT_G <= npk && (kpb + SPLIT_G) * PANEL_K <= d.K) {
        // Every panel of this wavefront lies inside K: issue all loads, then round.
        float x[SPLIT_G][16];
        if (!d.strided && d.vec) {
            static_assert(SPLIT_G * PANEL_K == 128, "staged loads cover 2 rows x 128 k per instruction");
            load_panels_staged(d, stage + wv * 32 * STAGE_PITCH, item, r0, kpb, lane, x);
        } else if (!d.strided) {
            load_panels_staged_scalar(d, stage + wv * 32 * STAGE_PITCH, item, r0, kpb, lane, x);
        } else {
#pragma unroll
            for (int g = 0; g < SPLIT_G; ++g) load_panel(d, kpb + g, rowp, h, false, x[g]);
        }
#pragma unroll
        for (int g = 0; g < SPLIT_G; ++g) emit_panel<S, INT32_OUT>(d, x[g], rs, rp, kpb + g, q, h, lane);
    } else {
        for (int g = 0; g < SPLIT_G; ++g) {
            const int kp = kpb + g;
            if (kp >= npk) break;
            float x[16];
            load_panel(d, kp, rowp, h, true, x);
            emit_panel<S, INT32_OUT>(d, x, rs, rp, kp, q, h, lane);
        }
    }
}

template <int S, bool INT32_OUT>
__global__ void __launch_bounds__(256) split_kernel(SliceDesc a, SliceDesc b) {
    const long long blk = blockIdx.x;
    if (blk < a.split_blocks) split_operand<S, INT32_OUT>(a, blk);
    else split_operand<S, INT32_OUT>(b, blk - a.split_blocks);
}

// One pass for padded K <= 256 * NF4 (both operands share K): block blk of an operand owns a
// strip of 8 rows of op(X), a quarter of a 32-row panel, over all of K, held in registers (NF4
// float4 per lane, so two blocks fit on a CU and one loads while the other rounds and
// stores). Wavefront w covers k in [32*NF4*w, 32*NF4*(w+1)) for all 8 rows; instruction i
// covers its k-panel i:
//   row access    lane L loads row L/8, k = 4*(L%8)..+3 of the panel: 8 rows x 128 bytes;
//   column access lane L loads k = L/2 of the panel, columns 4*(L%2)..+3: 32 k-rows x 32 bytes.
// The rows' maxima are reduced with lane shuffles and across the 8 wavefronts in LDS, then each
// lane rounds 4 values and writes their digits as one 4-byte word per digit plane: for row
// access the lane's own values (four consecutive lanes fill a 16-byte run, eight rows a
// 128-byte run); for column access after a transpose of the panel's 32 k x 8 columns through
// the wavefront's LDS tile. Blocks blk, blk+8, blk+16, blk+24, which the dispatcher places on
// the same XCD, take four neighbouring strips, so a column-access operand's 128-byte lines
// (32 columns) are fetched into one L2 once.
//
// Wave-strip form (WS, padded K <= 256, NF4 = its k-panels): each wavefront owns its own strip
// (strip 8 blk + w) over all of K, so short rows keep all 8 wavefronts busy; the maxima are
// then reduced within the wavefront only and no block barrier is needed.
// Four consecutive values k .. k+3 (those below K) of row `row` of the implicit im2col matrix
// whose window origin in image xn is (y0, x0); zero in the padding and past K.
__device__ __forceinline__ float4 im2col_values(const Im2col& g, const float* xn, int y0, int x0,
                                                int k, int K) {
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        t[j] = 0.0f;
        const int kk = k + j;
        if (kk < K) {
            const int c = (int)fdiv((uint32_t)kk, g.dKHW), r = kk - c * (g.KH * g.KW);
            const int ky = (int)fdiv((uint32_t)r, g.dKW), kx = r - ky * g.KW;
            const int y = y0 + ky, x = x0 + kx;
            if (y >= 0 && y < g.H && x >= 0 && x < g.W) t[j] = xn[((size_t)c * g.H + y) * g.W + x];
        }
    }
    return make_float4(t[0], t[1], t[2], t[3]);
}

// NT: row-access loads are non-temporal (the fp32 values are read once and need not stay in
// the caches), used where another operand is read twice in the same GEMM.
template <int S, int NF4, bool WS = false, bool G = false, bool NT = false>
__device__ __forceinline__ void slice_onepass(const SliceDesc& d, long long blk) {
    __shared__ float smax[8][8];
    __shared__ int sse[8];
    __shared__ float tr[8][8][33];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int per_item = d.Rp / 8;
    const long long nstrips = (long long)d.batch * per_item;
    const long long st = WS ? blk * 8 + w : (blk >> 5) * 32 + (blk & 7) * 4 + ((blk >> 3) & 3);
    if (st >= nstrips) return;  // the whole block (a whole wavefront for WS)
    const int item = (int)(st / per_item);
    const int r0 = (int)(st - (long long)item * per_item) * 8;  // first row within the item
    const int rp = (item * d.Rp + r0) / PANEL_ROWS;              // stacked 32-row panel
    const int r_in = r0 & 24;                                    // strip offset in the panel
    const float* base = d.src + (size_t)item * d.bstride;
    const int kp0 = WS ? 0 : w * NF4;                            // this wavefront's first k-panel
    const int npk = d.Kp / PANEL_K;
    float4 v[NF4];
    float wmax = 0.0f;
    if (G && d.im2col) {  // rows of the implicit im2col matrix (one item, row access)
        const int row = r0 + (lane >> 3);
        const Im2col& g = d.g;
        int y0 = 0, x0 = 0;
        const float* xn = g.x;
        if (row < d.R) {
            const int n = (int)fdiv((uint32_t)row, g.dP), p = row - n * g.P;
            const int oy = (int)fdiv((uint32_t)p, g.dOW), ox = p - oy * g.OW;
            y0 = oy * g.SY - g.PY;
            x0 = ox * g.SX - g.PX;
            xn = g.x + (size_t)n * g.C * g.H * g.W;
        }
#pragma unroll
        for (int i = 0; i < NF4; ++i) {
            const int k = (kp0 + i) * PANEL_K + 4 * (lane & 7);
            v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (row < d.R && k < d.K) v[i] = im2col_values(g, xn, y0, x0, k, d.K);
        }
        // A window's maximum compares magnitude bits, so a NaN in the window wins and the
        // window takes exponent 0 (repro_conv_math.cuh:73-86); the reduction across the
        // wavefronts below keeps it (bits).
        unsigned mb = 0;
#pragma unroll
        for (int i = 0; i < NF4; ++i) mb = max(mb, max4_bits(v[i]));
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) mb = max(mb, (unsigned)__shfl_xor((int)mb, off, 64));
        const float m = __uint_as_float(mb);
        if (WS) wmax = m;  // lanes 8j..8j+7 all hold row j's maximum
        else if ((lane & 7) == 0) smax[w][lane >> 3] = m;
    } else if (!d.strided) {
        const int row = r0 + (lane >> 3);
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < NF4; ++i) {
            const int k = (kp0 + i) * PANEL_K + 4 * (lane & 7);
            v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (row < d.R && k < d.K) {
                const float* q = base + (size_t)row * d.ld + k;
                if (d.vec) {
                    if constexpr (NT) {
                        typedef float f4nt __attribute__((ext_vector_type(4)));
                        const f4nt t = __builtin_nontemporal_load(reinterpret_cast<const f4nt*>(q));
                        v[i] = make_float4(t.x, t.y, t.z, t.w);
                    } else {
                        v[i] = *reinterpret_cast<const float4*>(q);
                    }
                } else {  // unaligned rows or K % 4 != 0: four scalar loads inside K (in the one
                          // pass they cost no more than load_row_realigned: 8192 rows, K = 4095,
                          // 1-2 us faster; K = 767 within 1 us)
                    v[i].x = q[0];
                    if (k + 1 < d.K) v[i].y = q[1];
                    if (k + 2 < d.K) v[i].z = q[2];
                    if (k + 3 < d.K) v[i].w = q[3];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NF4; ++i) m = fmaxf(m, max4(v[i]));
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        if (WS) wmax = m;  // lanes 8j..8j+7 all hold row j's maximum
        else if ((lane & 7) == 0) smax[w][lane >> 3] = m;
    } else {
        const int c = r0 + 4 * (lane & 1);
        float4 m = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < NF4; ++i) {
            const int k = (kp0 + i) * PANEL_K + (lane >> 1);
            v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (k < d.K && c < d.R) {
                const float* q = base + (size_t)k * d.ld + c;
                if (d.vec) {
                    v[i] = *reinterpret_cast<const float4*>(q);
                } else {  // unaligned or R % 4 != 0: four scalar loads inside R
                    v[i].x = q[0];
                    if (c + 1 < d.R) v[i].y = q[1];
                    if (c + 2 < d.R) v[i].z = q[2];
                    if (c + 3 < d.R) v[i].w = q[3];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NF4; ++i) {
            m.x = fmaxf(m.x, fabsf(v[i].x));
            m.y = fmaxf(m.y, fabsf(v[i].y));
            m.z = fmaxf(m.z, fabsf(v[i].z));
            m.w = fmaxf(m.w, fabsf(v[i].w));
        }
#pragma unroll
        for (int off = 2; off < 64; off <<= 1) {
            m.x = fmaxf(m.x, __shfl_xor(m.x, off, 64));
            m.y = fmaxf(m.y, __shfl_xor(m.y, off, 64));
            m.z = fmaxf(m.z, __shfl_xor(m.z, off, 64));
            m.w = fmaxf(m.w, __shfl_xor(m.w, off, 64));
        }
        if (WS) {  // column lane/8 of the strip: component (lane/8) % 4 of lane (lane/8) / 4
            const int c = lane >> 3;
            const float mx = __shfl(m.x, c >> 2, 64), my = __shfl(m.y, c >> 2, 64);
            const float mz = __shfl(m.z, c >> 2, 64), mw = __shfl(m.w, c >> 2, 64);
            wmax = (c & 3) == 0 ? mx : (c & 3) == 1 ? my : (c & 3) == 2 ? mz : mw;
        } else if (lane < 2) {
            smax[w][4 * lane + 0] = m.x;
            smax[w][4 * lane + 1] = m.y;
            smax[w][4 * lane + 2] = m.z;
            smax[w][4 * lane + 3] = m.w;
        }
    }
    int lane_se = 0;  // WS: exponent of this lane's row (row or column lane / 8 of the strip)
    if (WS) {
        // rows >= R have a zero maximum, so exponent 0
        lane_se = row_exponent(d, (size_t)item * d.Rp + r0 + (lane >> 3), wmax);
        if ((lane & 7) == 0) d.expo[(size_t)item * d.Rp + r0 + (lane >> 3)] = lane_se;
    } else {
        __syncthreads();
        if (threadIdx.x < 8) {
            // The partial maxima are non-negative, so their bits order like them (a gathered
            // window's NaN wins).
            unsigned mb = __float_as_uint(smax[0][threadIdx.x]);
#pragma unroll
            for (int i = 1; i < 8; ++i) mb = max(mb, __float_as_uint(smax[i][threadIdx.x]));
            // rows >= R have a zero maximum, so exponent 0
            const int se = row_exponent(d, (size_t)item * d.Rp + r0 + threadIdx.x, __uint_as_float(mb));
            sse[threadIdx.x] = se;
            d.expo[(size_t)item * d.Rp + r0 + threadIdx.x] = se;
        }
        __syncthreads();
    }
    // Output word of lane (row or column ro of the strip, 16-k half h, word wd) in panel kp.
    uint32_t* out = static_cast<uint32_t*>(d.out);
    const int ro = lane >> 3, h = (lane >> 2) & 1, wd = lane & 3;
    const RowScale rs = row_scale<S>(WS ? lane_se : sse[ro]);
    uint32_t* o0 = out + (size_t)rp * npk * S * (PANEL_BYTES / 4) + 4 * (r_in + ro + 32 * h) + wd;
    float (*tile)[33] = tr[w];
#pragma unroll
    for (int i = 0; i < NF4; ++i) {
        const int kp = kp0 + i;
        if (kp >= npk) break;
        float x[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        if (d.strided) {
            // this lane's k-row lane/2, columns 4*(lane%2)..+3 -> tile[column][k-row]; then
            // lane L takes column L/8, k = 4*(L%8)..+3
            const int c4 = 4 * (lane & 1), kr = lane >> 1;
            tile[c4 + 0][kr] = x[0];
            tile[c4 + 1][kr] = x[1];
            tile[c4 + 2][kr] = x[2];
            tile[c4 + 3][kr] = x[3];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = tile[ro][4 * (lane & 7) + j];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        int dg[S][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int d[S];
            digits_of<S>(round_fixed(x[j], rs), d);
#pragma unroll
            for (int p = 0; p < S; ++p) dg[p][j] = d[p];
        }
        uint32_t* o = o0 + (size_t)kp * S * (PANEL_BYTES / 4);
#pragma unroll
        for (int p = 0; p < S; ++p) o[p * (PANEL_BYTES / 4)] = pack4(dg[p][0], dg[p][1], dg[p][2], dg[p][3]);
    }
}

template <int S, int NF4, bool WS, bool G>
__global__ void __launch_bounds__(512) slice_onepass_kernel(SliceDesc a, SliceDesc b, long long a_blocks) {
    const long long blk = blockIdx.x;
    if (blk < a_blocks) slice_onepass<S, NF4, WS, G>(a, blk);
    else slice_onepass<S, NF4, WS, G>(b, blk - a_blocks);
}

// The one pass of operand `one` fused with the partial maxima (first of the two passes) of
// operand `two`, so the two share the memory system instead of running one after the other.
// The maxima use 8 wavefronts per block here (every 8th k of a chunk, or 8 rows). `one` is read
// with non-temporal loads so that `two`, which its split pass reads again, stays in the
// memory-side cache (4096^3 NN: slicing -2.4%, GEMM -0.9%; the same loads where both operands
// take one pass made 8192x768x768 3-5% slower).
template <int S, int NF4>
__global__ void __launch_bounds__(512) onepass_absmax_kernel(SliceDesc one, SliceDesc two, long long one_blocks) {
    const long long blk = blockIdx.x;
    if (blk < one_blocks) slice_onepass<S, NF4, false, false, true>(one, blk);
    else if (two.strided) absmax_cols<8>(two, blk - one_blocks);
    else absmax_rows<8>(two, blk - one_blocks);
}

// Blocks of the partial-maxima pass of d with 8 wavefronts per block.
static long long absmax8_blocks(const SliceDesc& d) {
    if (d.strided) return d.max_blocks;  // one block per (item, column group, chunk)
    const long long per_block = 8LL * rows_per_wave(d);
    return ((long long)d.batch * d.R * d.nch + per_block - 1) / per_block;
}

// Blocks of the one-pass slicing for one operand: its 8-row strips, rounded up to a multiple
// of 32 so the XCD grouping of neighbouring strips stays inside the operand's blocks.
static long long onepass_blocks(const SliceDesc& d) {
    const long long strips = (long long)d.batch * (d.Rp / 8);
    return (strips + 31) / 32 * 32;
}

// k panels per wavefront of the block-strip one pass: the smallest instantiated count with which
// the 8 wavefronts cover every k panel, so few wavefronts of a block sit idle (K = 768: 3 each;
// K = 2304: 9).
static int onepass_nf4(int Kp) {
    const int need = (Kp / PANEL_K + 7) / 8;
    for (int nf : {3, 4, 6, 8, 9, 12, 16})
        if (nf >= need) return nf;
    return 16;
}

bool onepass_eligible(const SliceDesc& d) {
    return d.Kp <= (d.strided ? ONEPASS_MAX_K_COLUMNS : ONEPASS_MAX_K);
}

void launch_onepass(const SliceDesc& a, bool use_a, const SliceDesc& b, bool use_b, int S,
                    hipStream_t stream) {
    const int kp = use_a ? a.Kp : b.Kp;
    // Gathering (implicit im2col) instantiations only when an operand gathers, so the plain
    // GEMM's kernels carry none of that code.
    const bool gather = (use_a && a.im2col) || (use_b && b.im2col);
    if (kp <= 256) {  // wave strips: 8 strips per block
        const long long na = use_a ? ((long long)a.batch * (a.Rp / 8) + 7) / 8 : 0;
        const long long nb = use_b ? ((long long)b.batch * (b.Rp / 8) + 7) / 8 : 0;
        if (na + nb == 0) return;
        const unsigned blocks = (unsigned)(na + nb);
        const int nf4 = kp <= 64 ? 2 : (kp <= 128 ? 4 : 8);
#define RG_ONEPASS_WS(SS, NF)                                                                  \
    (gather ? slice_onepass_kernel<SS, NF, true, true><<<blocks, 512, 0, stream>>>(a, b, na)  \
            : slice_onepass_kernel<SS, NF, true, false><<<blocks, 512, 0, stream>>>(a, b, na))
        switch (S * 100 + nf4) {
            case 102: RG_ONEPASS_WS(1, 2); break;
            case 104: RG_ONEPASS_WS(1, 4); break;
            case 108: RG_ONEPASS_WS(1, 8); break;
            case 202: RG_ONEPASS_WS(2, 2); break;
            case 204: RG_ONEPASS_WS(2, 4); break;
            case 208: RG_ONEPASS_WS(2, 8); break;
            case 302: RG_ONEPASS_WS(3, 2); break;
            case 304: RG_ONEPASS_WS(3, 4); break;
            case 308: RG_ONEPASS_WS(3, 8); break;
            default: break;
        }
#undef RG_ONEPASS_WS
        return;
    }
    const long long na = use_a ? onepass_blocks(a) : 0;
    const long long nb = use_b ? onepass_blocks(b) : 0;
    if (na + nb == 0) return;
    const unsigned blocks = (unsigned)(na + nb);
    const int nf4 = onepass_nf4(kp);
#define RG_ONEPASS(SS, NF)                                                                      \
    (gather ? slice_onepass_kernel<SS, NF, false, true><<<blocks, 512, 0, stream>>>(a, b, na) \
            : slice_onepass_kernel<SS, NF, false, false><<<blocks, 512, 0, stream>>>(a, b, na))
#define RG_ONEPASS_S(SS)                                                                        \
    case SS * 100 + 3: RG_ONEPASS(SS, 3); break;                                                \
    case SS * 100 + 4: RG_ONEPASS(SS, 4); break;                                                \
    case SS * 100 + 6: RG_ONEPASS(SS, 6); break;                                                \
    case SS * 100 + 8: RG_ONEPASS(SS, 8); break;                                                \
    case SS * 100 + 9: RG_ONEPASS(SS, 9); break;                                                \
    case SS * 100 + 12: RG_ONEPASS(SS, 12); break;                                              \
    case SS * 100 + 16: RG_ONEPASS(SS, 16); break;
    switch (S * 100 + nf4) {
        RG_ONEPASS_S(1)
        RG_ONEPASS_S(2)
        RG_ONEPASS_S(3)
        default: break;
    }
#undef RG_ONEPASS_S
#undef RG_ONEPASS
}

void launch_onepass_absmax(const SliceDesc& one, const SliceDesc& two, int S, hipStream_t stream) {
    const long long n1 = onepass_blocks(one);
    const unsigned blocks = (unsigned)(n1 + absmax8_blocks(two));
    const int nf4 = onepass_nf4(one.Kp);
#define RG_FUSED(SS, NF) onepass_absmax_kernel<SS, NF><<<blocks, 512, 0, stream>>>(one, two, n1)
#define RG_FUSED_S(SS)                                                                          \
    case SS * 100 + 3: RG_FUSED(SS, 3); break;                                                  \
    case SS * 100 + 4: RG_FUSED(SS, 4); break;                                                  \
    case SS * 100 + 6: RG_FUSED(SS, 6); break;                                                  \
    case SS * 100 + 8: RG_FUSED(SS, 8); break;                                                  \
    case SS * 100 + 9: RG_FUSED(SS, 9); break;                                                  \
    case SS * 100 + 12: RG_FUSED(SS, 12); break;                                                \
    case SS * 100 + 16: RG_FUSED(SS, 16); break;
    switch (S * 100 + nf4) {
        RG_FUSED_S(1)
        RG_FUSED_S(2)
        RG_FUSED_S(3)
        default: break;
    }
#undef RG_FUSED_S
#undef RG_FUSED
}

// One read of a column-access operand past the one-pass limit (element (r, k) of item b at
// src[b*bstride + k*ld + r]). Block (rp, part) owns the 32-row panel rp of op(X) (32
// neighbouring columns of the stored matrix) over the k panels [part*8*KPW, (part+1)*8*KPW):
// wavefront w takes KPW of them, lane L column L % 32 and the 16 k of half L / 32 of each, as
// scalar loads (each load instruction reads two 128-byte k-row segments), and keeps them in
// registers. The panel's row maxima need every part: each block publishes its 32 partial maxima
// in its slots pmax[part][rows] and waits until the other parts' slots of the panel hold values
// (an earlier launch of the same call marked every slot PM_EMPTY, so any other value in a slot
// is this call's); then every block rounds its own values and writes their digit panels, so
// the input is read once. The wait is bounded: a block that does not see every part's maxima
// after spin_limit polls reads the panel's whole K itself for them (the same values: the
// maximum is exact and order-free), so no block depends on another being resident or visible.
// Part 0 writes the exponents.
// Blocks run on XCD blk % 8 (the dispatcher deals workgroups to the XCDs in turn) and each XCD
// takes a contiguous range of (panel, part) in panel order, a whole number of panels
// (pslice_unit), so a panel's parts are dispatched one after another on one XCD, and the
// neighbouring panels of an unaligned operand, which share the lines at their edges, run on one
// XCD too. The slots are
// therefore written with plain stores, which land in the XCD's L2 (the compute unit's L1 is
// write-through), and polled with non-temporal loads, which skip the L1 (where a polled line
// would stay stale) and are served by that L2. A device-scope exchange instead goes to the
// memory-side coherence point and, with acquire/release fences, writes back and invalidates the
// XCD's whole L2 while the launch's other blocks fill it with digits. A block whose parts ran on
// another XCD can only see PM_EMPTY or this call's maxima (the slots were marked by an earlier
// launch, whose writes the launch boundary made visible everywhere), so at worst it takes the
// fallback: placement never changes a bit. KPW = PS_KPW_WIDE (K past 32768) makes each part
// 2.5 times longer, so that a panel has at most 26 parts, which one XCD holds at once with room
// to spare.
// Eight slot words read past the L1 with one wait: a poll costs one round trip per eight parts
// (the LM head's weight gradient, 8 parts: slicing 0.605 -> 0.595 ms against four per wait,
// 0.65 ms with one).
__device__ __forceinline__ void load8_bypass_l1(const unsigned* const (&p)[8], unsigned (&v)[8]) {
    asm volatile(
        "global_load_dword %0, %8, off nt\n\t"
        "global_load_dword %1, %9, off nt\n\t"
        "global_load_dword %2, %10, off nt\n\t"
        "global_load_dword %3, %11, off nt\n\t"
        "global_load_dword %4, %12, off nt\n\t"
        "global_load_dword %5, %13, off nt\n\t"
        "global_load_dword %6, %14, off nt\n\t"
        "global_load_dword %7, %15, off nt\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
        : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6]), "v"(p[7])
        : "memory");
}

__device__ __forceinline__ bool panel_exchange(unsigned* pm, size_t part_stride, int part, int parts,
                                               int spin_limit, int lane, int nl, float* mm) {
    if (spin_limit <= 0) return false;
    if (lane < nl) pm[(size_t)part * part_stride] = __float_as_uint(*mm);
    for (int n = 0;; ++n) {
        float m = *mm;
        bool seen = true;
        if (lane < nl)
            for (int p0 = 0; p0 < parts; p0 += 8) {
                // slots p0 .. p0 + 7 (past the last part: the last part's again), own slot ignored
                const unsigned* q[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) q[j] = pm + (size_t)min(p0 + j, parts - 1) * part_stride;
                unsigned v[8];
                load8_bypass_l1(q, v);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (p0 + j >= parts || p0 + j == part) continue;
                    if (v[j] == PM_EMPTY) seen = false;
                    else m = fmaxf(m, __uint_as_float(v[j]));
                }
            }
        if (__all(seen)) {
            *mm = m;
            return true;
        }
        if (n >= spin_limit) return false;
        __builtin_amdgcn_s_sleep(2);
    }
}

template <int S, int KPW>
__device__ __forceinline__ void pslice_cols(const SliceDesc& d, long long blk) {
    __shared__ float smax[16][32];
    __shared__ float sfin[32];
    __shared__ int sse[32];
    __shared__ int sok;
    const int npk = d.Kp / PANEL_K;
    const int parts = d.ps_parts;
    const long long rpanels = (long long)d.batch * (d.Rp / PANEL_ROWS);
    const long long lin = pslice_unit(blk, d.ps_blocks);
    if (lin >= rpanels * parts) return;  // padding block (whole block)
    const int rp = (int)(lin / parts), part = (int)(lin - (long long)rp * parts);
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int item = (rp * PANEL_ROWS) / d.Rp;
    const int r0 = rp * PANEL_ROWS - item * d.Rp;  // the panel's first row within its item
    const size_t rows_total = (size_t)d.batch * d.Rp;
    const int r = r0 + (lane & 31), h = lane >> 5;
    const int q = rp * PANEL_ROWS + (lane & 31);
    const float* colp = d.src + (size_t)item * d.bstride + r;
    const bool live = r < d.R;
    const int kp0 = part * (PS_WAVES * KPW) + wv * KPW;
    float x[KPW][16];
    if (live && (kp0 + KPW) * PANEL_K <= d.K) {  // every value of this wavefront inside K
#pragma unroll
        for (int i = 0; i < KPW; ++i) {
            const float* p = colp + (size_t)((kp0 + i) * PANEL_K + 16 * h) * d.ld;
#pragma unroll
            for (int j = 0; j < 16; ++j) x[i][j] = p[(size_t)j * d.ld];
        }
    } else {
#pragma unroll
        for (int i = 0; i < KPW; ++i) {
            const int k0 = (kp0 + i) * PANEL_K + 16 * h;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                x[i][j] = (live && k0 + j < d.K) ? colp[(size_t)(k0 + j) * d.ld] : 0.0f;
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < KPW; ++i)
#pragma unroll
        for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(x[i][j]));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (lane < 32) smax[wv][lane] = m;
    __syncthreads();
    if (wv == 0) {
        float mm = 0.0f;
        if (lane < 32) {
            mm = smax[0][lane];
#pragma unroll
            for (int w = 1; w < PS_WAVES; ++w) mm = fmaxf(mm, smax[w][lane]);
        }
        int ok = 1;
        if (parts > 1) {
            unsigned* pm = reinterpret_cast<unsigned*>(d.pmax) + rp * PANEL_ROWS + (lane & 31);
            ok = panel_exchange(pm, rows_total, part, parts, d.spin_limit, lane, 32, &mm) ? 1 : 0;
        }
        if (lane < 32) sfin[lane] = mm;
        if (lane == 0) sok = ok;
    }
    __syncthreads();
    if (!sok) {  // the other parts' maxima were not all seen: the panel's maxima over all of K
        const int c = t & 31, kph = t >> 5;  // 16 k phases of 32 columns
        float mm = 0.0f;
        if (r0 + c < d.R) {
            const float* p = d.src + (size_t)item * d.bstride + r0 + c;
            for (int k = kph; k < d.K; k += 16) mm = fmaxf(mm, fabsf(p[(size_t)k * d.ld]));
        }
        smax[kph][c] = mm;
        __syncthreads();
        if (t < 32) {
            float f = smax[0][t];
#pragma unroll
            for (int i = 1; i < 16; ++i) f = fmaxf(f, smax[i][t]);
            sfin[t] = f;
        }
        __syncthreads();
    }
    if (t < 32) {
        // rows >= R have a zero maximum, so se == 0
        const int se = row_exponent(d, rp * PANEL_ROWS + t, sfin[t]);
        sse[t] = se;
        if (part == 0) d.expo[rp * PANEL_ROWS + t] = se;
    }
    __syncthreads();
    const RowScale rs = row_scale<S>(sse[lane & 31]);
#pragma unroll
    for (int i = 0; i < KPW; ++i)
        if (kp0 + i < npk) emit_panel<S, false>(d, x[i], rs, rp, kp0 + i, q, h, lane);
}

// One read of a row-access operand past the one-pass limit (element (r, k) of item b at
// src[b*bstride + r*ld + k]): block (strip, part) holds a strip of 8 rows over the k panels
// [part*PS_ROW_NPB, (part+1)*PS_ROW_NPB) in registers, laid out as the one pass lays out its
// strip (wavefront w: PS_ROW_NF4 k panels, lane L: row L/8 and k 4*(L%8)..+3 of each panel, 16-byte
// loads), and exchanges its 8 partial maxima with the strip's other parts as pslice_cols does.
template <int S>
__device__ __forceinline__ void pslice_rows(const SliceDesc& d, long long blk) {
    __shared__ float smax[8][8];
    __shared__ float sfin[8];
    __shared__ int sse[8];
    __shared__ int sok;
    const int npk = d.Kp / PANEL_K;
    const int parts = d.ps_parts;
    const int per_item = d.Rp / 8;
    const long long nstrips = (long long)d.batch * per_item;
    const long long lin = pslice_unit(blk, d.ps_blocks);
    if (lin >= nstrips * parts) return;  // padding block (whole block)
    const long long st = lin / parts;
    const int part = (int)(lin - st * parts);
    const int item = (int)(st / per_item);
    const int r0 = (int)(st - (long long)item * per_item) * 8;  // first row within the item
    const int rp = (item * d.Rp + r0) / PANEL_ROWS;              // stacked 32-row panel
    const int r_in = r0 & 24;                                    // strip offset in the panel
    const size_t rows_total = (size_t)d.batch * d.Rp;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float* base = d.src + (size_t)item * d.bstride;
    const int kp0 = part * PS_ROW_NPB + w * PS_ROW_NF4;
    const int row = r0 + (lane >> 3);
    float4 v[PS_ROW_NF4];
    float m = 0.0f;
    if (d.vec) {
#pragma unroll
        for (int i = 0; i < PS_ROW_NF4; ++i) {
            const int k = (kp0 + i) * PANEL_K + 4 * (lane & 7);
            v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (row < d.R && k < d.K) v[i] = *reinterpret_cast<const float4*>(base + (size_t)row * d.ld + k);
        }
    } else {  // rows not 16-byte aligned
        load_row_realigned<PS_ROW_NF4>(base + (size_t)row * d.ld, d.K, kp0 * PANEL_K, lane, row < d.R, v);
    }
#pragma unroll
    for (int i = 0; i < PS_ROW_NF4; ++i) m = fmaxf(m, max4(v[i]));
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((lane & 7) == 0) smax[w][lane >> 3] = m;
    __syncthreads();
    if (w == 0) {
        float mm = 0.0f;
        if (lane < 8) {
            mm = smax[0][lane];
#pragma unroll
            for (int i = 1; i < 8; ++i) mm = fmaxf(mm, smax[i][lane]);
        }
        int ok = 1;
        if (parts > 1) {
            unsigned* pm = reinterpret_cast<unsigned*>(d.pmax) + (size_t)item * d.Rp + r0 + (lane & 7);
            ok = panel_exchange(pm, rows_total, part, parts, d.spin_limit, lane, 8, &mm) ? 1 : 0;
        }
        if (lane < 8) sfin[lane] = mm;
        if (lane == 0) sok = ok;
    }
    __syncthreads();
    if (!sok) {  // the other parts' maxima were not all seen: wavefront w reads row r0 + w whole
        float mm = 0.0f;
        if (r0 + w < d.R) {
            const float* q = base + (size_t)(r0 + w) * d.ld;
            for (int k = lane; k < d.K; k += 64) mm = fmaxf(mm, fabsf(q[k]));
        }
        mm = wave_max(mm);
        if (lane == 0) sfin[w] = mm;
        __syncthreads();
    }
    if (t < 8) {
        // rows >= R have a zero maximum, so se == 0
        const int se = row_exponent(d, (size_t)item * d.Rp + r0 + t, sfin[t]);
        sse[t] = se;
        if (part == 0) d.expo[(size_t)item * d.Rp + r0 + t] = se;
    }
    __syncthreads();
    uint32_t* out = static_cast<uint32_t*>(d.out);
    const int ro = lane >> 3, h = (lane >> 2) & 1, wd = lane & 3;
    const RowScale rs = row_scale<S>(sse[ro]);
    uint32_t* o0 = out + (size_t)rp * npk * S * (PANEL_BYTES / 4) + 4 * (r_in + ro + 32 * h) + wd;
#pragma unroll
    for (int i = 0; i < PS_ROW_NF4; ++i) {
        const int kp = kp0 + i;
        if (kp >= npk) break;
        const float x[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        int dg[S][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int dd[S];
            digits_of<S>(round_fixed(x[j], rs), dd);
#pragma unroll
            for (int p = 0; p < S; ++p) dg[p][j] = dd[p];
        }
        uint32_t* o = o0 + (size_t)kp * S * (PANEL_BYTES / 4);
#pragma unroll
        for (int p = 0; p < S; ++p) o[p * (PANEL_BYTES / 4)] = pack4(dg[p][0], dg[p][1], dg[p][2], dg[p][3]);
    }
}

// WIDE: the launch's column-access operands take PS_KPW_WIDE k panels per wavefront (instantiated
// apart, so that the common form keeps its register budget).
template <int S, bool WIDE>
__device__ __forceinline__ void pslice_block(const SliceDesc& d, long long blk) {
    if (d.strided) pslice_cols<S, WIDE ? PS_KPW_WIDE : PS_KPW>(d, blk);
    else pslice_rows<S>(d, blk);
}

template <int S, bool WIDE>
__global__ void __launch_bounds__(64 * PS_WAVES, WIDE ? 2 : 4) pslice_kernel(SliceDesc a, SliceDesc b) {
    const long long blk = blockIdx.x;
    if (blk < a.ps_blocks) pslice_block<S, WIDE>(a, blk);
    else pslice_block<S, WIDE>(b, blk - a.ps_blocks);
}

// The one read of operand `two` and the one pass of operand `one` in one launch (two's slots
// marked by a launch before it), so that one's traffic keeps the memory busy while two's
// blocks exchange their maxima. two's blocks come first.
template <int S, int NF4>
__global__ void __launch_bounds__(512) onepass_pslice_kernel(SliceDesc one, SliceDesc two) {
    const long long blk = blockIdx.x;
    if (blk < two.ps_blocks) pslice_block<S, false>(two, blk);  // K <= 4096: never wide
    else slice_onepass<S, NF4>(one, blk - two.ps_blocks);
}

// The one read of operand `ps` and the partial maxima (first of the two passes) of operand `two`
// in one launch (ps's slots marked by a launch before it). ps's blocks come first.
template <int S>
__global__ void __launch_bounds__(512) pslice_absmax_kernel(SliceDesc ps, SliceDesc two) {
    const long long blk = blockIdx.x;
    if (blk < ps.ps_blocks) pslice_block<S, false>(ps, blk);  // a wide ps runs on its own
    else if (two.strided) absmax_cols<8>(two, blk - ps.ps_blocks);
    else absmax_rows<8>(two, blk - ps.ps_blocks);
}

// Marks the slots of m PM_EMPTY, spread over the launch's blocks.
__device__ __forceinline__ void mark_slots(const MarkRange& m) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < m.n;
         i += (long long)gridDim.x * blockDim.x)
        m.p[i] = PM_EMPTY;
}

__global__ void __launch_bounds__(256) mark_kernel(MarkRange a, MarkRange b) {
    mark_slots(a);
    mark_slots(b);
}

namespace {
int g_spin_limit = DEFAULT_SPIN_LIMIT;
}

int slice_spin_limit() { return g_spin_limit; }
void set_slice_spin_limit(int polls) { g_spin_limit = polls < 0 ? 0 : polls; }

void pslice_grid(SliceDesc& d) {
    d.ps_parts = pslice_parts(d.strided != 0, d.Kp);
    d.ps_kpw = pslice_kpw(d.strided != 0, d.Kp);
    // Whole panels (strips) per XCD: a panel's parts must not be split between two XCDs, whose
    // L2s do not see each other's slots (they would wait out their bound and re-read K).
    const long long panels = (long long)d.batch * (d.Rp / (d.strided ? PANEL_ROWS : 8));
    d.ps_blocks = 8 * ((panels + 7) / 8 * d.ps_parts);
}

MarkRange pslice_slots(const SliceDesc& d) {
    MarkRange m;
    if (d.ps_parts > 1) {
        m.p = reinterpret_cast<unsigned*>(d.pmax);
        m.n = (long long)d.ps_parts * d.batch * d.Rp;
    }
    return m;
}

void launch_pslice(const SliceDesc& a, bool use_a, const SliceDesc& b, bool use_b, int S,
                   hipStream_t stream) {
    SliceDesc x = a, y = b;
    if (!use_a) x.ps_blocks = 0;
    if (!use_b) y.ps_blocks = 0;
    const unsigned blocks = (unsigned)(x.ps_blocks + y.ps_blocks);
    if (blocks == 0) return;
    const bool wx = x.ps_blocks && x.ps_kpw == PS_KPW_WIDE, wy = y.ps_blocks && y.ps_kpw == PS_KPW_WIDE;
    if (x.ps_blocks && y.ps_blocks && wx != wy) {
        // The wide form holds half the waves per SIMD: the other operand takes a launch of its own.
        launch_pslice(a, true, b, false, S, stream);
        launch_pslice(a, false, b, true, S, stream);
        return;
    }
    const bool wide = wx || wy;
#define RG_PS(SS, W) pslice_kernel<SS, W><<<blocks, 64 * PS_WAVES, 0, stream>>>(x, y)
    switch (S * 2 + (wide ? 1 : 0)) {
        case 2: RG_PS(1, false); break;
        case 3: RG_PS(1, true); break;
        case 4: RG_PS(2, false); break;
        case 5: RG_PS(2, true); break;
        case 7: RG_PS(3, true); break;
        default: RG_PS(3, false); break;
    }
#undef RG_PS
}

void launch_onepass_pslice(const SliceDesc& one, const SliceDesc& two, int S, hipStream_t stream) {
    const unsigned blocks = (unsigned)(onepass_blocks(one) + two.ps_blocks);
#define RG_OPS(SS, NF) onepass_pslice_kernel<SS, NF><<<blocks, 512, 0, stream>>>(one, two)
#define RG_OPS_S(SS)                                                                            \
    case SS * 100 + 3: RG_OPS(SS, 3); break;                                                    \
    case SS * 100 + 4: RG_OPS(SS, 4); break;                                                    \
    case SS * 100 + 6: RG_OPS(SS, 6); break;                                                    \
    case SS * 100 + 8: RG_OPS(SS, 8); break;                                                    \
    case SS * 100 + 9: RG_OPS(SS, 9); break;                                                    \
    case SS * 100 + 12: RG_OPS(SS, 12); break;                                                  \
    case SS * 100 + 16: RG_OPS(SS, 16); break;
    switch (S * 100 + onepass_nf4(one.Kp)) {
        RG_OPS_S(1)
        RG_OPS_S(2)
        RG_OPS_S(3)
        default: break;
    }
#undef RG_OPS_S
#undef RG_OPS
}

void launch_pslice_absmax(const SliceDesc& ps, const SliceDesc& two, int S, hipStream_t stream) {
    SliceDesc x = ps;
    if (ps.strided && ps.ps_kpw == PS_KPW_WIDE) {
        // the wide form (half the waves per SIMD) on its own, then two's maxima
        launch_pslice(ps, true, ps, false, S, stream);
        x.ps_blocks = 0;
    }
    const unsigned blocks = (unsigned)(x.ps_blocks + absmax8_blocks(two));
    switch (S) {
        case 1: pslice_absmax_kernel<1><<<blocks, 512, 0, stream>>>(x, two); break;
        case 2: pslice_absmax_kernel<2><<<blocks, 512, 0, stream>>>(x, two); break;
        default: pslice_absmax_kernel<3><<<blocks, 512, 0, stream>>>(x, two); break;
    }
}

void launch_mark(MarkRange a, MarkRange b, hipStream_t stream) {
    const long long n = a.n + b.n;
    if (n <= 0) return;
    const long long blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
    mark_kernel<<<(unsigned)blocks, 256, 0, stream>>>(a, b);
}

// Grid sizes of the two passes for one operand.
void slice_grid(SliceDesc& d) {
    if (d.strided) {
        const int cols = d.vec ? 256 : 64;
        d.max_blocks = (long long)d.batch * ((d.R + cols - 1) / cols) * d.nch;
        if (!d.vec && d.R > 32) d.max_blocks = (d.max_blocks + 7) / 8 * 8;  // whole XCD rounds
    } else {
        const long long per_block = 4LL * rows_per_wave(d);
        d.max_blocks = ((long long)d.batch * d.R * d.nch + per_block - 1) / per_block;
    }
    const int npk = d.Kp / PANEL_K;
    d.split_blocks = (long long)d.batch * (d.Rp / PANEL_ROWS) *
                     ((npk + 4 * SPLIT_G - 1) / (4 * SPLIT_G));
    if (d.strided && !d.vec) d.split_blocks = (d.split_blocks + 7) / 8 * 8;  // whole XCD rounds
}

// Group scales: every row of each group of `group` consecutive rows gets the group's largest
// magnitude. Block g reduces the partial maxima pmax[c][r] of its rows over every chunk c,
// then writes the maximum back to all of them, so the split sees one maximum per group.
// GroupMax: one operand's share of a launch, its blocks [0, blocks).
struct GroupMax {
    float* pmax;
    int R, Rp, nch, group, blocks;
};

__device__ void group_max_block(const GroupMax& d, int blk) {
    __shared__ float red[4];
    const int r0 = blk * d.group;
    const int r1 = min(d.R, r0 + d.group);
    float m = 0.0f;
    for (int c = 0; c < d.nch; ++c)
        for (int r = r0 + (int)threadIdx.x; r < r1; r += 256) m = fmaxf(m, d.pmax[(size_t)c * d.Rp + r]);
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int c = 0; c < d.nch; ++c)
        for (int r = r0 + (int)threadIdx.x; r < r1; r += 256) d.pmax[(size_t)c * d.Rp + r] = m;
}

// Both operands' groups in one launch (b.blocks may be 0).
__global__ void __launch_bounds__(256) group_max_kernel(GroupMax a, GroupMax b) {
    if ((int)blockIdx.x < a.blocks) group_max_block(a, blockIdx.x);
    else group_max_block(b, blockIdx.x - a.blocks);
}

static GroupMax group_max_of(const SliceDesc* d, int group) {
    GroupMax g{nullptr, 0, 0, 0, 1, 0};
    if (!d || group <= 0) return g;
    g.pmax = d->pmax;
    g.R = d->R;
    g.Rp = d->Rp;
    g.nch = d->nch;
    g.group = group >= d->R ? d->R : group;
    g.blocks = (d->R + g.group - 1) / g.group;
    return g;
}

void launch_group_max2(const SliceDesc* a, int group_a, const SliceDesc* b, int group_b,
                       hipStream_t stream) {
    const GroupMax ga = group_max_of(a, group_a), gb = group_max_of(b, group_b);
    if (ga.blocks + gb.blocks == 0) return;
    group_max_kernel<<<(unsigned)(ga.blocks + gb.blocks), 256, 0, stream>>>(ga, gb);
}

void launch_group_max(const SliceDesc& d, int group, hipStream_t stream) {
    launch_group_max2(&d, group, nullptr, 0, stream);
}

void launch_absmax(const SliceDesc& a, const SliceDesc& b, hipStream_t stream) {
    absmax_kernel<<<(unsigned)(a.max_blocks + b.max_blocks), 256, 0, stream>>>(a, b);
}

void launch_split(const SliceDesc& a, const SliceDesc& b, int S, bool int32_out, hipStream_t stream) {
    const unsigned blocks = (unsigned)(a.split_blocks + b.split_blocks);
    const bool staged = (a.split_blocks > 0 && !a.strided) || (b.split_blocks > 0 && !b.strided);
    const size_t lds = staged ? 4 * 32 * STAGE_PITCH * sizeof(float) : 0;
    switch (S * 2 + (int32_out ? 1 : 0)) {
        case 2: split_kernel<1, false><<<blocks, 256, lds, stream>>>(a, b); break;
        case 3: split_kernel<1, true><<<blocks, 256, lds, stream>>>(a, b); break;
        case 4: split_kernel<2, false><<<blocks, 256, lds, stream>>>(a, b); break;
        case 5: split_kernel<2, true><<<blocks, 256, lds, stream>>>(a, b); break;
        case 6: split_kernel<3, false><<<blocks, 256, lds, stream>>>(a, b); break;
        case 7: split_kernel<3, true><<<blocks, 256, lds, stream>>>(a, b); break;
        default: break;
    }
}

}  // namespace rg
