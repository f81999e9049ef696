// Exact contraction of the sliced operands and the final rounding.
//
// Replaces gemm_wmma_i8 / gemm_tiled_dp4a / gemm_reference / reduce_round / write_output
// (repro_gemm_cuda/repro_gemm.cu:124-165, 189-364).
//
// contract_mfma: a block of WGM x WGN wavefronts owns a (32*WGM*WTI) x (32*WGN*WTJ) tile of
// C; each wavefront owns WTI x WTJ tiles of 32x32 and runs V_MFMA_I32_32X32X32_I8 on them.
// Digit pairs (p, q) with the same level p + q share one int32 accumulator per output,
// so a wavefront holds (2S-1) * WTI * WTJ accumulator tiles. Each pipeline stage brings
// the block's digit panels for 64 values of k from HBM into a three-slot LDS ring with
// direct global->LDS loads issued two stages ahead; operand fragments are read from LDS
// with one 16-byte read per lane and panel. All level
// accumulators of one output sit in the same lane and register index, so the epilogue
// combines them in int64 without any data exchange:
//     T = sum_L acc_L * 2^(7 (2S-2-L)) = sum_k X[r,k] * Y[c,k]   (exact)
// and either rounds T once to FP32 (no partial buffer: one part) or stores it as an int64
// partial (split-K, or a caller that wants the exact integers).
// Integer addition is associative, so the tile shape, the split and the order of k
// never change T.
#include "rg_internal.h"
#include <type_traits>
#include "repro_gemm_math.h"

namespace rg {

// round_to_float for the rare inputs the binary64 paths hand over (|T| near or above 2^53),
// kept out of line so the epilogue's common path stays short.
__device__ __noinline__ float round_to_float_rare(int64_t T, int E) {
    return repro_gemm::round_to_float(T, E);
}

// T = sum_l lv[l] * 2^(7 (L-1-l)) as an exact int64.
template <int L>
__device__ __forceinline__ int64_t combine_levels(const int (&lv)[L]) {
    int64_t t = 0;
#pragma unroll
    for (int l = 0; l < L; ++l) t += (int64_t)lv[l] * ((int64_t)1 << (7 * (L - 1 - l)));
    return t;
}

// round_to_float(T, E) for T = combine_levels(lv), with the levels combined in binary64:
// Horner steps h = 128 h + lv[l] over int32 levels stay below 2^53 in magnitude up to the
// next-to-last level (|h| < 2^31 (1 + 2^7 + 2^14 + 2^21) < 2^53 for L = 5), so they are
// exact; the last step is exact when the next-to-last |h| < 2^45 (then |T| < 2^52 + 2^31).
// Scaling by 2^E is exact in binary64 when f64_scale_exact(E) (every exponent the slicing
// produces is: |E| <= 2 * 149 + 28), and the conversion to binary32 is the one IEEE rounding
// (nearest-even, subnormals, -0.0, overflow to infinity). *ok = false when a condition fails;
// the value is then meaningless and round_to_float(combine_levels(lv), E) is the result.
template <int L>
__device__ __forceinline__ float round_levels_try(const int (&lv)[L], int E, bool* ok) {
    double h = (double)lv[0];
#pragma unroll
    for (int l = 1; l + 1 < L; ++l) h = __builtin_fma(h, 128.0, (double)lv[l]);
    bool exact = repro_gemm::f64_scale_exact(E);
    if (L > 1) {
        exact = exact && __builtin_fabs(h) < 0x1p45;
        h = __builtin_fma(h, 128.0, (double)lv[L - 1]);
    }
    *ok = exact;
    return (float)__builtin_ldexp(h, E);
}

template <int L>
__device__ __forceinline__ float round_levels(const int (&lv)[L], int E) {
    bool ok;
    const float r = round_levels_try<L>(lv, E, &ok);
    return __builtin_expect(ok, 1) ? r : round_to_float_rare(combine_levels<L>(lv), E);
}

// round_to_float(T, E) for an int64 T: repro_gemm::round_to_float_f64 with its rare
// fallback out of line.
__device__ __forceinline__ float round_output(int64_t T, int E) {
    bool ok;
    const float r = repro_gemm::round_to_float_f64_try(T, E, &ok);
    return __builtin_expect(ok, 1) ? r : round_to_float_rare(T, E);
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// s_waitcnt on vector-memory operations only: wait until at most n are outstanding.
#define RG_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
// s_waitcnt on LDS (and scalar memory) operations only: wait until none is outstanding.
#define RG_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8))
// Lambdas of the kernels hold references to register arrays: they must be inlined, or the
// arrays would move to scratch memory.
#define RG_INLINE __attribute__((always_inline))
#define RG_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// Wavefronts per SIMD that the block tile's LDS ring allows (blocks per CU x wavefronts per
// block / 4), capped at 2 unless one block alone needs more (12 wavefronts: 3): the register
// budget the kernel is compiled for (at most 512 / that).
template <int S, int WTI, int WTJ, int WGM, int WGN>
constexpr int contract_waves_per_simd() {
    constexpr int lds = 3 * (WGM * WTI + WGN * WTJ) * 2 * S * PANEL_BYTES;
    constexpr int blocks = (160 * 1024) / lds;
    constexpr int need = (WGM * WGN + 3) / 4;  // one block's wavefronts per SIMD
    constexpr int w = blocks * WGM * WGN / 4;
    constexpr int cap = need > 2 ? need : 2;
    return w < need ? need : (w > cap ? cap : w);
}

template <int S, int WTI, int WTJ, int WGM, int WGN>
__global__ void __launch_bounds__(64 * WGM * WGN, (contract_waves_per_simd<S, WTI, WTJ, WGM, WGN>()))
contract_mfma(const int8_t* __restrict__ QA, const int8_t* __restrict__ QB,
              const int* __restrict__ eA, const int* __restrict__ eB, float* __restrict__ C,
              int64_t* __restrict__ partial, int M, int N, int Kp, int split, int tiles_n,
              int Mp, int Np, long long ldc, long long c_item, int xcd_chunk, int group_m) {
#if defined(__HIP_DEVICE_COMPILE__)  // buffer resources exist only in the device pass
    constexpr int L = 2 * S - 1;
    constexpr int NW = WGM * WGN;                  // wavefronts per block
    constexpr int BM = WGM * WTI * 32, BN = WGN * WTJ * 32;
    constexpr int PA = (BM / PANEL_ROWS) * 2 * S;  // A panels per stage
    constexpr int PB = (BN / PANEL_ROWS) * 2 * S;  // B panels per stage
    constexpr int PT = PA + PB;
    // Copies: with more than 4 wavefronts only wavefronts 0..3 (one per SIMD) issue the
    // stage's copies, so a SIMD's other wavefronts never stall on the address unit's command
    // queue and keep its matrix core fed while the copying one waits.
    constexpr int CW = (NW > 4 && PT % 4 == 0) ? 4 : NW;  // copying wavefronts
    constexpr int PW = PT / CW;                    // panels copied per copying wavefront per stage
    static_assert(PT % CW == 0, "stage panels must split evenly over the copying wavefronts");
    static_assert(PW < 64, "vmcnt immediate");
    // Three-stage ring, filled by direct global->LDS loads (buffer_load_dwordx4 ... lds: lane
    // i's 16 bytes land at the wavefront-uniform LDS base + 16 i, which is the panel layout).
    __shared__ v4i lds[3][PT][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    // The grid is (tiles, split, batch); which tile, part and item this block computes follows
    // the XCD-aware block order (xcd_order, block_tile), a bijection of the grid's blocks.
    int tm, tn, part, item;
    {
        const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        const int total = gridDim.x * gridDim.y * gridDim.z;
        block_tile(xcd_order(lin, total, xcd_chunk), gridDim.x / tiles_n, tiles_n, split, group_m,
                   &item, &part, &tm, &tn);
    }
    // Item of a batch: its digit panels, exponents, output and partials follow the previous
    // item's (item 0 for a single GEMM).
    QA += (size_t)item * Mp * Kp * S;
    QB += (size_t)item * Np * Kp * S;
    eA += (size_t)item * Mp;
    eB += (size_t)item * Np;
    if (C != nullptr) C += (size_t)item * c_item;
    if (partial != nullptr) partial += (size_t)item * split * M * N;
    const int nsteps = Kp / STEP_K;
    const int s0 = (int)((long long)nsteps * part / split);
    const int s1 = (int)((long long)nsteps * (part + 1) / split);
    const size_t row_stride = (size_t)(Kp / PANEL_K) * S * (PANEL_BYTES / 16);  // in v4i

    // One buffer resource per panel this wavefront copies: base = the panel at stage s0,
    // range = this part's stages, so every offset is 32-bit whatever K is and an offset out
    // of range would read zeros instead of faulting. Everything here is wavefront-uniform
    // (scalar registers); the only per-lane operand of the copies is lane * 16.
    const uint32_t step_bytes = 2u * S * PANEL_BYTES;
    const uint32_t part_bytes = (uint32_t)(s1 - s0) * step_bytes;
    const bool copier = wave < CW;
    __amdgpu_buffer_rsrc_t rsrc[PW];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        // (non-copying wavefronts never use rsrc)
        const int pi = CW == NW ? wave + NW * i : (copier ? wave + CW * i : 0);
        const int8_t* base;
        if (pi < PA) {
            const int rl = pi / (2 * S), o = pi % (2 * S);
            base = QA + ((size_t)(tm * (BM / PANEL_ROWS) + rl) * row_stride + (size_t)o * (PANEL_BYTES / 16)) * 16;
        } else {
            const int pb = pi - PA;
            const int cl = pb / (2 * S), o = pb % (2 * S);
            base = QB + ((size_t)(tn * (BN / PANEL_ROWS) + cl) * row_stride + (size_t)o * (PANEL_BYTES / 16)) * 16;
        }
        base += (size_t)s0 * step_bytes;
        rsrc[i] = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)part_bytes, 0x00020000);
    }
    const uint32_t voff = (uint32_t)lane * 16u;

    // The tile's exponents, loaded before the pipeline so that the epilogue does not wait for
    // them: lane L holds row L % (32 WTI) of this wavefront's rows (the epilogue takes each
    // row's exponent from its lane with a shuffle) and the exponents of its own columns. The
    // arrays cover the padded rows and columns, so the loads need no bounds check.
    const int e0 = -14 * (S - 1);
    int er_lane = 0;
    int ec[WTJ];
    if (partial == nullptr) {
        er_lane = eA[tm * BM + wm * WTI * 32 + lane % (WTI * 32)];
#pragma unroll
        for (int tj = 0; tj < WTJ; ++tj) ec[tj] = eB[tn * BN + (wn * WTJ + tj) * 32 + (lane & 31)] + e0;
    }

    v16i acc[L][WTI][WTJ];
#pragma unroll
    for (int l = 0; l < L; ++l)
#pragma unroll
        for (int ti = 0; ti < WTI; ++ti)
#pragma unroll
            for (int tj = 0; tj < WTJ; ++tj)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[l][ti][tj][e] = 0;

    // COPY (a std::integral_constant): whether this wavefront copies; the stage loop is
    // instantiated once for copying and once for non-copying wavefronts, so neither version
    // branches per stage.
    auto issue = [&](v4i (*slot)[64], int step, auto copy) RG_INLINE {
        if constexpr (decltype(copy)::value) {
            const uint32_t soff = (uint32_t)(step - s0) * step_bytes;
#pragma unroll
            for (int i = 0; i < PW; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc[i], RG_LDS_PTR(&slot[wave + CW * i][0]), 16,
                                                         voff, soff, 0, 0);
        }
    };
    // One stage: two k-steps of 32. Digits are read in the order a0 b0 a1 b1 ... and each
    // digit product is issued as soon as both of its digits are in registers, with the reads
    // of the next group already in flight, so a wavefront's first MFMA waits for a few
    // fragment reads rather than for the whole step. The last product group of a stage
    // (products (p, S-1) of its second k-step, operands already in registers) is issued
    // after the next stage barrier, interleaved with that stage's first reads and its copy
    // issue: deferred product (0, S-1), the opening reads, product (1, S-1), the copies into
    // the freed slot, product (2, S-1). The matrix cores start right after the barrier and
    // keep working through the reads' latency and the copy issue instead of draining. The
    // scheduling-group barriers pin the order: DS read groups (mask 0x100), VMEM groups
    // (0x020) and MFMA groups (0x008).
    v4i a[2][S][WTI], b[2][S][WTJ];
    auto load_a = [&](v4i (*slot)[64], int kk, int p) RG_INLINE {
#pragma unroll
        for (int ti = 0; ti < WTI; ++ti) a[kk][p][ti] = slot[((wm * WTI + ti) * 2 + kk) * S + p][lane];
    };
    auto load_b = [&](v4i (*slot)[64], int kk, int q) RG_INLINE {
#pragma unroll
        for (int tj = 0; tj < WTJ; ++tj) b[kk][q][tj] = slot[PA + ((wn * WTJ + tj) * 2 + kk) * S + q][lane];
    };
    auto mma = [&](int kk, int p, int q) RG_INLINE {
#pragma unroll
        for (int ti = 0; ti < WTI; ++ti)
#pragma unroll
            for (int tj = 0; tj < WTJ; ++tj)
                acc[p + q][ti][tj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                    a[kk][p][ti], b[kk][q][tj], acc[p + q][ti][tj], 0, 0, 0);
    };
    constexpr int T = WTI * WTJ;  // MFMAs per digit product
    constexpr int OPEN = WTI + WTJ + (S > 1 ? WTI : 0);
    // Reads that open a k-step: a0, b0 and (S > 1) a1.
    auto open_step = [&](v4i (*slot)[64], int kk) RG_INLINE {
        load_a(slot, kk, 0);
        load_b(slot, kk, 0);
        if (S > 1) load_a(slot, kk, 1);
    };
    // The deferred group of the previous stage: products (p, S-1) of its second k-step.
    auto tail = [&]() RG_INLINE {
#pragma unroll
        for (int p = 0; p < S; ++p) mma(1, p, S - 1);
    };
    auto compute = [&](v4i (*slot)[64], bool with_tail, v4i (*refill)[64], int s_refill, bool do_issue,
                       auto copy) RG_INLINE {
        if (with_tail) {
            mma(1, 0, S - 1);
            __builtin_amdgcn_sched_group_barrier(0x008, T, 0);
        }
        open_step(slot, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, OPEN, 0);
        if (with_tail && S > 1) {
            mma(1, 1, S - 1);
            __builtin_amdgcn_sched_group_barrier(0x008, T, 0);
        }
        if constexpr (decltype(copy)::value) {
            if (do_issue) {
                issue(refill, s_refill, copy);
                __builtin_amdgcn_sched_group_barrier(0x020, PW, 0);
            }
        }
        if (with_tail && S > 2) {
            mma(1, 2, S - 1);
            __builtin_amdgcn_sched_group_barrier(0x008, T, 0);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            if (S == 1 && kk == 1) break;  // its only product is the deferred group
            mma(kk, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, T, 0);
            if (S == 1) {
                open_step(slot, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, OPEN, 0);
            }
#pragma unroll
            for (int t = 1; t < S; ++t) {  // S <= 3: t is 1 or 2
                // digit a_t is in: products (t, q < t); meanwhile read b_t
                load_b(slot, kk, t);
                __builtin_amdgcn_sched_group_barrier(0x100, WTJ, 0);
#pragma unroll
                for (int q = 0; q < t; ++q) mma(kk, t, q);
                if (t == 1) __builtin_amdgcn_sched_group_barrier(0x008, T, 0);
                else __builtin_amdgcn_sched_group_barrier(0x008, 2 * T, 0);
                // digit b_t is in: products (p <= t, t); meanwhile read a_{t+1}, or open the
                // next k-step. The second k-step's last group is deferred (tail).
                if (t + 1 < S) {
                    load_a(slot, kk, t + 1);
                    __builtin_amdgcn_sched_group_barrier(0x100, WTI, 0);
                } else if (kk == 0) {
                    open_step(slot, 1);
                    __builtin_amdgcn_sched_group_barrier(0x100, OPEN, 0);
                }
                if (kk == 1 && t == S - 1) break;
#pragma unroll
                for (int p = 0; p <= t; ++p) mma(kk, p, t);
                if (t == 1) __builtin_amdgcn_sched_group_barrier(0x008, 2 * T, 0);
                else __builtin_amdgcn_sched_group_barrier(0x008, 3 * T, 0);
            }
        }
    };
    // Stage s: wait for this wavefront's loads of stage s (stage s+1's may stay in flight) and
    // for its reads of stage s-1 (the deferred group's operands are in registers then),
    // barrier (everyone's stage s has landed and everyone's reads of stage s-1 are done, so
    // its slot can be refilled), contract stage s, issuing stage s+2 into that slot.
    auto stage = [&](v4i (*cur)[64], v4i (*refill)[64], int s, bool do_issue, bool with_tail,
                     auto copy) RG_INLINE {
        if constexpr (decltype(copy)::value) {
            if (s + 1 < s1) RG_WAIT_VMCNT(PW);
            else RG_WAIT_VMCNT(0);
        }
        RG_WAIT_LGKMCNT0();
        // The hardware barrier, plus a compiler barrier for LDS accesses (the s_barrier
        // intrinsic alone does not keep memory operations from moving across it, and
        // __syncthreads() would also wait for the loads still in flight into other slots).
        asm volatile("s_barrier" ::: "memory");
        compute(cur, with_tail, refill, s + 2, do_issue, copy);
    };

    // The slot of stage s - 1 is the slot of stage s + 2. The first stage has nothing deferred;
    // the steady state issues and has a deferred group (no branches); the last two issue nothing.
    auto pipeline = [&](auto copy) RG_INLINE {
        if (s0 < s1) issue(lds[0], s0, copy);
        if (s0 + 1 < s1) issue(lds[1], s0 + 1, copy);
        int cur = 0, s = s0;
        auto refill = [&]() RG_INLINE { return cur == 0 ? 2 : cur - 1; };
        auto next = [&]() RG_INLINE { cur = cur == 2 ? 0 : cur + 1; ++s; };
        if (s < s1) {
            stage(lds[cur], lds[refill()], s, s + 2 < s1, false, copy);
            next();
        }
        for (; s + 2 < s1; next()) stage(lds[cur], lds[refill()], s, true, true, copy);
        for (; s < s1; next()) stage(lds[cur], lds[refill()], s, false, true, copy);
        if (s0 < s1) tail();
    };
    if constexpr (CW == NW) {
        pipeline(std::true_type());
    } else {
        if (copier) pipeline(std::true_type());
        else pipeline(std::false_type());
    }

    // Epilogue. Register e of a 32x32 accumulator tile holds row 8*(e/4) + 4*(lane/32) + e%4,
    // column lane%32.
    const int row0 = tm * BM + wm * WTI * 32 + 4 * (lane >> 5);
    const bool rows_inside = tm * BM + BM <= M;  // uniform: no row of the block is past M
    int col[WTJ];
#pragma unroll
    for (int tj = 0; tj < WTJ; ++tj) col[tj] = tn * BN + (wn * WTJ + tj) * 32 + (lane & 31);
    if (partial == nullptr) {
        const bool inside = rows_inside && tn * BN + BN <= N;  // uniform: the whole block tile
#pragma unroll
        for (int ti = 0; ti < WTI; ++ti) {
            int er[16];
#pragma unroll
            for (int e = 0; e < 16; ++e)
                er[e] = __shfl(er_lane, ti * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3), 64);
#pragma unroll
            for (int tj = 0; tj < WTJ; ++tj) {
                float* cp = C + (size_t)(row0 + ti * 32) * ldc + col[tj];
                // Four rows at a time (registers e = 4q .. 4q+3: rows 8q .. 8q+3 of the lane's
                // column), so few values are live at once.
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v[4];
                    bool all_ok = true;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        int lv[L];
#pragma unroll
                        for (int l = 0; l < L; ++l) lv[l] = acc[l][ti][tj][4 * q + i];
                        bool ok;
                        v[i] = round_levels_try<L>(lv, er[4 * q + i] + ec[tj], &ok);
                        all_ok = all_ok && ok;
                    }
                    if (__builtin_expect(!all_ok, 0)) {  // rare: these outputs exactly in int64
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            int lv[L];
#pragma unroll
                            for (int l = 0; l < L; ++l) lv[l] = acc[l][ti][tj][4 * q + i];
                            v[i] = round_to_float_rare(combine_levels<L>(lv), er[4 * q + i] + ec[tj]);
                        }
                    }
                    // Non-temporal stores: C is not read again here, and streaming it past the
                    // caches made the contraction faster (4096^3 steady state 0.466 -> 0.459 ms,
                    // 8192x3072x768 NT 0.166 -> 0.158 ms, LM-head forward -1.5%; A/B on one box).
                    if (inside) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) __builtin_nontemporal_store(v[i], &cp[(size_t)(8 * q + i) * ldc]);
                    } else if (col[tj] < N) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (rows_inside || row0 + ti * 32 + 8 * q + i < M)
                                __builtin_nontemporal_store(v[i], &cp[(size_t)(8 * q + i) * ldc]);
                    }
                    // Keep the scheduler from hoisting every accumulator read to the top.
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    } else {
#pragma unroll
        for (int ti = 0; ti < WTI; ++ti) {
#pragma unroll
            for (int tj = 0; tj < WTJ; ++tj) {
                if (col[tj] >= N) continue;
                int64_t* pp = partial + ((size_t)part * M + row0 + ti * 32) * N + col[tj];
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = 8 * (e >> 2) + (e & 3);
                    int lv[L];
#pragma unroll
                    for (int l = 0; l < L; ++l) lv[l] = acc[l][ti][tj][e];
                    if (rows_inside || row0 + ti * 32 + r < M) pp[(size_t)r * N] = combine_levels<L>(lv);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#endif
}

// One-launch GEMM for small shapes (K <= SMALL_MAX_K): a block of 16 wavefronts owns a 32x32
// tile of C and does every step of the definition for it. Its 32 rows of op(A) and 32 columns
// of op(B) are cut into slots of 16 consecutive k of one row (the 16 bytes one lane contributes
// to a digit panel); each thread loads its slots' values into registers at once (one memory
// latency for the block), takes their maxima into the rows' maxima (LDS atomics on the
// non-negative floats' bit patterns, which order as the values do), and after the exponents
// rounds them to fixed point and writes their digits into LDS panels. Wavefront w < 4 contracts
// k panels w, w + 4, ... with V_MFMA_I32_32X32X32_I8; the four wavefronts' level sums are added
// in LDS and every output is rounded once. Sixteen wavefronts (four per SIMD) keep the code
// short (two slots per thread) and hide the latency of the rounding's dependent instructions. Neighbouring tiles round the same rows again; for
// shapes this small that costs less than the slicing launch it replaces. The values and integer
// sums are the pipeline's, so are the bits.
// Operand o (0: op(A), row r = tile row; 1: op(B), row r = tile column) has element (r, k) at
// src[r * ld + k] (row access) or src[k * ld + r] (strided); vec: row access with 16-byte
// aligned rows and K % 4 == 0.
struct SmallOperand {
    const float* src;
    long long ld;
    int R;        // rows of op(X) (M or N)
    int strided;
    int vec;
};

constexpr int SMALL_SLOTS = 2 * (SMALL_MAX_K / PANEL_K) * 64 / SMALL_THREADS;  // per thread, at most

template <int S>
struct SmallLds {
    static constexpr int PANELS = 2 * S * (SMALL_MAX_K / PANEL_K);  // digit panels of both operands
    static constexpr int RED = 4 * (2 * S - 1) * 16;                 // 64-lane int rows of the sums
    static constexpr int V4 = (PANELS * 64 > RED * 16 ? PANELS * 64 : RED * 16);  // in v4i
};

template <int S>
__global__ void __launch_bounds__(SMALL_THREADS, 1)
contract_small(SmallOperand a, SmallOperand b, float* __restrict__ C, int K, long long ldc,
               long long stride_a, long long stride_b, long long stride_c, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int L = 2 * S - 1;
    __shared__ v4i buf[SmallLds<S>::V4];
    __shared__ int rmax[2][32];   // bit patterns of the rows' maxima
    __shared__ int sexp[2][32];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int npk = (K + PANEL_K - 1) / PANEL_K;
    const int slots = 2 * npk * 64;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
    const int item = blockIdx.z;
    a.src += (size_t)item * stride_a;
    b.src += (size_t)item * stride_b;
    C += (size_t)item * stride_c;
    const int r0[2] = {tm * 32, tn * 32};
    if (t < 64) rmax[t >> 5][t & 31] = 0;
    __syncthreads();

    // Slot i = t + SMALL_THREADS j: operand o = i / (64 npk), k panel kp, lane s of the panel: row s % 32,
    // k = 32 kp + 16 (s / 32) .. + 15. Every load of every slot is issued before any is used.
    float x[SMALL_SLOTS][16];
#pragma unroll
    for (int j = 0; j < SMALL_SLOTS; ++j) {
        const int i = t + SMALL_THREADS * j;
        const int o = i >= npk * 64 ? 1 : 0;
        const int rem = i - o * npk * 64;
        const int kp = rem >> 6, s = rem & 63;
        const int r = r0[o] + (s & 31), k0 = kp * PANEL_K + 16 * (s >> 5);
        const SmallOperand& op = o == 0 ? a : b;
        const bool live = i < slots && r < op.R;
        if (live && op.vec) {
            const float4* p = reinterpret_cast<const float4*>(op.src + (size_t)r * op.ld + k0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (k0 + 4 * q < K) v = p[q];  // K % 4 == 0: a float4 is wholly in or out
                x[j][4 * q] = v.x;
                x[j][4 * q + 1] = v.y;
                x[j][4 * q + 2] = v.z;
                x[j][4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int k = k0 + e;
                x[j][e] = 0.0f;
                if (live && k < K)
                    x[j][e] = op.strided ? op.src[(size_t)k * op.ld + r] : op.src[(size_t)r * op.ld + k];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < SMALL_SLOTS; ++j) {
        const int i = t + SMALL_THREADS * j;
        if (i < slots) {
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(x[j][e]));
            const int o = i >= npk * 64 ? 1 : 0;
            atomicMax(&rmax[o][(i - o * npk * 64) & 31], __float_as_int(m));
        }
    }
    __syncthreads();
    if (t < 64) {
        const float m = __int_as_float(rmax[t >> 5][t & 31]);
        sexp[t >> 5][t & 31] = repro_gemm::scale_exponent(m);  // rows past R: m == 0, exponent 0
    }
    __syncthreads();

    // Digits of every slot into the panels: buf[((o S + p) npk + kp) 64 + s].
#pragma unroll
    for (int j = 0; j < SMALL_SLOTS; ++j) {
        const int i = t + SMALL_THREADS * j;
        if (i < slots) {
            const int o = i >= npk * 64 ? 1 : 0;
            const int rem = i - o * npk * 64;
            const int kp = rem >> 6, s = rem & 63;
            const RowScale rs = row_scale<S>(sexp[o][s & 31]);
            int dg[S][16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                int d[S];
                digits_of<S>(round_fixed(x[j][e], rs), d);
#pragma unroll
                for (int p = 0; p < S; ++p) dg[p][e] = d[p];
            }
#pragma unroll
            for (int p = 0; p < S; ++p) {
                v4i w;
                w[0] = (int)pack4(dg[p][0], dg[p][1], dg[p][2], dg[p][3]);
                w[1] = (int)pack4(dg[p][4], dg[p][5], dg[p][6], dg[p][7]);
                w[2] = (int)pack4(dg[p][8], dg[p][9], dg[p][10], dg[p][11]);
                w[3] = (int)pack4(dg[p][12], dg[p][13], dg[p][14], dg[p][15]);
                buf[((o * S + p) * npk + kp) * 64 + s] = w;
            }
        }
    }
    __syncthreads();

    v16i acc[L];
#pragma unroll
    for (int l = 0; l < L; ++l)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[l][e] = 0;
    for (int kp = wave; kp < npk && wave < 4; kp += 4) {
        v4i fa[S], fb[S];
#pragma unroll
        for (int p = 0; p < S; ++p) {
            fa[p] = buf[(p * npk + kp) * 64 + lane];
            fb[p] = buf[((S + p) * npk + kp) * 64 + lane];
        }
#pragma unroll
        for (int p = 0; p < S; ++p)
#pragma unroll
            for (int q = 0; q < S; ++q)
                acc[p + q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[p], fb[q], acc[p + q], 0, 0, 0);
    }
    __syncthreads();  // every panel read: the buffer now takes the level sums
    int* red = reinterpret_cast<int*>(buf);
    if (wave < 4) {
#pragma unroll
        for (int l = 0; l < L; ++l)
#pragma unroll
            for (int e = 0; e < 16; ++e) red[((wave * L + l) * 16 + e) * 64 + lane] = acc[l][e];
    }
    __syncthreads();
    // Output slot (e, l): accumulator register e of lane l, i.e. row 8 (e / 4) + 4 (l / 32) + e % 4,
    // column l % 32 of the tile.
    const int e0 = -14 * (S - 1);
    {
        const int i = t;  // one output per thread
        const int e = i >> 6, ln = i & 63;
        const int row = 8 * (e >> 2) + 4 * (ln >> 5) + (e & 3), col = ln & 31;
        const int gr = r0[0] + row, gc = r0[1] + col;
        if (gr >= a.R || gc >= b.R) return;
        int lv[L];
#pragma unroll
        for (int l = 0; l < L; ++l) {
            int v = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) v += red[((w * L + l) * 16 + e) * 64 + ln];
            lv[l] = v;
        }
        C[(size_t)gr * ldc + gc] = round_levels<L>(lv, sexp[0][row] + sexp[1][col] + e0);
    }
#endif
}

// Band kernel, for op(A) read along rows with K <= BAND_MAX_K and many rows (the GPT-2 layers'
// forward and input-gradient GEMMs at K = 768). Block (band, g) owns the 32 rows
// [32 band, 32 band + 32) of op(A) and the output columns [g W, (g + 1) W). It slices its rows
// itself, as the one-pass slicing does (every value loaded once into registers, the rows'
// maxima in LDS, scale_exponent, rounding, bit-field digits), into digit panels in LDS, where
// they stay for the rest of the launch. op(B)'s digit panels (sliced by the launch before) are
// streamed from the caches straight into registers, D steps ahead: wavefront w takes the block's
// column tiles w, w + 8, ..., contracts each 32x32 tile over all of K with
// V_MFMA_I32_32X32X32_I8 (the digit pairs of one level in one int32 accumulator, as in
// contract_mfma) and rounds and stores it as soon as its last k panel is done. Against slicing
// op(A) in a launch of its own and contracting 64x64 tiles in three rounds of blocks, the digits
// of op(A) never go through memory and the GEMM is one round of blocks (one per compute unit).
// The values, the integer sums and the rounding are the pipeline's, so are the bits.
// The loads of op(B) go through a buffer resource over its digit region, so an offset out of
// the region would read zeros instead of faulting.
template <int S, int NSL>
__global__ void __launch_bounds__(BAND_THREADS, BAND_THREADS / 256)
contract_band(const float* __restrict__ A, long long lda, int vec_a, const int8_t* __restrict__ QB,
              int qb_bytes, const int* __restrict__ eB, float* __restrict__ C, long long ldc,
              int M, int N, int K, int Kp_ws, int W, int groups) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int L = 2 * S - 1;
    constexpr int D = BAND_DEPTH;
    __shared__ v4i band[(BAND_MAX_K / PANEL_K) * S][64];  // [k panel * S + digit][lane]
    __shared__ int rmax[32];  // bit patterns of the rows' maxima (non-negative floats)
    __shared__ int sexp[32];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    // Workgroup i runs on XCD i mod 8: with groups dividing 8, an XCD streams one column group.
    const int g = blockIdx.x % groups, bnd = blockIdx.x / groups;
    const int r0 = bnd * 32;
    const int nkp = (K + PANEL_K - 1) / PANEL_K;  // k panels holding some k < K
    const int npk_ws = Kp_ws / PANEL_K;           // k panels per 32-column panel of QB
    const int ntile = W / 32;
    const int tc0 = g * ntile;                    // first column tile of the block
    constexpr int NW = BAND_THREADS / 64;        // wavefronts per block
    const int my_tiles = ntile > wave ? (ntile - wave + NW - 1) / NW : 0;
    const int total = my_tiles * nkp;             // (tile, k panel) steps of this wavefront
    auto tile_of = [&](int j) RG_INLINE { return tc0 + wave + NW * j; };

    // op(B)'s panels of this wavefront's steps, fetched D steps ahead, in step order.
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)QB, (short)0, qb_bytes, 0x00020000);
    const uint32_t voff = (uint32_t)lane * 16u;
    int pj = 0, pk = 0;  // next (tile of this wavefront, k panel) to fetch
    auto fetch = [&](v4i (&buf)[S]) RG_INLINE {
        const uint32_t base =
            (uint32_t)((tile_of(pj) * npk_ws + pk) * S) * (uint32_t)PANEL_BYTES;
#pragma unroll
        for (int q = 0; q < S; ++q)
            buf[q] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, base + q * PANEL_BYTES, 0);
        if (++pk == nkp) {
            pk = 0;
            ++pj;
        }
    };
    v4i bq[D][S];
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (d < total) fetch(bq[d]);
    int ec = 0;  // column exponent (lane % 32) of the current tile
    if (total > 0) ec = eB[tile_of(0) * 32 + (lane & 31)];

    // Slicing of the band: slot i = t + BAND_THREADS j is lane s = i % 64 of k panel i / 64,
    // i.e. row s % 32 and k = 32 (i / 64) + 16 (s / 32) .. + 15. Every load is issued first.
    if (t < 32) rmax[t] = 0;
    __syncthreads();
    float x[NSL][16];
#pragma unroll
    for (int j = 0; j < NSL; ++j) {
        const int i = t + BAND_THREADS * j;
        const int kp = i >> 6, s = i & 63;
        const int r = r0 + (s & 31), k0 = kp * PANEL_K + 16 * (s >> 5);
        const bool live = kp < nkp && r < M;
        const float* row = A + (size_t)r * lda;
        if (live && vec_a) {
            const float4* p = reinterpret_cast<const float4*>(row + k0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (k0 + 4 * q < K) v = p[q];  // K % 4 == 0: a float4 is wholly in or out
                x[j][4 * q] = v.x;
                x[j][4 * q + 1] = v.y;
                x[j][4 * q + 2] = v.z;
                x[j][4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) x[j][e] = (live && k0 + e < K) ? row[k0 + e] : 0.0f;
        }
    }
#pragma unroll
    for (int j = 0; j < NSL; ++j) {
        const int i = t + BAND_THREADS * j;
        if ((i >> 6) < nkp) {
            float m = 0.0f;  // the maximum skips NaN (fmaxf), as the definition's CPU path does
#pragma unroll
            for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(x[j][e]));
            atomicMax(&rmax[i & 31], __float_as_int(m));
        }
    }
    __syncthreads();
    if (t < 32) sexp[t] = repro_gemm::scale_exponent(__int_as_float(rmax[t]));  // rows past M: 0
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NSL; ++j) {
        const int i = t + BAND_THREADS * j;
        const int kp = i >> 6, s = i & 63;
        if (kp < nkp) {
            const RowScale rs = row_scale<S>(sexp[s & 31]);
            int dg[S][16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                int dd[S];
                digits_of<S>(round_fixed(x[j][e], rs), dd);
#pragma unroll
                for (int p = 0; p < S; ++p) dg[p][e] = dd[p];
            }
#pragma unroll
            for (int p = 0; p < S; ++p) {
                v4i w;
                w[0] = (int)pack4(dg[p][0], dg[p][1], dg[p][2], dg[p][3]);
                w[1] = (int)pack4(dg[p][4], dg[p][5], dg[p][6], dg[p][7]);
                w[2] = (int)pack4(dg[p][8], dg[p][9], dg[p][10], dg[p][11]);
                w[3] = (int)pack4(dg[p][12], dg[p][13], dg[p][14], dg[p][15]);
                band[kp * S + p][s] = w;
            }
        }
    }
    __syncthreads();

    // Exponents of this lane's output rows: register e of a 32x32 accumulator tile holds row
    // 8 (e / 4) + 4 (lane / 32) + e % 4, column lane % 32.
    const int e0 = -14 * (S - 1);
    int er[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) er[e] = sexp[8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)] + e0;

    v16i acc[L];
    int jt = 0, ks = 0;  // current tile of this wavefront, k panel
    auto epilogue = [&]() RG_INLINE {
        const int col = tile_of(jt) * 32 + (lane & 31);
        const int rbase = r0 + 4 * (lane >> 5);
        float* cp = C + (size_t)rbase * ldc + col;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v[4];
            bool all_ok = true;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int lv[L];
#pragma unroll
                for (int l = 0; l < L; ++l) lv[l] = acc[l][4 * q + i];
                bool ok;
                v[i] = round_levels_try<L>(lv, er[4 * q + i] + ec, &ok);
                all_ok = all_ok && ok;
            }
            if (__builtin_expect(!all_ok, 0)) {  // rare: these outputs exactly in int64
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    int lv[L];
#pragma unroll
                    for (int l = 0; l < L; ++l) lv[l] = acc[l][4 * q + i];
                    v[i] = round_to_float_rare(combine_levels<L>(lv), er[4 * q + i] + ec);
                }
            }
            if (col < N) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (rbase + 8 * q + i < M)
                        __builtin_nontemporal_store(v[i], &cp[(size_t)(8 * q + i) * ldc]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto step = [&](v4i (&buf)[S], int it) RG_INLINE {
        if (ks == 0) {
#pragma unroll
            for (int l = 0; l < L; ++l)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[l][e] = 0;
        }
        v4i fa[S];
#pragma unroll
        for (int p = 0; p < S; ++p) fa[p] = band[ks * S + p][lane];
#pragma unroll
        for (int p = 0; p < S; ++p)
#pragma unroll
            for (int q = 0; q < S; ++q)
                acc[p + q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[p], buf[q], acc[p + q], 0, 0, 0);
        if (it + D < total) fetch(buf);
        if (++ks == nkp) {
            epilogue();
            ks = 0;
            ++jt;
            if (jt < my_tiles) ec = eB[tile_of(jt) * 32 + (lane & 31)];
        }
    };
    for (int it = 0; it < total; it += D) {
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (it + d < total) step(bq[d], it + d);
    }
#endif
}

// The definition, as plainly as possible: one thread per output, int64 sum of X * Y over
// this part's share of k. Always writes an int64 partial.
__global__ void __launch_bounds__(256)
contract_reference(const int32_t* __restrict__ X, const int32_t* __restrict__ Y,
                   int64_t* __restrict__ partial, int M, int N, int K, int Kp, int split, int Mp,
                   int Np) {
    const int c = blockIdx.x * 16 + (threadIdx.x & 15);
    const int r = blockIdx.y * 16 + (threadIdx.x >> 4);
    const int part = blockIdx.z % split, item = blockIdx.z / split;
    if (r >= M || c >= N) return;
    const int k0 = (int)((long long)K * part / split);
    const int k1 = (int)((long long)K * (part + 1) / split);
    const int32_t* x = X + ((size_t)item * Mp + r) * Kp;
    const int32_t* y = Y + ((size_t)item * Np + c) * Kp;
    int64_t t = 0;
    for (int k = k0; k < k1; ++k) t += (int64_t)x[k] * y[k];
    partial[(((size_t)item * split + part) * M + r) * N + c] = t;
}

// Sums the split partials in int64 (order irrelevant: exact) and rounds once. TPO threads share
// an output: each sums every TPO-th part, and the block adds their sums in LDS, so that a few
// outputs with many parts (a long K over a small M x N) still spread over the GPU instead of
// leaving one thread a long chain of dependent loads. Consecutive threads take consecutive
// outputs, so every load instruction reads consecutive int64 partials.
// RU: loads of a thread's parts in flight at once (1: one at a time).
template <int TPO, int RU>
__global__ void __launch_bounds__(256)
reduce_round(const int64_t* __restrict__ partial, const int* __restrict__ eA,
             const int* __restrict__ eB, float* __restrict__ C, int M, int N, int split, int e0,
             int batch, int Mp, int Np, long long ldc, long long c_item) {
    constexpr int OPB = 256 / TPO;  // outputs per block
    const int t = threadIdx.x;
    const int ol = t % OPB, sub = t / OPB;
    const size_t idx = (size_t)blockIdx.x * OPB + ol;
    const size_t MN = (size_t)M * N;
    const bool live = idx < MN * batch;
    int item = 0, r = 0, c = 0, ea = 0, eb = 0;
    size_t rc = 0;
    int64_t acc = 0;
    if (live) {
        item = (int)(idx / MN);
        rc = idx - (size_t)item * MN;
        if (sub == 0) {  // the output's exponents, loaded along with its partials, used after
            r = (int)(rc / N);
            c = (int)(rc % N);
            ea = eA[(size_t)item * Mp + r];
            eb = eB[(size_t)item * Np + c];
        }
        const int64_t* p0 = partial + (size_t)item * split * MN + rc;
        for (int p = sub; p < split; p += TPO * RU) {
            int64_t v[RU];
#pragma unroll
            for (int u = 0; u < RU; ++u)
                v[u] = p + u * TPO < split ? p0[(size_t)(p + u * TPO) * MN] : 0;
#pragma unroll
            for (int u = 0; u < RU; ++u) acc += v[u];
        }
    }
    if (TPO > 1) {
        __shared__ int64_t red[256];
        red[t] = acc;
#pragma unroll
        for (int s = TPO / 2; s >= 1; s >>= 1) {
            __syncthreads();
            if (sub < s) red[t] += red[t + s * OPB];
        }
        acc = red[t];  // complete for sub == 0, which wrote it last
    }
    if (live && sub == 0)
        C[(size_t)item * c_item + (size_t)r * ldc + c] = round_output(acc, ea + eb + e0);
}

// Test hooks: the epilogue roundings on arrays. levels: n x (2S-1) int32, most significant
// level first.
template <int L>
__global__ void __launch_bounds__(256)
round_levels_kernel(const int* __restrict__ lv, const int* __restrict__ E, float* __restrict__ out,
                    long long n) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    int v[L];
#pragma unroll
    for (int l = 0; l < L; ++l) v[l] = lv[i * L + l];
    out[i] = round_levels<L>(v, E[i]);
}

__global__ void __launch_bounds__(256)
round_output_kernel(const int64_t* __restrict__ T, const int* __restrict__ E,
                    float* __restrict__ out, long long n) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = round_output(T[i], E[i]);
}

void launch_test_round(const int* levels, const int64_t* T, const int* E, float* out, long long n,
                       int S, hipStream_t stream) {
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (levels == nullptr) round_output_kernel<<<blocks, 256, 0, stream>>>(T, E, out, n);
    else if (S == 1) round_levels_kernel<1><<<blocks, 256, 0, stream>>>(levels, E, out, n);
    else if (S == 2) round_levels_kernel<3><<<blocks, 256, 0, stream>>>(levels, E, out, n);
    else round_levels_kernel<5><<<blocks, 256, 0, stream>>>(levels, E, out, n);
}

template <int S>
static void launch_mfma_s(const Layout& L, const int8_t* qa, const int8_t* qb, const int* ea,
                          const int* eb, float* C, OutAddr out, int64_t* partial,
                          hipStream_t stream) {
    const int tiles_m = L.Mp / (64 * L.ti), tiles_n = L.Np / (64 * L.tj);
    dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)L.split, (unsigned)L.batch);
    // Block tiles: 128x128 = 8 wavefronts of 64x32; 128x64 and 64x128 = 8 wavefronts of 32x32
    // (two per SIMD); 64x64 = 4 wavefronts of 32x32; 64x192 and 192x64 = 12 wavefronts of
    // 32x32 (three per SIMD).
#define RG_CONTRACT_ARGS qa, qb, ea, eb, C, partial, L.M, L.N, L.Kp, L.split, tiles_n, L.Mp, L.Np, \
                         out.ldc, out.c_item, L.xcd_chunk, L.group_m
    // (The twelve-wavefront tiles exist for S = 3 only: their 48 stage panels split evenly over
    // 12 wavefronts; the planner never gives them to S < 3.)
    if constexpr (S == 3) {
        if (L.ti == 1 && L.tj == 3) {
            contract_mfma<S, 1, 1, 2, 6><<<grid, 768, 0, stream>>>(RG_CONTRACT_ARGS);
            return;
        }
        if (L.ti == 3 && L.tj == 1) {
            contract_mfma<S, 1, 1, 6, 2><<<grid, 768, 0, stream>>>(RG_CONTRACT_ARGS);
            return;
        }
    }
    if (L.ti == 2 && L.tj == 2)
        contract_mfma<S, 2, 1, 2, 4><<<grid, 512, 0, stream>>>(RG_CONTRACT_ARGS);
    else if (L.ti == 2 && L.tj == 1)
        contract_mfma<S, 1, 1, 4, 2><<<grid, 512, 0, stream>>>(RG_CONTRACT_ARGS);
    else if (L.ti == 1 && L.tj == 2)
        contract_mfma<S, 1, 1, 2, 4><<<grid, 512, 0, stream>>>(RG_CONTRACT_ARGS);
    else
        contract_mfma<S, 1, 1, 2, 2><<<grid, 256, 0, stream>>>(RG_CONTRACT_ARGS);
#undef RG_CONTRACT_ARGS
}

void launch_contract_mfma(const Layout& L, const int8_t* qa, const int8_t* qb, const int* ea,
                          const int* eb, float* C, OutAddr out, int64_t* partial,
                          hipStream_t stream) {
    switch (L.S) {
        case 1: launch_mfma_s<1>(L, qa, qb, ea, eb, C, out, partial, stream); break;
        case 2: launch_mfma_s<2>(L, qa, qb, ea, eb, C, out, partial, stream); break;
        case 3: launch_mfma_s<3>(L, qa, qb, ea, eb, C, out, partial, stream); break;
        default: break;
    }
}

void launch_contract_small(const Layout& L, const float* A, const float* B, float* C,
                           const GemmAddressing& addr, hipStream_t stream) {
    const int tiles_m = (L.M + 31) / 32, tiles_n = (L.N + 31) / 32;
    // 16-byte loads for a row-access operand whose rows (and items) start 16-byte aligned
    auto vec = [&](const float* p, long long ld, long long stride, bool strided) {
        return !strided && (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 4 == 0 &&
               (L.batch == 1 || stride % 4 == 0) && L.K % 4 == 0;
    };
    const SmallOperand a{A, addr.lda, L.M, L.a_strided ? 1 : 0,
                         vec(A, addr.lda, addr.stride_a, L.a_strided) ? 1 : 0};
    const SmallOperand b{B, addr.ldb, L.N, L.b_strided ? 1 : 0,
                         vec(B, addr.ldb, addr.stride_b, L.b_strided) ? 1 : 0};
    const dim3 grid((unsigned)(tiles_m * tiles_n), 1, (unsigned)L.batch);
#define RG_SMALL(SS)                                                                            \
    contract_small<SS><<<grid, SMALL_THREADS, 0, stream>>>(a, b, C, L.K, addr.ldc, addr.stride_a, \
                                                 addr.stride_b, addr.stride_c, tiles_n)
    switch (L.S) {
        case 1: RG_SMALL(1); break;
        case 2: RG_SMALL(2); break;
        case 3: RG_SMALL(3); break;
        default: break;
    }
#undef RG_SMALL
}

void launch_contract_band(const Layout& L, const float* A, long long lda, const int8_t* qb,
                          const int* eb, float* C, long long ldc, hipStream_t stream) {
    // 16-byte loads for rows that start 16-byte aligned with K % 4 == 0
    const int vec_a = (reinterpret_cast<uintptr_t>(A) & 15) == 0 && lda % 4 == 0 && L.K % 4 == 0;
    const int nkp = (L.K + PANEL_K - 1) / PANEL_K;
    const int nsl = (nkp * 64 + BAND_THREADS - 1) / BAND_THREADS;  // slots per thread, <= 4
    const int qb_bytes = (int)((size_t)L.Np * L.Kp * L.S);  // < 2^31 (plan_layout)
    const unsigned blocks = (unsigned)((L.Mp / 32) * L.band_groups);
#define RG_BAND(SS, NS)                                                                         \
    contract_band<SS, NS><<<blocks, BAND_THREADS, 0, stream>>>(A, lda, vec_a, qb, qb_bytes, eb,  \
                                                              C, ldc, L.M, L.N, L.K, L.Kp,      \
                                                              L.band_w, L.band_groups)
#define RG_BAND_S(SS)                       \
    switch (nsl) {                          \
        case 1: RG_BAND(SS, 1); break;      \
        case 2: RG_BAND(SS, 2); break;      \
        case 3: RG_BAND(SS, 3); break;      \
        default: RG_BAND(SS, 4); break;     \
    }
    switch (L.S) {
        case 1: RG_BAND_S(1); break;
        case 2: RG_BAND_S(2); break;
        case 3: RG_BAND_S(3); break;
        default: break;
    }
#undef RG_BAND_S
#undef RG_BAND
}

void launch_contract_reference(const Layout& L, const int32_t* xa, const int32_t* xb,
                               int64_t* partial, hipStream_t stream) {
    dim3 grid((unsigned)((L.N + 15) / 16), (unsigned)((L.M + 15) / 16),
              (unsigned)(L.split * L.batch));
    contract_reference<<<grid, 256, 0, stream>>>(xa, xb, partial, L.M, L.N, L.K, L.Kp, L.split,
                                                 L.Mp, L.Np);
}

void launch_reduce_round(const Layout& L, const int64_t* partial, const int* ea, const int* eb,
                         float* C, OutAddr out, hipStream_t stream) {
    const size_t total = (size_t)L.M * L.N * L.batch;
    // Threads per output: enough for about 2^18 threads in all, at most 256, no more than the
    // parts.
    int tpo = 1;
    while (tpo < 256 && tpo < L.split && total * tpo < ((size_t)1 << 18)) tpo *= 4;
    const unsigned blocks = (unsigned)((total * tpo + 255) / 256);
    // Below 2^20 threads the reduction is latency-bound: each thread issues up to eight of its
    // parts' loads at once (the one-at-a-time loop paid one memory latency per part; reduction
    // stage, one box: 768x768x8192 split 5 9.7 -> 8.6 us, 512x512x16384 split 8 7.8 -> 6.9 us).
    // Above, one load at a time keeps the memory streams in order (1024x1024x65536 split 4:
    // 0.3 us slower with eight).
    const bool many = total * tpo < ((size_t)1 << 20);
#define RG_REDUCE(T)                                                                              \
    (many ? reduce_round<T, 8><<<blocks, 256, 0, stream>>>(partial, ea, eb, C, L.M, L.N, L.split,  \
                                                           -14 * (L.S - 1), L.batch, L.Mp, L.Np, \
                                                           out.ldc, out.c_item)                 \
          : reduce_round<T, 1><<<blocks, 256, 0, stream>>>(partial, ea, eb, C, L.M, L.N, L.split,  \
                                                           -14 * (L.S - 1), L.batch, L.Mp, L.Np, \
                                                           out.ldc, out.c_item))
    switch (tpo) {
        case 1: RG_REDUCE(1); break;
        case 4: RG_REDUCE(4); break;
        case 16: RG_REDUCE(16); break;
        case 64: RG_REDUCE(64); break;
        default: RG_REDUCE(256); break;
    }
#undef RG_REDUCE
}

}  // namespace rg
