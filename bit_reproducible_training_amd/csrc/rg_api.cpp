// Host side of librepro_gemm.so: planner, workspace layout, launch sequence and the flat
// C ABI declared in include/repro_gemm.h.
//
// Replaces make_layout / make_plan / launch_quantize / launch_all / repro_gemm_fp32_ws /
// repro_gemm_fp32 / algo_name (repro_gemm_cuda/repro_gemm.cu:370-542). Stateless apart
// from a per-device cache of (architecture, compute-unit count); every entry point is
// re-entrant and stream-ordered.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "repro_gemm.h"
#include "rg_internal.h"

namespace rg {
namespace {

constexpr size_t ALIGN = 256;
size_t align_up(size_t x) { return (x + ALIGN - 1) / ALIGN * ALIGN; }
int round_up(int x, int m) { return (x + m - 1) / m * m; }
int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

// Largest |X| the bound check assumes, as the reference defines it
// (repro_gemm_cuda/repro_gemm.cu:383-388): 127*128^(S-1) + 64*(128^(S-2) + ... + 1).
double max_fixed_point(int S) {
    double top = 127.0 * std::ldexp(1.0, 7 * (S - 1)), low = 0.0;
    for (int t = 0; t < S - 1; ++t) low += 64.0 * std::ldexp(1.0, 7 * t);
    return top + low;
}

// Largest |sum over one k of the digit products that share a level|, for the digits the
// slicing writes (|d0| <= 127, lower digits in [0, 127]; every product at most 127*127 = 16129
// in magnitude): S=1: one product; S=2: level 1 has two; S=3: level 2 has three.
int level_bound_per_k(int S) { return S == 1 ? 16129 : (S == 2 ? 32258 : 48387); }

// Stages (of STEP_K values of k) one part may span with every int32 level sum exact.
int max_steps_per_part(int S) {
    long long n = 2147483647LL / level_bound_per_k(S);
    return (int)(n / STEP_K);
}

// Row-max pass chunking, from shapes only (so the workspace size never depends on pointer
// alignment): enough blocks to keep HBM busy, at most 16 (row access) or 32 (column access)
// partial maxima per row, chunk lengths a multiple of 4 for float4 loads. Column-access
// operands of at most 32 columns per item (read as whole rows, few blocks per chunk), and long
// columns over few column groups, take up to 256 chunks of at least 256 k. R is the item's
// row count, rows all items' rows.
void choose_chunks(int R, int rows, int K, bool strided, int* nch, int* kch) {
    int n;
    if (strided && R <= 32) {
        n = std::min(256, ceil_div(K, 256));
    } else if (strided) {
        int groups = ceil_div(rows, rows % 4 == 0 ? 256 : 64);
        n = std::min(ceil_div(1024, groups), std::min(32, ceil_div(K, 16)));
        // A long K over few column groups (a convolution's weight gradient: 576 positions
        // over 100352 windows) needs more chunks to give the pass enough blocks.
        n = std::max(n, std::min(ceil_div(1024, groups), std::min(256, ceil_div(K, 256))));
    } else {
        n = std::min(ceil_div(2048, rows), std::min(16, ceil_div(K, 256)));
    }
    n = std::max(1, n);
    *kch = round_up(ceil_div(K, n), 4);
    *nch = ceil_div(K, *kch);
}

// Estimated contraction time (microseconds) of one block-tile / split choice, used only to
// choose between plans (any choice gives the same bits). Blocks run in waves over the GPU's
// block slots (compute units x blocks resident per compute unit, from the block's LDS ring);
// a block costs a fixed prologue/epilogue plus one pipeline stage per 64 values of k of its
// part; a split adds the int64 partials' traffic (written once, read once) at about 4 TB/s.
// The per-tile constants (S = 3) were chosen so that the planner picks the fastest measured plan
// on a sweep of every block tile x split over 22 shapes on MI355X (the GEMMs of BASELINE
// configurations 3 and 5, squares, tall and long-K shapes; the GPU brought out of idle first):
// 21 of the 22 picks are the fastest measured plan, the other within 5.9% of it. The
// stage time's MFMA part scales with S^2 for fewer slices.
// Blocks of one MFMA tile resident per compute unit: the LDS ring (3 stages of the block's
// digit panels) against 160 KiB, at most 2.
int blocks_per_cu(int ti, int tj, int S) {
    const int lds_bytes = 3 * (2 * ti + 2 * tj) * 2 * S * PANEL_BYTES;
    return std::max(1, std::min(2, (160 * 1024) / lds_bytes));
}

// Tile rows per group of the contraction's block order (block_tile): the power of two that
// keeps the digit panels touched by one XCD's run of `chunk` consecutive tiles (row panels of
// 64 ti rows, column panels of 64 tj columns) fewest. A run from the start of a group covers
// that group column by column, then the next group.
int group_rows(int chunk, int ti, int tj, int tiles_m, int tiles_n) {
    int best_g = 1;
    long long best = -1;
    for (int g = 1; g <= tiles_m; g *= 2) {
        long long left = std::min<long long>(chunk, (long long)tiles_m * tiles_n);
        long long rows = 0, cols = 0;
        for (int r0 = 0; r0 < tiles_m && left > 0; r0 += g) {
            const int gr = std::min(g, tiles_m - r0);
            const long long here = std::min<long long>(left, (long long)gr * tiles_n);
            rows += std::min<long long>(gr, here);
            cols = std::max<long long>(cols, (here + gr - 1) / gr);
            left -= here;
        }
        const long long panels = rows * ti + cols * tj;
        if (best < 0 || panels < best) {
            best = panels;
            best_g = g;
        }
    }
    return best_g;
}

double plan_cost(int M, int N, int nsteps, int batch, int ti, int tj, int split, int S,
                 int num_cus, bool raw) {
    const double tiles = (double)ceil_div(M, 64 * ti) * ceil_div(N, 64 * tj) * batch;
    const int per_cu = blocks_per_cu(ti, tj, S);
    const double slots = (double)std::max(1, num_cus) * per_cu;
    const double waves = std::ceil(tiles * split / slots);
    // per block wave at S = 3: 128x128 (8 wavefronts, one block per CU), 64x64 (4 wavefronts,
    // two per CU), 64x192 and 192x64 (12 wavefronts), 128x64 and 64x128 (8 wavefronts of 32x32)
    double stage3 = 0.8, fixed_us = 3.0;
    if (ti == 2 && tj == 2) {
        stage3 = 1.276;
        fixed_us = 8.5;
    } else if (ti == 1 && tj == 1) {
        stage3 = 0.803;
        fixed_us = 3.0;
    } else if (ti * tj == 3) {
        stage3 = 0.978;
        fixed_us = 9.66;
    } else if (ti * tj == 2) {
        stage3 = 0.704;
        fixed_us = 8.5;
    }
    const double stage_us = 0.1 + (stage3 - 0.1) * (S * S / 9.0);
    const double steps = std::ceil((double)nsteps / split);
    double t = waves * (steps * stage_us + fixed_us);
    if (split > 1 || raw) {
        const double outs = (double)M * N * batch;
        t += 3.0 + (8.0 * outs * (split + 1) + 4.0 * outs) / 4.0e6;
    }
    return t;
}

// Block tiles a caller may pin through Config.tile_m / tile_n: 64 or 128 by 64 or 128, and (at
// S = 3) the twelve-wavefront 64x192 and 192x64.
bool pinned_tile(int tile_m, int tile_n, int S) {
    if ((tile_m == 64 || tile_m == 128) && (tile_n == 64 || tile_n == 128)) return true;
    return S == 3 && ((tile_m == 64 && tile_n == 192) || (tile_m == 192 && tile_n == 64));
}

// The one-launch small-shape kernel (contract_small): for plain GEMMs with the default split and
// no pinned 64/128 tile (RG_ALGO_TILED pins 64x64), K within its LDS panels, and either a pinned
// 32x32 tile or at most one block per compute unit. Measured on MI355X (GPU time per GEMM, S = 3):
// 256^3 7.7 us against 12.1 us for the two-launch pipeline, the LeNet layers 5.6-8.4 us against
// 7.4-10.0 us, 512x512x512 (256 tiles) 10.5 against 12.0 us; with four blocks per compute unit
// (1024x1024x64) it takes 20 us against 8.4 us, so more tiles than compute units keep the
// pipeline.
bool small_path(int M, int N, int K, int batch, int split_k, int tile_m, int tile_n, int algo,
                const PlanExtras& extras, int num_cus) {
    if (algo == RG_ALGO_TILED || split_k != 1 || K > SMALL_MAX_K) return false;
    if (!extras.one_launch || extras.raw || !extras.gemm_bound) return false;
    // A launch dimension holds fewer than 2^32 work-items: the kernel's grid is one block of
    // SMALL_THREADS per 32x32 tile, so a pinned 32x32 tile beyond that takes the pipeline.
    const long long tiles32 = (long long)ceil_div(M, 32) * ceil_div(N, 32);
    if (tiles32 * SMALL_THREADS >= (1ll << 32)) return false;
    if (tile_m == 32 && tile_n == 32) return true;
    if (pinned_tile(tile_m, tile_n, 3)) return false;
    const double tiles = (double)ceil_div(M, 32) * ceil_div(N, 32) * batch;
    return tiles <= std::max(1, num_cus);
}

// The band kernel (contract_band) can run the GEMM: op(A) read along rows, K within the band's
// LDS panels, one item, the default split, a plain GEMM, and op(B)'s digit region addressable
// with 32-bit offsets (Np columns of W-column blocks).
bool band_eligible(int N, int K, int S, bool ta, int batch, int split_k, int algo, int W,
                   const PlanExtras& extras) {
    if (ta || batch != 1 || split_k != 1 || K > BAND_MAX_K || algo == RG_ALGO_TILED) return false;
    if (!extras.one_launch || extras.raw || !extras.gemm_bound) return false;
    if (W < 64 || W % 32 != 0) return false;
    const long long np = (long long)ceil_div(N, W) * W;
    return np * round_up(K, STEP_K) * S < (1ll << 31);
}

// Estimated time (microseconds) of the band kernel with G column groups of W columns, and of
// the op(A) slicing that it saves against the tile plans (both read and write op(A) at about
// 4.5 TB/s), to weigh it against plan_cost's best tile plan; any choice gives the same bits.
// Blocks (one per compute unit) run in rounds; a round loads its bands of op(A) (32 rows of K
// values each, HBM-bound), then each wavefront contracts its ceil(W / 256) column tiles, one step
// per 32 values of k. Fitted on MI355X at S = 3 (the GPT-2 layers at 8192 tokens, K = 768:
// 0.53 us per step, the band load about 5.6 us): it picks the band for N = 768 and 2304 (3-18%
// faster than the 64x64 tiles plus op(A)'s slicing) and the 128x128 tiles for N = 3072 (2%
// faster than the band).
double band_cost(int M, int K, int S, int W, int G, int num_cus) {
    const double blocks = (double)ceil_div(M, 32) * G;
    const double slots = std::max(1, num_cus);
    const double rounds = std::ceil(blocks / slots);
    const double load_us = std::min(blocks, slots) * 32.0 * K * 4.0 / 4.5e6;
    const double step_us = 0.05 + 0.48 * (S * S / 9.0);
    const double steps = (double)ceil_div(W / 32, 8) * ceil_div(K, 32);
    return rounds * (load_us + steps * step_us);
}
double slice_a_cost(int M, int K, int S) { return (double)M * K * (4 + S) / 4.5e6; }

}  // namespace

int plan_layout(int M, int N, int K, int split_k, int tile_m, int tile_n, int algo, int S,
                bool ta, bool tb, const DeviceInfo& dev, Layout* Lp, const PlanExtras& extras) {
    if (M <= 0 || N <= 0 || K <= 0 || split_k <= 0) return hipErrorInvalidValue;
    if (S < 1 || S > 3) return hipErrorInvalidValue;
    const int batch = extras.batch;
    if (batch < 1 || batch > 65535) return hipErrorInvalidValue;  // grid z
    const double d = max_fixed_point(S);
    if (extras.gemm_bound && (double)K * d * d > std::ldexp(1.0, 62)) return hipErrorInvalidValue;
    if (algo < RG_ALGO_AUTO || algo > RG_ALGO_TENSOR_CORE) return hipErrorInvalidValue;

    Layout L;
    std::memset(&L, 0, sizeof L);
    L.S = S;
    L.M = M;
    L.N = N;
    L.K = K;
    L.batch = batch;
    L.ta = ta;
    L.tb = tb;
    L.a_strided = ta;   // A stored KxM: row r of op(A) is a column
    L.b_strided = !tb;  // B stored KxN: column c of op(B) is a column
    L.Kp = round_up(K, STEP_K);

    if (algo == RG_ALGO_REFERENCE) {
        L.algo = RG_ALGO_REFERENCE;
        L.Mp = round_up(M, PANEL_ROWS);
        L.Np = round_up(N, PANEL_ROWS);
        L.split = std::min(split_k, K);
        if ((long long)L.split * batch > 65535) return hipErrorInvalidValue;  // grid z
        L.has_partial = true;
    } else {
        if (!dev.gfx950) return hipErrorNotSupported;
        L.algo = algo == RG_ALGO_TILED ? RG_ALGO_TILED : RG_ALGO_TENSOR_CORE;
        // A pinned 32 x W tile (W >= 64) asks for the band kernel with blocks of W columns.
        if (tile_m == 32 && band_eligible(N, K, S, ta, batch, split_k, algo, tile_n, extras)) {
            L.band_w = tile_n;
            L.band_groups = ceil_div(N, tile_n);
        }
        if (L.band_w == 0 &&
            small_path(M, N, K, batch, split_k, tile_m, tile_n, algo, extras, dev.num_cus)) {
            L.small = true;
            L.Mp = round_up(M, PANEL_ROWS);
            L.Np = round_up(N, PANEL_ROWS);
            L.split = 1;
            L.has_partial = false;
            // Nothing of the workspace is used; a non-empty one keeps the callers' contract
            // (a workspace of at least the planned size) the same for every plan.
            L.total = 256;
            *Lp = L;
            return hipSuccess;
        }
    }
    if (L.band_w > 0) {
        L.Mp = round_up(M, PANEL_ROWS);
        L.Np = L.band_groups * L.band_w;
        L.split = 1;
        L.has_partial = false;
    } else if (L.algo != RG_ALGO_REFERENCE) {
        const int nsteps = L.Kp / STEP_K;
        const int min_split = ceil_div(nsteps, max_steps_per_part(S));
        // Candidate block tiles: the forced one, or 128x128 and 64x64; candidate splits: the
        // caller's (raised to the int32-exactness minimum), or, for the default split_k == 1,
        // that minimum, the next 8 splits and the splits that exactly fill 1..16 waves of the
        // GPU's block slots. The planner keeps the candidate with the lowest estimated time
        // (plan_cost); ties keep the earlier candidate.
        int tiles_cand[6][2];
        int ntile = 0;
        if (algo == RG_ALGO_TILED) {
            tiles_cand[ntile][0] = 1; tiles_cand[ntile++][1] = 1;
        } else if (pinned_tile(tile_m, tile_n, S)) {
            tiles_cand[ntile][0] = tile_m / 64; tiles_cand[ntile++][1] = tile_n / 64;
        } else {
            tiles_cand[ntile][0] = 2; tiles_cand[ntile++][1] = 2;
            tiles_cand[ntile][0] = 1; tiles_cand[ntile++][1] = 1;
            if (S == 3) {  // 192x64 first: where the two tie (the same tile count), it was the
                           // faster on every measured shape (the GPT-2 weight gradients, ~1.5%)
                tiles_cand[ntile][0] = 3; tiles_cand[ntile++][1] = 1;
                tiles_cand[ntile][0] = 1; tiles_cand[ntile++][1] = 3;
                // the eight-wavefront 128x64 / 64x128 (costs fitted at S = 3 only)
                tiles_cand[ntile][0] = 2; tiles_cand[ntile++][1] = 1;
                tiles_cand[ntile][0] = 1; tiles_cand[ntile++][1] = 2;
            }
        }
        const int split_lo = std::min(std::max(split_k, min_split), nsteps);
        double best = -1.0;
        int ti = 0, tj = 0, split = split_lo;
        for (int c = 0; c < ntile; ++c) {
            const int cti = tiles_cand[c][0], ctj = tiles_cand[c][1];
            auto consider = [&](int sp) {
                if (sp < split_lo || sp > nsteps) return;
                const double t = plan_cost(M, N, nsteps, batch, cti, ctj, sp, S, dev.num_cus,
                                           extras.raw);
                if (best < 0.0 || t < best) {
                    best = t;
                    ti = cti;
                    tj = ctj;
                    split = sp;
                }
            };
            consider(split_lo);
            if (split_k != 1) continue;
            for (int sp = split_lo + 1; sp <= split_lo + 8; ++sp) consider(sp);
            const long long tiles = (long long)ceil_div(M, 64 * cti) * ceil_div(N, 64 * ctj) * batch;
            const long long slots = (long long)std::max(1, dev.num_cus) * blocks_per_cu(cti, ctj, S);
            for (int waves = 1; waves <= 16; ++waves) {
                const long long sp = waves * slots / tiles;
                if (sp > split_lo + 8 && sp <= nsteps) consider((int)sp);
            }
        }
        L.ti = ti;
        L.tj = tj;
        L.Mp = round_up(M, 64 * ti);
        L.Np = round_up(N, 64 * tj);
        L.split = std::min(split, nsteps);
        L.has_partial = L.split > 1 || extras.raw;
        const int tiles_m = L.Mp / (64 * ti), tiles_n = L.Np / (64 * tj);
        // The contraction's grid must fit the int block order (any workspace that fits in
        // memory is far below this).
        if ((long long)tiles_m * tiles_n * L.split * batch > (1ll << 31) - 1)
            return hipErrorInvalidValue;
        // Block order. With a multiple of 8 tile columns the hardware's dealing (workgroup i
        // to XCD i mod 8) already keeps each XCD on tiles_n / 8 fixed tile columns for the
        // whole grid, whose column panels then stay in its L2 from one round of blocks to the
        // next when K is short; that plain order is kept (8192x3072x768: 2% faster than
        // grouped). Otherwise an XCD's resident blocks take a run of consecutive tiles in
        // groups of tile rows (N = 768 at 64x64: 1.5% faster; the LM head's 393 tile columns:
        // 1%). Any order gives the same bits.
        if (tiles_n % 8 == 0) {
            L.xcd_chunk = 0;
            L.group_m = 1;
        } else {
            L.xcd_chunk = std::max(1, dev.num_cus / 8) * blocks_per_cu(ti, tj, S);
            L.group_m = group_rows(L.xcd_chunk, ti, tj, tiles_m, tiles_n);
        }
        // The band kernel instead, when the caller pinned no tile and it is estimated faster
        // than this plan plus op(A)'s slicing (column groups: 1, 2, 4 or 8, W a multiple of 32).
        const bool pinned = algo == RG_ALGO_TILED || pinned_tile(tile_m, tile_n, S) ||
                            tile_m == 32;
        if (!pinned && split_k == 1) {
            double band_best = best + slice_a_cost(M, K, S);
            for (int G = 1; G <= 8; G *= 2) {
                const int W = round_up(ceil_div(N, G), 32);
                if (G > 1 && W == round_up(ceil_div(N, G / 2), 32)) break;  // no narrower
                if (!band_eligible(N, K, S, ta, batch, split_k, algo, W, extras)) continue;
                const double t = band_cost(M, K, S, W, ceil_div(N, W), dev.num_cus);
                if (t < band_best) {
                    band_best = t;
                    L.band_w = W;
                    L.band_groups = ceil_div(N, W);
                }
            }
            if (L.band_w > 0) {
                L.ti = L.tj = 0;
                L.Mp = round_up(M, PANEL_ROWS);
                L.Np = L.band_groups * L.band_w;
                L.split = 1;
                L.has_partial = false;
                L.xcd_chunk = 0;
                L.group_m = 1;
            }
        }
    }

    const int rows_a = (int)std::min<long long>((long long)M * batch, 1 << 30);
    const int rows_b = (int)std::min<long long>((long long)N * batch, 1 << 30);
    choose_chunks(M, rows_a, K, L.a_strided, &L.nch_a, &L.kch_a);
    choose_chunks(N, rows_b, K, L.b_strided, &L.nch_b, &L.kch_b);

    // One-read slicing of long column-access operands (MFMA algorithms): its partial maxima go
    // to the partial-maxima region, one row of slots per part.
    if (L.algo != RG_ALGO_REFERENCE && !L.small) {
        L.ps_a = pslice_route(L.a_strided, L.Kp) ? pslice_parts(L.a_strided, L.Kp) : 0;
        L.ps_b = pslice_route(L.b_strided, L.Kp) ? pslice_parts(L.b_strided, L.Kp) : 0;
    }

    const size_t q_elem = L.algo == RG_ALGO_REFERENCE ? sizeof(int32_t) : (size_t)S;
    // (the band kernel keeps op(A)'s digits and exponents in LDS: no op(A) regions)
    const size_t Mt = L.band_w > 0 ? 0 : (size_t)L.Mp * batch, Nt = (size_t)L.Np * batch;
    size_t off = 0;
    L.qa = off;
    off += align_up(Mt * L.Kp * q_elem);
    L.qb = off;
    off += align_up(Nt * L.Kp * q_elem);
    L.ea = off;
    off += align_up(Mt * sizeof(int));
    L.eb = off;
    off += align_up(Nt * sizeof(int));
    L.pma = off;
    off += align_up((size_t)std::max(L.nch_a, L.ps_a) * Mt * sizeof(float));
    L.pmb = off;
    off += align_up((size_t)std::max(L.nch_b, L.ps_b) * Nt * sizeof(float));
    L.part = off;
    if (L.has_partial) off += align_up((size_t)batch * L.split * M * N * sizeof(int64_t));
    L.total = off;
    *Lp = L;
    return hipSuccess;
}

namespace {

struct DevCache {
    std::atomic<int> state{0};  // 0 unknown, 1 known
    bool gfx950 = false;
    int num_cus = 0;
};
DevCache g_dev[64];

}  // namespace

int query_device(DeviceInfo* info) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev >= 0 && dev < 64 && g_dev[dev].state.load(std::memory_order_acquire) == 1) {
        info->gfx950 = g_dev[dev].gfx950;
        info->num_cus = g_dev[dev].num_cus;
        return hipSuccess;
    }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, dev)) != hipSuccess) return e;
    info->gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    info->num_cus = prop.multiProcessorCount;
    if (dev >= 0 && dev < 64) {
        g_dev[dev].gfx950 = info->gfx950;
        g_dev[dev].num_cus = info->num_cus;
        g_dev[dev].state.store(1, std::memory_order_release);
    }
    return hipSuccess;
}

int layout_for_current_device(int M, int N, int K, const rg_config* cfg, Layout* L,
                              const PlanExtras& extras) {
    if (!cfg) return hipErrorInvalidValue;
    DeviceInfo dev{false, 0};
    if (cfg->algo != RG_ALGO_REFERENCE) {
        int e = query_device(&dev);
        if (e != hipSuccess) return e;
    }
    return plan_layout(M, N, K, cfg->split_k, cfg->tile_m, cfg->tile_n, cfg->algo, cfg->slices,
                       cfg->trans_a != 0, cfg->trans_b != 0, dev, L, extras);
}

GemmAddressing dense_addressing(const Layout& L) {
    GemmAddressing a;
    a.lda = L.ta ? L.M : L.K;
    a.ldb = L.tb ? L.K : L.N;
    a.ldc = L.N;
    a.stride_a = (long long)L.M * L.K;
    a.stride_b = (long long)L.K * L.N;
    a.stride_c = (long long)L.M * L.N;
    return a;
}

int gemm_launch(const float* A, const float* B, float* C, const Layout& L, char* base,
                hipStream_t stream, void* const* stage_events, const GemmOptions& opt,
                const GemmAddressing& addr) {
    if ((opt.group_a > 0 || opt.group_b > 0) && L.batch != 1) return hipErrorInvalidValue;
    auto record = [&](int i) {
        if (stage_events) (void)hipEventRecord(static_cast<hipEvent_t>(stage_events[i]), stream);
    };
    if (L.small) {  // slicing, contraction and rounding in one kernel
        if (opt.group_a > 0 || opt.group_b > 0 || opt.raw || opt.im2col_a || opt.nanrows_a ||
            opt.nanrows_b || !A || L.K > SMALL_MAX_K)
            return hipErrorInvalidValue;
        record(0);
        record(1);
        launch_contract_small(L, A, B, C, addr, stream);
        record(2);
        record(3);
        return hipGetLastError();
    }
    void* qa = base + L.qa;
    void* qb = base + L.qb;
    int* ea = reinterpret_cast<int*>(base + L.ea);
    int* eb = reinterpret_cast<int*>(base + L.eb);
    float* pma = reinterpret_cast<float*>(base + L.pma);
    float* pmb = reinterpret_cast<float*>(base + L.pmb);
    int64_t* part = L.has_partial ? reinterpret_cast<int64_t*>(base + L.part) : nullptr;
    const bool i32 = L.algo == RG_ALGO_REFERENCE;

    auto desc = [&](const float* src, int R, int Rp, bool strided, long long ld, long long bstride,
                    int nch, int kch, float* pm, void* out, int* expo) {
        SliceDesc d;
        d.src = src;
        d.R = R;
        d.K = L.K;
        d.Rp = Rp;
        d.Kp = L.Kp;
        d.ld = ld;
        d.batch = L.batch;
        d.bstride = L.batch > 1 ? bstride : 0;
        d.strided = strided ? 1 : 0;
        const bool aligned = (reinterpret_cast<uintptr_t>(src) & 15) == 0 && ld % 4 == 0 &&
                             d.bstride % 4 == 0;
        d.vec = aligned && (strided ? (R % 4 == 0) : (L.K % 4 == 0)) ? 1 : 0;
        d.nch = nch;
        d.kch = kch;
        d.pmax = pm;
        d.out = out;
        d.expo = expo;
        d.im2col = 0;
        std::memset(&d.g, 0, sizeof d.g);
        d.nanrows = nullptr;
        slice_grid(d);
        d.spin_limit = slice_spin_limit();
        pslice_grid(d);
        return d;
    };
    SliceDesc da = desc(A, L.M, L.Mp, L.a_strided, addr.lda, addr.stride_a, L.nch_a,
                        L.kch_a, pma, qa, ea);
    if (opt.im2col_a) {  // op(A) gathered: only the one-pass route reads through Im2col
        if (i32 || L.batch != 1 || L.a_strided || opt.group_a > 0 || !onepass_eligible(da))
            return hipErrorInvalidValue;
        da.im2col = 1;
        da.g = *opt.im2col_a;
        da.vec = 0;
    }
    SliceDesc db = desc(B, L.N, L.Np, L.b_strided, addr.ldb, addr.stride_b, L.nch_b,
                        L.kch_b, pmb, qb, eb);
    da.nanrows = opt.nanrows_a;
    db.nanrows = opt.nanrows_b;
    const OutAddr out{addr.ldc, addr.stride_c};

    if (L.band_w > 0) {  // op(B)'s one pass, then op(A)'s slicing, contraction, rounding
        if (opt.group_a > 0 || opt.group_b > 0 || opt.raw || opt.im2col_a || opt.nanrows_a ||
            opt.nanrows_b || L.batch != 1 || L.K > BAND_MAX_K || !onepass_eligible(db))
            return hipErrorInvalidValue;
        record(0);
        launch_onepass(db, false, db, true, L.S, stream);
        record(1);
        launch_contract_band(L, A, addr.lda, static_cast<const int8_t*>(qb), eb, C, addr.ldc,
                             stream);
        record(2);
        record(3);
        return hipGetLastError();
    }

    record(0);
    // Operands sliced in one pass (short K), or in one read with parts along K (long K, column
    // access); the others (and group scales, and the reference algorithm's int32 values) take
    // the two passes.
    const bool one_a = !i32 && opt.group_a == 0 && onepass_eligible(da);
    const bool one_b = !i32 && opt.group_b == 0 && onepass_eligible(db);
    const bool ps_a = !i32 && opt.group_a == 0 && !da.im2col && L.ps_a > 0;
    const bool ps_b = !i32 && opt.group_b == 0 && L.ps_b > 0;
    if (one_a && one_b) {
        launch_onepass(da, true, db, true, L.S, stream);
    } else if (!da.im2col && (one_a || ps_a) && (one_b || ps_b)) {
        // The one-read blocks wait on partial-maximum slots that a launch before them marks
        // empty. With the other operand in one pass, both share one launch (its traffic keeps
        // the memory busy while the one-read blocks exchange maxima: 4096^3 NN slicing 59.9 ->
        // 55.3 us against a one-pass launch that marks the slots followed by the one read).
        const MarkRange ma = ps_a ? pslice_slots(da) : MarkRange();
        const MarkRange mb = ps_b ? pslice_slots(db) : MarkRange();
        launch_mark(ma, mb, stream);
        if (one_a || one_b) launch_onepass_pslice(one_a ? da : db, one_a ? db : da, L.S, stream);
        else launch_pslice(da, ps_a, db, ps_b, L.S, stream);
    } else if (da.im2col) {
        // the gathering operand on its own, then op(B)'s two passes
        launch_onepass(da, true, db, false, L.S, stream);
        SliceDesc none = da;
        none.max_blocks = 0;
        none.split_blocks = 0;
        launch_absmax(none, db, stream);
        if (opt.group_b > 0) launch_group_max(db, opt.group_b, stream);
        launch_split(none, db, L.S, i32, stream);
    } else if (ps_a || ps_b) {
        // one operand in one read, the other in two passes (past the one read's part limit,
        // or group scales): the one read and the other's maxima in one launch,
        // then the other's split (1024x1024x65536 NN slicing 287 -> ~230 us)
        const SliceDesc& ps = ps_a ? da : db;
        const SliceDesc& two = ps_a ? db : da;
        const int group = ps_a ? opt.group_b : opt.group_a;
        SliceDesc none = ps;
        none.split_blocks = 0;
        launch_mark(pslice_slots(ps), MarkRange(), stream);
        launch_pslice_absmax(ps, two, L.S, stream);
        if (group > 0) launch_group_max(two, group, stream);
        if (ps_a) launch_split(none, two, L.S, i32, stream);
        else launch_split(two, none, L.S, i32, stream);
    } else if (one_a != one_b) {
        // one launch for the one-pass operand and the other's maxima, then the other's split
        const SliceDesc& one = one_a ? da : db;
        const SliceDesc& two = one_a ? db : da;
        const int group = one_a ? opt.group_b : opt.group_a;
        launch_onepass_absmax(one, two, L.S, stream);
        if (group > 0) launch_group_max(two, group, stream);
        SliceDesc none = one;
        none.split_blocks = 0;
        if (one_a) launch_split(none, two, L.S, i32, stream);
        else launch_split(two, none, L.S, i32, stream);
    } else {
        launch_absmax(da, db, stream);
        launch_group_max2(&da, opt.group_a, &db, opt.group_b, stream);
        launch_split(da, db, L.S, i32, stream);
    }
    record(1);
    if (i32)
        launch_contract_reference(L, static_cast<const int32_t*>(qa),
                                  static_cast<const int32_t*>(qb), part, stream);
    else
        launch_contract_mfma(L, static_cast<const int8_t*>(qa), static_cast<const int8_t*>(qb),
                             ea, eb, C, out, part, stream);
    record(2);
    if (L.has_partial && !opt.raw) launch_reduce_round(L, part, ea, eb, C, out, stream);
    record(3);
    return hipGetLastError();
}

// Workspace of rg_gemm_fp32_noalloc: a fixed array in device memory, one copy per GPU (each
// GPU that loads the code object gets its own). Host code must never pass `scratch` itself to a
// kernel or a copy: on the host the name is only a stand-in for the symbol. Its device address
// on the current GPU comes from hipGetSymbolAddress, taken once per device and kept in
// g_scratch.
static __device__ __align__(256) unsigned char scratch[RG_NOALLOC_SCRATCH_BYTES];

namespace {

struct ScratchSlot {
    std::atomic<void*> ptr{nullptr};
    std::mutex mu;
};
ScratchSlot g_scratch[64];

// The scratch array's address on the current device, looked up on the first successful call per
// device and kept; a failed lookup is returned and not kept, so a later call tries again.
int scratch_on_current_device(void** out) {
    int dev = 0;
    int e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    ScratchSlot& slot = g_scratch[dev];
    void* p = slot.ptr.load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(slot.mu);
        p = slot.ptr.load(std::memory_order_relaxed);
        if (p == nullptr) {
            if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
            if (p == nullptr) return hipErrorInvalidSymbol;
            slot.ptr.store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

}  // namespace rg

extern "C" {

void rg_config_init(rg_config* cfg) {
    if (!cfg) return;
    cfg->split_k = 1;
    cfg->tile_m = 16;
    cfg->tile_n = 16;
    cfg->tile_k = 32;
    cfg->algo = RG_ALGO_AUTO;
    cfg->slices = 3;
    cfg->trans_a = 0;
    cfg->trans_b = 0;
}

int rg_make_plan(int M, int N, int K, const rg_config* cfg, rg_plan* plan) {
    if (!plan) return hipErrorInvalidValue;
    rg::Layout L;
    int e = rg::layout_for_current_device(M, N, K, cfg, &L);
    if (e != hipSuccess) return e;
    plan->algo = L.algo;
    plan->split_k = L.split;
    plan->workspace_bytes = L.total;
    plan->tile_m = L.small || L.band_w > 0 ? 32 : 64 * L.ti;
    plan->tile_n = L.small ? 32 : (L.band_w > 0 ? L.band_w : 64 * L.tj);
    return hipSuccess;
}

int rg_plan_for_device(int M, int N, int K, const rg_config* cfg, int is_gfx950, int num_cus,
                       rg_plan* plan, rg_layout_info* info) {
    if (!cfg || !plan) return hipErrorInvalidValue;
    rg::DeviceInfo dev{is_gfx950 != 0, num_cus};
    rg::Layout L;
    int e = rg::plan_layout(M, N, K, cfg->split_k, cfg->tile_m, cfg->tile_n, cfg->algo,
                            cfg->slices, cfg->trans_a != 0, cfg->trans_b != 0, dev, &L);
    if (e != hipSuccess) return e;
    plan->algo = L.algo;
    plan->split_k = L.split;
    plan->workspace_bytes = L.total;
    plan->tile_m = L.small || L.band_w > 0 ? 32 : 64 * L.ti;
    plan->tile_n = L.small ? 32 : (L.band_w > 0 ? L.band_w : 64 * L.tj);
    if (info) {
        info->qa = L.qa;
        info->qb = L.qb;
        info->ea = L.ea;
        info->eb = L.eb;
        info->part = L.has_partial ? (long long)L.part : -1;
        info->Mp = L.Mp;
        info->Np = L.Np;
        info->Kp = L.Kp;
        info->split_k = L.split;
    }
    return hipSuccess;
}

int rg_test_block_order(int M, int N, int K, const rg_config* cfg, int is_gfx950, int num_cus,
                        int batch, int* coords, long long capacity, long long* blocks) {
    if (!cfg || !blocks) return hipErrorInvalidValue;
    rg::DeviceInfo dev{is_gfx950 != 0, num_cus};
    rg::PlanExtras extras;
    extras.batch = batch;
    rg::Layout L;
    int e = rg::plan_layout(M, N, K, cfg->split_k, cfg->tile_m, cfg->tile_n, cfg->algo,
                            cfg->slices, cfg->trans_a != 0, cfg->trans_b != 0, dev, &L, extras);
    if (e != hipSuccess) return e;
    *blocks = 0;
    if (L.algo == RG_ALGO_REFERENCE || L.small || L.band_w > 0) return hipSuccess;
    const int tiles_m = L.Mp / (64 * L.ti), tiles_n = L.Np / (64 * L.tj);
    const long long total = (long long)tiles_m * tiles_n * L.split * L.batch;
    *blocks = total;
    if (!coords || capacity < 4 * total) return hipSuccess;
    for (long long i = 0; i < total; ++i) {
        int item, part, tm, tn;
        rg::block_tile(rg::xcd_order((int)i, (int)total, L.xcd_chunk), tiles_m, tiles_n, L.split,
                       L.group_m, &item, &part, &tm, &tn);
        coords[4 * i] = item;
        coords[4 * i + 1] = part;
        coords[4 * i + 2] = tm;
        coords[4 * i + 3] = tn;
    }
    return hipSuccess;
}

int rg_test_pslice_placement(int M, int N, int K, const rg_config* cfg, int num_cus, int batch,
                             long long* blocks, long long* split_panels) {
    if (!cfg || !blocks || !split_panels) return hipErrorInvalidValue;
    rg::DeviceInfo dev{true, num_cus};
    rg::PlanExtras extras;
    extras.batch = batch;
    rg::Layout L;
    const int e = rg::plan_layout(M, N, K, cfg->split_k, cfg->tile_m, cfg->tile_n, cfg->algo,
                                  cfg->slices, cfg->trans_a != 0, cfg->trans_b != 0, dev, &L,
                                  extras);
    if (e != hipSuccess) return e;
    *blocks = 0;
    *split_panels = 0;
    const struct {
        int parts, Rp;
        bool strided;
    } ops[2] = {{L.ps_a, L.Mp, L.a_strided}, {L.ps_b, L.Np, L.b_strided}};
    for (const auto& op : ops) {
        if (op.parts <= 0) continue;
        rg::SliceDesc d;
        std::memset(&d, 0, sizeof d);
        d.Rp = op.Rp;
        d.Kp = L.Kp;
        d.batch = L.batch;
        d.strided = op.strided ? 1 : 0;
        rg::pslice_grid(d);
        const long long panels = (long long)d.batch * (d.Rp / (d.strided ? rg::PANEL_ROWS : 8));
        std::vector<int> xcd((size_t)panels, -1);
        for (long long blk = 0; blk < d.ps_blocks; ++blk) {
            const long long u = rg::pslice_unit(blk, d.ps_blocks);
            if (u >= panels * d.ps_parts) continue;
            int& x = xcd[(size_t)(u / d.ps_parts)];
            if (x == -1) x = (int)(blk & 7);
            else if (x != (int)(blk & 7) && x != 8) {
                x = 8;  // seen on two XCDs
                ++*split_panels;
            }
        }
        *blocks += d.ps_blocks;
    }
    return hipSuccess;
}

int rg_test_set_spin_limit(int polls) {
    const int prev = rg::slice_spin_limit();
    rg::set_slice_spin_limit(polls < 0 ? rg::DEFAULT_SPIN_LIMIT : polls);
    return prev;
}

int rg_workspace_layout(int M, int N, int K, const rg_config* cfg, rg_layout_info* info) {
    if (!info) return hipErrorInvalidValue;
    rg::Layout L;
    int e = rg::layout_for_current_device(M, N, K, cfg, &L);
    if (e != hipSuccess) return e;
    info->qa = L.qa;
    info->qb = L.qb;
    info->ea = L.ea;
    info->eb = L.eb;
    info->part = L.has_partial ? (long long)L.part : -1;
    info->Mp = L.Mp;
    info->Np = L.Np;
    info->Kp = L.Kp;
    info->split_k = L.split;
    return hipSuccess;
}

int rg_test_round(const int* levels, const long long* T, const int* E, float* out, long long n,
                  int S, void* stream) {
    if ((levels == nullptr) == (T == nullptr) || !E || !out || n < 0 || n > (1ll << 30))
        return hipErrorInvalidValue;
    if (levels && (S < 1 || S > 3)) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    rg::launch_test_round(levels, reinterpret_cast<const int64_t*>(T), E, out, n, S,
                          static_cast<hipStream_t>(stream));
    return hipGetLastError();
}

int rg_gemm_fp32_ws(const float* A, const float* B, float* C, int M, int N, int K,
                    const rg_config* cfg, void* workspace, size_t workspace_bytes, void* stream,
                    void* const* stage_events) {
    if (!A || !B || !C) return hipErrorInvalidValue;
    rg::Layout L;
    int e = rg::layout_for_current_device(M, N, K, cfg, &L);
    if (e != hipSuccess) return e;
    if (!workspace || workspace_bytes < L.total) return hipErrorInvalidValue;
    return rg::gemm_launch(A, B, C, L, static_cast<char*>(workspace),
                           static_cast<hipStream_t>(stream), stage_events, rg::GemmOptions(),
                           rg::dense_addressing(L));
}

int rg_gemm_fp32_noalloc(const float* A, const float* B, float* C, int M, int N, int K,
                         const rg_config* cfg, void* stream) {
    if (!A || !B || !C) return hipErrorInvalidValue;
    rg::Layout L;
    int e = rg::layout_for_current_device(M, N, K, cfg, &L);
    if (e != hipSuccess) return e;
    if (L.total > RG_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
    void* ws = nullptr;
    if ((e = rg::scratch_on_current_device(&ws)) != hipSuccess) return e;
    return rg::gemm_launch(A, B, C, L, static_cast<char*>(ws), static_cast<hipStream_t>(stream),
                           nullptr, rg::GemmOptions(), rg::dense_addressing(L));
}

int rg_make_plan_strided_batched(int M, int N, int K, int batch, const rg_config* cfg,
                                 rg_plan* plan) {
    if (!plan) return hipErrorInvalidValue;
    rg::PlanExtras ex;
    ex.batch = batch;
    rg::Layout L;
    int e = rg::layout_for_current_device(M, N, K, cfg, &L, ex);
    if (e != hipSuccess) return e;
    plan->algo = L.algo;
    plan->split_k = L.split;
    plan->workspace_bytes = L.total;
    plan->tile_m = L.small || L.band_w > 0 ? 32 : 64 * L.ti;
    plan->tile_n = L.small ? 32 : (L.band_w > 0 ? L.band_w : 64 * L.tj);
    return hipSuccess;
}

int rg_gemm_strided_batched_fp32_ws(const float* A, long long lda, long long stride_a,
                                    const float* B, long long ldb, long long stride_b, float* C,
                                    long long ldc, long long stride_c, int M, int N, int K,
                                    int batch, const rg_config* cfg, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    if (!A || !B || !C || !cfg) return hipErrorInvalidValue;
    rg::PlanExtras ex;
    ex.batch = batch;
    rg::Layout L;
    int e = rg::layout_for_current_device(M, N, K, cfg, &L, ex);
    if (e != hipSuccess) return e;
    if (lda < (L.ta ? M : K) || ldb < (L.tb ? K : N) || ldc < N) return hipErrorInvalidValue;
    if (stride_a < 0 || stride_b < 0 || stride_c < 0) return hipErrorInvalidValue;
    if (!workspace || workspace_bytes < L.total) return hipErrorInvalidValue;
    rg::GemmAddressing addr{lda, ldb, ldc, stride_a, stride_b, stride_c};
    return rg::gemm_launch(A, B, C, L, static_cast<char*>(workspace),
                           static_cast<hipStream_t>(stream), nullptr, rg::GemmOptions(), addr);
}

int rg_gemm_fp32(const float* A, const float* B, float* C, int M, int N, int K,
                 const rg_config* cfg, void* stream) {
    rg_plan plan;
    int e = rg_make_plan(M, N, K, cfg, &plan);
    if (e != hipSuccess) return e;
    void* ws = nullptr;
    if ((e = hipMalloc(&ws, plan.workspace_bytes)) != hipSuccess) return e;
    e = rg_gemm_fp32_ws(A, B, C, M, N, K, cfg, ws, plan.workspace_bytes, stream, nullptr);
    // Synchronise to surface asynchronous kernel errors at this API boundary.
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    (void)hipFree(ws);
    return e;
}

const char* rg_algo_name(int algo) {
    switch (algo) {
        case RG_ALGO_AUTO: return "auto";
        case RG_ALGO_REFERENCE: return "ref";
        case RG_ALGO_TILED: return "tiled";
        case RG_ALGO_TENSOR_CORE: return "tc";
        default: return "?";
    }
}

const char* rg_error_string(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }

}  // extern "C"
