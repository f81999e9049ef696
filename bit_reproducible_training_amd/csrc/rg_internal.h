#pragma once
// Internal declarations shared by the slicing kernels, the contraction kernels and the
// host API of librepro_gemm.so. Nothing here is part of the public ABI.
#include <hip/hip_runtime.h>

#include "repro_gemm.h"
#include "rg_fastdiv.h"

#include <cstddef>
#include <cstdint>

namespace rg {

// Per-row constants of the rounding X = RNE(x * 2^(7(S-1) - se)), clamped to +-lim.
// The scale is applied as two multiplications by normal powers of two, as the definition
// does (repro_gemm_math.cuh:44-55, 71-83): with n = 7(S-1) - se in [-122, 163], both
// factors are normal; the product is exact unless it is subnormal, and then |v| < 2^-126
// rounds to 0 whatever the intermediate rounding was. Needs IEEE f32 denormals, which the
// gfx950 kernels of this library run with (denorm mode 3, no flushing).
struct RowScale {
    float p1, p2;
    int lim;
};

__device__ __forceinline__ RowScale row_scale(int S, int se) {
    const int n = 7 * (S - 1) - se;
    const int n1 = n >> 1, n2 = n - n1;
    RowScale rs;
    rs.p1 = __uint_as_float((uint32_t)(n1 + 127) << 23);
    rs.p2 = __uint_as_float((uint32_t)(n2 + 127) << 23);
    rs.lim = 127 << (7 * (S - 1));
    return rs;
}

template <int S>
__device__ __forceinline__ RowScale row_scale(int se) {
    return row_scale(S, se);
}

__device__ __forceinline__ int round_fixed(float x, const RowScale& rs) {
    if (!__builtin_isfinite(x)) return -rs.lim;  // NaN, +-inf: as repro_gemm::fixed_point
    const float v = (x * rs.p1) * rs.p2;
    const int X = (int)__builtin_rintf(v);  // v_rndne_f32: nearest-even; |v| < 2^22 here
    return min(max(X, -rs.lim), rs.lim);
}

// Four bytes (low byte of each argument) packed little-endian with v_perm_b32.
__device__ __forceinline__ uint32_t pack4(int b0, int b1, int b2, int b3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b1, (uint32_t)b0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)b3, (uint32_t)b2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// The base-128 digits of a fixed-point value X (|X| <= 127 * 128^(S-1)), most significant
// first: X = sum_p d[p] 128^(S-1-p) with a signed top digit d[0] = floor(X / 128^(S-1)) in
// [-127, 127] and unsigned lower digits d[p] in [0, 127] (the bit fields of X). Any digit split
// with these weights gives the same exact products; this one keeps the lower digits' sign bits
// clear, which lowers the matrix cores' switching power (about 2% more int8 MFMA throughput
// measured on MI355X with N(0,1) digit planes than balanced digits in [-64, 63]).
template <int S>
__device__ __forceinline__ void digits_of(int X, int (&d)[S]) {
#pragma unroll
    for (int p = S - 1; p >= 1; --p) {
        d[p] = X & 127;
        X >>= 7;  // arithmetic: floor(X / 128)
    }
    d[0] = X;
}

// Largest |x| over a 64-lane wavefront, in every lane.
__device__ __forceinline__ float wave_max(float m) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    return m;
}

// Sliced operands are stored in 1 KiB panels of 32 rows x 32 k x one digit, in the
// order the CDNA4 MFMA reads its operands: byte lane*16 + j of a panel holds element
// (row = lane % 32, k = 16 * (lane / 32) + j). Panels are laid out
// [row / 32][k / 32][digit], so one pipeline stage of a block (its row panels x two
// k panels x S digits) is a few contiguous runs of 2*S KiB.
constexpr int PANEL_ROWS = 32;
constexpr int PANEL_K = 32;
constexpr int PANEL_BYTES = 1024;
constexpr int STEP_K = 64;  // k consumed per pipeline stage of the contraction
// Longest K of the one-launch small-shape kernel (its digit panels of both operands sit in LDS).
constexpr int SMALL_MAX_K = 512;
// Threads of a block of the one-launch small-shape kernel (one block per 32x32 tile of C).
constexpr int SMALL_THREADS = 1024;
// Band kernel (contract_band): longest K whose digit panels of a 32-row band of op(A) it keeps in
// LDS (32 k panels x S KiB), threads per block, and k panels of op(B) each wavefront has in
// flight.
constexpr int BAND_MAX_K = 1024;
constexpr int BAND_THREADS = 768;
constexpr int BAND_DEPTH = 2;

// Which output tile a contraction block computes. The hardware deals a launch's workgroups to
// the 8 XCDs in turn (linear workgroup id mod 8), and each XCD has its own L2. The block at
// linear id `lin` (of `total`) computes logical block xcd_order(lin, total, chunk): an XCD's
// successive workgroups take runs of `chunk` consecutive logical blocks (chunk = the blocks an
// XCD holds at once), so the blocks resident on one XCD are neighbours in the logical order
// and fetch their shared digit panels into that XCD's L2 once. A grid that is not a multiple
// of 8 * chunk has its remainder dealt the same way with a smaller run, and its last
// (total mod 8) blocks keep their own ids. chunk = 0 keeps every id (the plain row-major
// order). The mapping is a bijection of [0, total).
__host__ __device__ inline int xcd_order(int lin, int total, int chunk) {
    if (chunk == 0) return lin;
    const int full = total / (8 * chunk) * (8 * chunk);
    const int xcd = lin & 7, loc = lin >> 3;
    if (lin < full) return loc / chunk * (8 * chunk) + xcd * chunk + loc % chunk;
    const int run = (total - full) / 8;  // full is a multiple of 8: lin & 7 is still the XCD
    const int l2 = lin - full;
    if (l2 < 8 * run) return full + xcd * run + (l2 >> 3);
    return lin;
}

// Logical block t -> (item, split part, tile row, tile column). Logical blocks run item by
// item, part by part; within a part, tiles go through groups of `group_m` tile rows (the last
// group may be shorter), column by column inside a group, so a run of consecutive tiles covers
// a few row panels of op(A) and a few column panels of op(B).
__host__ __device__ inline void block_tile(int t, int tiles_m, int tiles_n, int split,
                                           int group_m, int* item, int* part, int* tm, int* tn) {
    const int tiles = tiles_m * tiles_n;
    const int ip = t / tiles, tile = t - ip * tiles;
    *item = ip / split;
    *part = ip - *item * split;
    const int span = group_m * tiles_n;
    const int g = tile / span, w = tile - g * span;
    const int left = tiles_m - g * group_m;
    const int rows = left < group_m ? left : group_m;
    *tm = g * group_m + w % rows;
    *tn = w / rows;
}

// Where each region lives inside the caller's workspace, and how the work is split. A batch
// of `batch` independent GEMMs of one shape stacks its items: item b's digit panels, exponents
// and partial maxima follow item b-1's (per-item sizes Mp, Np), and its partials too.
struct Layout {
    int algo;           // resolved RG_ALGO_* (never AUTO)
    int S, M, N, K;
    int batch;          // items (1 for the plain GEMM)
    int Mp, Np, Kp;     // padded sizes: Mp, Np multiples of the block tile, Kp of STEP_K
    int ti, tj;         // MFMA block tile = (64*ti) x (64*tj); 0 for REFERENCE and small
    bool small;         // one launch of contract_small (32x32 tiles, no workspace use)
    int band_w;         // > 0: contract_band, blocks of 32 rows x band_w columns (op(B) sliced
                        // first; op(A)'s digits never in the workspace); 0 otherwise
    int band_groups;    // column groups of the band kernel (Np = band_groups * band_w)
    int split;          // split-K parts
    int xcd_chunk;      // contraction block order (xcd_order): blocks resident per XCD, or 0
    int group_m;        // tile rows per group of the block order (block_tile)
    bool ta, tb;
    bool a_strided, b_strided;  // operand read along k with a stride (column access)
    int nch_a, kch_a;   // row-max pass of op(A): chunks along K and chunk length
    int nch_b, kch_b;
    bool has_partial;
    int ps_a, ps_b;     // parts of the one-read column slicing (pslice_route), 0 when not taken
    size_t qa, qb, ea, eb, pma, pmb, part, total;  // byte offsets, 256-aligned
};

// Device facts the planner needs.
struct DeviceInfo {
    bool gfx950;
    int num_cus;
};

// Architecture and compute-unit count of the current device (cached per device).
int query_device(DeviceInfo* info);

// Planner options beyond the reference's make_plan. raw: keep the exact int64 sums T (the
// partial buffer [batch][split][M][N], summed by the caller) instead of rounding them to C.
// gemm_bound: apply the reference GEMM's K bound (K * max|X|^2 <= 2^62 with max|X| the
// largest digit-split value); callers with their own exactness bound (the convolution's, on
// the clamped |X| <= 127*128^(S-1)) pass false. batch: independent GEMMs of one shape.
struct PlanExtras {
    bool raw = false;
    bool gemm_bound = true;
    int batch = 1;
    bool one_launch = true;  // the small-shape kernel may be chosen (plain GEMMs only)
};

// Builds the layout; returns a hipError_t code (0, InvalidValue, NotSupported).
int plan_layout(int M, int N, int K, int split_k, int tile_m, int tile_n, int algo, int S,
                bool ta, bool tb, const DeviceInfo& dev, Layout* L,
                const PlanExtras& extras = PlanExtras());

// Implicit im2col: the operand's row w = (n, oy, ox) is window (oy, ox) of image n of
// x[N][C][H][W] (P = OH * OW windows per image), its element k = (c, ky, kx) the input value
// at (c, oy * SY - PY + ky, ox * SX - PX + kx), zero in the padding.
struct Im2col {
    const float* x;
    int C, H, W, KH, KW, SY, SX, PY, PX, OW, P;
    FastDiv dP, dOW, dKHW, dKW;
};

// One operand of the slice split: `batch` items, each op(X) of R rows of K values, item b at
// src + b * bstride. Element (r, k) of an item is at [r * ld + k] (row access), or at
// [k * ld + r] when `strided` (row r read along k with stride ld). Rows are stacked item by
// item, each item padded to Rp rows: stacked row q = b * Rp + r indexes the partial maxima,
// the exponents and the digit panels.
struct SliceDesc {
    const float* src;
    int R, K, Rp, Kp;   // per item
    long long ld;       // elements between rows (row access) or between k (column access)
    int batch;
    long long bstride;  // elements between items
    int strided;
    int vec;            // 16-byte vector loads allowed (alignment of src, ld, bstride; K or R % 4)
    int nch, kch;       // row-max chunks along K and their length
    float* pmax;        // [nch][batch * Rp] partial maxima
    void* out;          // digit panels (or int32 [batch * Rp][Kp] for the reference algorithm)
    int* expo;          // [batch * Rp] exponents
    long long max_blocks, split_blocks;
    int im2col;         // rows are gathered through `g` (one-pass route, row access, one item)
    Im2col g;
    // One-read slicing of a column-access operand past the one-pass limit (launch_pslice): parts
    // along K per 32-row panel (their partial maxima go to pmax[part], whose slots an earlier
    // launch of the same call marks PM_EMPTY), the bound on a block's wait for the other parts,
    // and the grid.
    int ps_parts;
    int spin_limit;
    long long ps_blocks;
    // k panels per wavefront of a column-access operand (pslice_kpw: PS_KPW, or PS_KPW_WIDE
    // for K past 32768).
    int ps_kpw;
    // Null, or one flag per stacked row (batch * Rp): a row whose flag is non-zero takes
    // exponent 0, the exponent of a maximum that a NaN wins (the convolution's window and
    // position maxima; the maxima computed here skip NaN).
    const unsigned* nanrows;
};

// Bit pattern of a partial-maximum slot not yet written by this call (a NaN; no maximum of
// magnitudes is NaN, the maxima skip NaN).
constexpr unsigned PM_EMPTY = 0xFFFFFFFFu;
// A region of slots to mark PM_EMPTY.
struct MarkRange {
    unsigned* p = nullptr;
    long long n = 0;
};

// Fills max_blocks / split_blocks of d.
void slice_grid(SliceDesc& d);

// Single-pass slicing (row maxima, exponents and digit panels in one launch, each input read
// once) of an operand, for padded K up to ONEPASS_MAX_K (row access) or ONEPASS_MAX_K_COLUMNS
// (column access, whose 32-byte row segments fetch slower than the two passes' wide ones at
// large K); 16-byte loads where the operand allows them, scalar loads otherwise.
// launch_onepass slices the operands whose use_* is set (both share K).
constexpr int ONEPASS_MAX_K = 4096;
constexpr int ONEPASS_MAX_K_COLUMNS = 3072;
bool onepass_eligible(const SliceDesc& d);
void launch_onepass(const SliceDesc& a, bool use_a, const SliceDesc& b, bool use_b, int S,
                    hipStream_t stream);

// One-read slicing of an operand whose padded K is past the one-pass limit: a block holds a
// 32-row panel of op(X) (column access: 32 columns of the stored matrix) over PS_WAVES * kpw k
// panels, or a strip of 8 rows (row access) over PS_ROW_NPB k panels, in registers, and the
// ps_parts blocks of a panel or strip exchange their partial maxima.
constexpr int PS_WAVES = 8;
constexpr int PS_KPW = 4;                        // k panels per wavefront (column access)
constexpr int PS_NPB = PS_WAVES * PS_KPW;        // k panels per block (column access)
constexpr int PS_ROW_NF4 = 16;                   // k panels per wavefront (row access)
constexpr int PS_ROW_NPB = PS_WAVES * PS_ROW_NF4;
// At most this many parts per panel exchanging through one XCD's L2: the parts of a panel wait
// for each other, so they must be resident together on that XCD (64 slots of these blocks per
// XCD at S = 3); with 64 parts they needed every slot at once and waited out their bound
// (measured: 1024x1024x65536 NN), with 32 they did not.
constexpr int PS_MAX_PARTS = 32;
// Column-access operands that would need more parts (K past 32768) take longer parts, the wide
// form: PS_KPW_WIDE k panels per wavefront (2560 k per part), at most PS_MAX_PARTS_WIDE parts
// per panel (K up to 66560). A wide block (205 registers at S = 3) fills its compute unit, so a
// panel's parts take 26 of an XCD's 32 compute units and exchange through its L2; the rest is
// slack for other streams' kernels: with a kernel of another stream holding two compute units
// per XCD, 1024x1024x65536 slicing stayed at 0.23 ms, where 32 parts of 2048 k took 3.5 ms (every
// panel's resident parts waiting out their bound, then re-reading K; same bits); with six held,
// both took 3.5 ms. Against 64 parts spread over every XCD exchanging through
// memory, 1024x1024x65536 slicing took 0.259 -> 0.222 ms with both operands column-access (TN)
// and 0.229 -> 0.224 ms with B alone (NN), on one box, with 2048 k per part (32 parts, no
// slack); 2560 k per part measured the same on NN and 2-4% slower on TN and TT (3072 k: 3-8%).
// Longer operands (column access past K = 66560, row access past 131072) keep the two passes.
constexpr int PS_KPW_WIDE = 10;
constexpr int PS_MAX_PARTS_WIDE = 26;
// k panels per wavefront of a column-access operand's one read (0 for row access).
__host__ __device__ inline int pslice_kpw(bool strided, int Kp) {
    if (!strided) return 0;
    return (Kp / PANEL_K + PS_NPB - 1) / PS_NPB > PS_MAX_PARTS ? PS_KPW_WIDE : PS_KPW;
}
__host__ __device__ inline int pslice_parts(bool strided, int Kp) {
    const int npb = strided ? PS_WAVES * pslice_kpw(strided, Kp) : PS_ROW_NPB;
    return (Kp / PANEL_K + npb - 1) / npb;
}
__host__ __device__ inline bool pslice_route(bool strided, int Kp) {
    const int cap = pslice_kpw(strided, Kp) == PS_KPW_WIDE ? PS_MAX_PARTS_WIDE : PS_MAX_PARTS;
    return Kp > (strided ? ONEPASS_MAX_K_COLUMNS : ONEPASS_MAX_K) && pslice_parts(strided, Kp) <= cap;
}
// Polls of a block's wait for the other parts of its panel before it reads their k ranges
// itself (rg_test_set_spin_limit sets it; 0: no exchange, every block reads its panel's whole K
// for the maxima). A poll (one L2 round trip per eight parts, then a short sleep) took about
// 0.45 us on MI355X when it read the slots one at a time, so the default bounds the wait at
// about 1 ms or less, far past a normal wait (parts that load together publish within a few
// tens of us).
constexpr int DEFAULT_SPIN_LIMIT = 2048;
int slice_spin_limit();
void set_slice_spin_limit(int polls);
// Fills ps_parts / ps_blocks of d (spin_limit is the caller's).
void pslice_grid(SliceDesc& d);
// Unit of one-read slicing block blk (units: panel or strip x part, in panel order). Block blk
// runs on XCD blk % 8, and each XCD takes a contiguous range of ps_blocks / 8 units, which
// pslice_grid makes a whole number of panels (or strips): the parts of a panel, which exchange
// their maxima through the XCD's L2, then all run on one XCD.
__host__ __device__ inline long long pslice_unit(long long blk, long long ps_blocks) {
    return (blk & 7) * (ps_blocks / 8) + (blk >> 3);
}
// The partial-maximum slots the one read of d waits on.
MarkRange pslice_slots(const SliceDesc& d);
void launch_pslice(const SliceDesc& a, bool use_a, const SliceDesc& b, bool use_b, int S,
                   hipStream_t stream);
// One launch: the one read of `two` and the one pass of `one` (padded K <= ONEPASS_MAX_K).
void launch_onepass_pslice(const SliceDesc& one, const SliceDesc& two, int S, hipStream_t stream);
// One launch: the one read of `ps` and the partial maxima of `two` (whose split follows).
void launch_pslice_absmax(const SliceDesc& ps, const SliceDesc& two, int S, hipStream_t stream);
// Marks two regions of slots PM_EMPTY (one small launch).
void launch_mark(MarkRange a, MarkRange b, hipStream_t stream);
// One launch: the one pass of `one` and the partial maxima of `two` (whose split follows).
void launch_onepass_absmax(const SliceDesc& one, const SliceDesc& two, int S, hipStream_t stream);

// Options of the launch sequence beyond the reference's GEMM, for the convolution's input
// gradient: group_a > 0 gives every group of group_a consecutive rows of op(A) one scale (the
// largest magnitude in the group; group_a >= M: one scale for all), likewise group_b for the
// columns of op(B); raw keeps the exact int64 sums in the workspace's partial buffer.
struct GemmOptions {
    int group_a = 0;
    int group_b = 0;
    bool raw = false;
    // op(A) gathered from an image tensor instead of read from A (the convolution's forward
    // pass on the implicit im2col matrix); needs the one-pass route (padded K <= ONEPASS_MAX_K,
    // no group scales, one item).
    const Im2col* im2col_a = nullptr;
    // Row flags of op(A) and of op(B)^T (SliceDesc::nanrows), padded to Mp and Np rows.
    const unsigned* nanrows_a = nullptr;
    const unsigned* nanrows_b = nullptr;
};

// Layout for the current device (queried once per device and cached).
int layout_for_current_device(int M, int N, int K, const rg_config* cfg, Layout* L,
                              const PlanExtras& extras = PlanExtras());

// Operand and output addressing of a launch: leading dimensions and, for a batch, the element
// strides between items. Plain row-major operands have lda = K (or M when transposed),
// ldb = N (or K), ldc = N.
struct GemmAddressing {
    long long lda, ldb, ldc;
    long long stride_a, stride_b, stride_c;
};
GemmAddressing dense_addressing(const Layout& L);

// The launch sequence of L.batch GEMMs on `stream` (slicing, contraction, final rounding
// unless raw) into a workspace laid out by L at `base`. events: NULL or 4 hipEvent_t.
int gemm_launch(const float* A, const float* B, float* C, const Layout& L, char* base,
                hipStream_t stream, void* const* events, const GemmOptions& opt,
                const GemmAddressing& addr);

// Kernel launchers (asynchronous on `stream`).
void launch_absmax(const SliceDesc& a, const SliceDesc& b, hipStream_t stream);
void launch_split(const SliceDesc& a, const SliceDesc& b, int S, bool int32_out, hipStream_t stream);
// Replaces the partial row maxima of d by the maximum over each group of `group` rows.
void launch_group_max(const SliceDesc& d, int group, hipStream_t stream);
// Both operands' group maxima in one launch (a null operand or a group <= 0 is skipped).
void launch_group_max2(const SliceDesc* a, int group_a, const SliceDesc* b, int group_b,
                       hipStream_t stream);
// Output addressing of the contraction and the final rounding: C of item b at
// C + b * c_item, rows ldc apart.
struct OutAddr {
    long long ldc, c_item;
};
void launch_contract_mfma(const Layout& L, const int8_t* qa, const int8_t* qb, const int* ea,
                          const int* eb, float* C, OutAddr out, int64_t* partial,
                          hipStream_t stream);
// Whole GEMM (or batch) in one launch, for a layout with L.small.
void launch_contract_small(const Layout& L, const float* A, const float* B, float* C,
                           const GemmAddressing& addr, hipStream_t stream);
// Slicing of op(A), contraction and rounding in one launch, for a layout with L.band_w > 0
// (op(B)'s digit panels qb and exponents eb already in the workspace).
void launch_contract_band(const Layout& L, const float* A, long long lda, const int8_t* qb,
                          const int* eb, float* C, long long ldc, hipStream_t stream);
void launch_contract_reference(const Layout& L, const int32_t* xa, const int32_t* xb,
                               int64_t* partial, hipStream_t stream);
void launch_reduce_round(const Layout& L, const int64_t* partial, const int* ea, const int* eb,
                         float* C, OutAddr out, hipStream_t stream);
// The epilogue roundings on arrays (rg_test_round): levels != nullptr rounds n x (2S-1) int32
// levels as the contraction's epilogue does, else n int64 values as reduce_round does.
void launch_test_round(const int* levels, const int64_t* T, const int* E, float* out, long long n,
                       int S, hipStream_t stream);

}  // namespace rg
