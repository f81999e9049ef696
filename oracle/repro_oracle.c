/*
 * repro_oracle.c -- CPU restatement of the reproducible FP32 GEMM definition.
 * TEST INFRASTRUCTURE ONLY (see repro_oracle.h): the product never links this.
 *
 * The definition (reference README and repro_gemm_cuda/repro_gemm.cuh:8-21):
 *   eA[r] = scale_exponent(max_k |op(A)[r,k]|),  eB[c] likewise over op(B)[.,c];
 *   X[r,k] = fixed_point(op(A)[r,k], eA[r], S),  Y[c,k] = fixed_point(op(B)[k,c], eB[c], S);
 *   T[r,c] = sum_k X[r,k] * Y[c,k]  exactly (int64);
 *   C[r,c] = round_to_float(T[r,c], eA[r] + eB[c] - 14 (S - 1)).
 */
#include "repro_oracle.h"

#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------- */
/* Scalars                                                                   */
/* ------------------------------------------------------------------------- */

static uint32_t f2u(float x) { uint32_t b; memcpy(&b, &x, 4); return b; }
static float u2f(uint32_t b) { float x; memcpy(&x, &b, 4); return x; }

/* x * 2^n as two multiplications by normal powers of two; exact except when the
 * result is subnormal, where it rounds once (repro_gemm_math.cuh:44-55). */
float oracle_scale_by_pow2(float x, int n) {
    int n1 = n >> 1;
    int n2 = n - n1;
    float p1 = u2f((uint32_t)(n1 + 127) << 23);
    float p2 = u2f((uint32_t)(n2 + 127) << 23);
    float t = x * p1;
    return t * p2;
}

/* Smallest e with 2^e >= fl32(m / 127); 0 when m / 127 is zero or m is not positive
 * (repro_gemm_math.cuh:57-69). For a normal quotient the exponent comes from its bits;
 * for a subnormal quotient from frexpf. */
int oracle_scale_exponent(float m) {
    if (!(m > 0.0f)) return 0;
    float v = m / 127.0f;
    uint32_t b = f2u(v);
    int E = (int)((b >> 23) & 0xFFu);
    if (E != 0) return (b & 0x7FFFFFu) == 0 ? E - 127 : E - 126;
    int e;
    float frac = frexpf(v, &e);
    if (frac == 0.0f) return 0;
    return frac == 0.5f ? e - 1 : e;
}

/* X = RNE(x * 2^(7(S-1) - se)), clamped to |X| <= 127 * 2^(7(S-1))
 * (repro_gemm_math.cuh:71-83). */
int oracle_fixed_point(float x, int se, int S) {
    float v = oracle_scale_by_pow2(x, 7 * (S - 1) - se);
    /* The reference converts with (int)nearbyintf(v); for a NaN or an infinity that is INT_MIN
     * on x86 (the "integer indefinite" of cvttss2si), stated here without the undefined cast. */
    int X = isfinite(v) ? (int)nearbyintf(v) : INT_MIN;
    int lim = 127 << (7 * (S - 1));
    return X > lim ? lim : (X < -lim ? -lim : X);
}

/* Correctly rounded (nearest-even) binary32 value of T * 2^E with subnormals,
 * signed zero for negative T below the smallest subnormal, and overflow to
 * infinity (repro_gemm_math.cuh:85-119). */
float oracle_round_to_float(int64_t T, int E) {
    if (T == 0) return 0.0f;
    int neg = T < 0;
    uint64_t m = neg ? (uint64_t)(-(T + 1)) + 1u : (uint64_t)T;
    int p = 63 - __builtin_clzll(m);
    int shift = p - 23;
    if (-149 - E > shift) shift = -149 - E;
    uint64_t q;
    int ex;
    if (shift <= 0) {
        q = m;
        ex = E;
    } else if (shift >= 64) {
        q = 0;
        ex = 0;
    } else {
        q = m >> shift;
        uint64_t rem = m & ((1ull << shift) - 1);
        uint64_t half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        ex = E + shift;
    }
    float f = (q != 0 && ex > 127) ? u2f(0x7F800000u) : oracle_scale_by_pow2((float)q, ex);
    return neg ? -f : f;
}

void oracle_scale_exponent_n(const float* m, int* e, size_t n) {
    for (size_t i = 0; i < n; ++i) e[i] = oracle_scale_exponent(m[i]);
}

void oracle_fixed_point_n(const float* x, const int* se, int S, int* X, size_t n) {
    for (size_t i = 0; i < n; ++i) X[i] = oracle_fixed_point(x[i], se[i], S);
}

void oracle_round_to_float_n(const int64_t* T, const int* E, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_round_to_float(T[i], E[i]);
}

/* ------------------------------------------------------------------------- */
/* Thread pool: threads pull indices from one atomic counter                  */
/* (repro_gemm_cuda/repro_gemm_cpu.h:14-23). Results never depend on it.     */
/* ------------------------------------------------------------------------- */

typedef void (*body_fn)(void* ctx, int i);

typedef struct {
    atomic_int next;
    int n;
    body_fn fn;
    void* ctx;
} pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    for (int i; (i = atomic_fetch_add(&p->next, 1)) < p->n;) p->fn(p->ctx, i);
    return NULL;
}

static int resolve_threads(int nthreads) {
    if (nthreads > 0) return nthreads;
    const char* env = getenv("REPRO_CPU_THREADS");
    if (env && atoi(env) > 0) return atoi(env);
    long hc = sysconf(_SC_NPROCESSORS_ONLN);
    return hc > 0 ? (int)hc : 1;
}

static void par_for(int n, int nthreads, body_fn fn, void* ctx) {
    pool_t p;
    atomic_init(&p.next, 0);
    p.n = n;
    p.fn = fn;
    p.ctx = ctx;
    if (nthreads <= 1 || n <= 1) {
        pool_worker(&p);
        return;
    }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
    int started = 0;
    for (int t = 0; t < nthreads; ++t)
        if (pthread_create(&th[t], NULL, pool_worker, &p) == 0) ++started;
    if (started == 0) pool_worker(&p);
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
    free(th);
}

/* ------------------------------------------------------------------------- */
/* Independent check of scale_exponent: fl32(m / 127) by exact integer        */
/* division with round-to-nearest-even, then the smallest power of two >= it. */
/* ------------------------------------------------------------------------- */

static int scale_exponent_integer(uint32_t bits) {
    uint32_t be = (bits >> 23) & 0xFFu, fr = bits & 0x7FFFFFu;
    if (be == 0 && fr == 0) return 0;
    uint64_t a = be ? (fr | 0x800000u) : fr; /* m = a * 2^q */
    int q = be ? (int)be - 150 : -149;
    uint64_t num = a << 40;                  /* m / 127 = (N + rem/127) * 2^(q-40) */
    uint64_t N = num / 127u, rem = num % 127u;
    int p = 63 - __builtin_clzll(N);
    int d = p - 23;                          /* bits to drop for 24 significant bits */
    if (-149 - (q - 40) > d) d = -149 - (q - 40); /* nothing below 2^-149 */
    uint64_t kept = N >> d, low = N & ((1ull << d) - 1), half = 1ull << (d - 1);
    if (low > half || (low == half && (rem != 0 || (kept & 1)))) ++kept;
    if (kept == 0) return 0;                 /* the quotient rounded to zero */
    int w = q - 40 + d;                      /* v = kept * 2^w */
    int pk = 63 - __builtin_clzll(kept);
    return (kept == (1ull << pk)) ? pk + w : pk + w + 1;
}

typedef struct {
    uint32_t lo, hi;
    int chunks;
    atomic_ullong bad;
    atomic_uint first;
} se_check_t;

static void se_check_body(void* ctx, int i) {
    se_check_t* c = (se_check_t*)ctx;
    uint64_t span = (uint64_t)c->hi - c->lo;
    uint32_t a = c->lo + (uint32_t)(span * (uint64_t)i / (uint64_t)c->chunks);
    uint32_t b = c->lo + (uint32_t)(span * (uint64_t)(i + 1) / (uint64_t)c->chunks);
    uint64_t bad = 0;
    uint32_t first = 0xFFFFFFFFu;
    for (uint32_t x = a; x < b; ++x) {
        if (oracle_scale_exponent(u2f(x)) != scale_exponent_integer(x)) {
            if (!bad) first = x;
            ++bad;
        }
    }
    if (bad) {
        atomic_fetch_add(&c->bad, bad);
        uint32_t cur = atomic_load(&c->first);
        while (first < cur && !atomic_compare_exchange_weak(&c->first, &cur, first)) {
        }
    }
}

uint64_t oracle_check_scale_exponent_range(uint32_t lo, uint32_t hi, uint32_t* first) {
    se_check_t c;
    c.lo = lo;
    c.hi = hi;
    c.chunks = 1024;
    atomic_init(&c.bad, 0);
    atomic_init(&c.first, 0xFFFFFFFFu);
    if (hi > lo) par_for(c.chunks, resolve_threads(0), se_check_body, &c);
    if (first) *first = atomic_load(&c.first);
    return atomic_load(&c.bad);
}

/* ------------------------------------------------------------------------- */
/* The GEMM                                                                  */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float* A;
    const float* B;
    float* C;
    int M, N, K, ta, tb, S, r0;
    int32_t* X;
    int32_t* Y;
    int* eA;
    int* eB;
    int64_t* T;
} gemm_ctx;

static float a_at(const gemm_ctx* g, int r, int k) {
    return g->ta ? g->A[(size_t)k * g->M + r] : g->A[(size_t)r * g->K + k];
}
static float b_at(const gemm_ctx* g, int k, int c) {
    return g->tb ? g->B[(size_t)c * g->K + k] : g->B[(size_t)k * g->N + c];
}

/* repro_gemm_cpu.h:30-35: row max, exponent, fixed point of every element of row r. */
static void quant_row(void* ctx, int r) {
    gemm_ctx* g = (gemm_ctx*)ctx;
    float m = 0.0f;
    for (int k = 0; k < g->K; ++k) m = fmaxf(m, fabsf(a_at(g, r, k)));
    int e = oracle_scale_exponent(m);
    g->eA[r] = e;
    int32_t* x = g->X + (size_t)r * g->K;
    for (int k = 0; k < g->K; ++k) x[k] = oracle_fixed_point(a_at(g, r, k), e, g->S);
}

/* repro_gemm_cpu.h:36-41: the same per column of op(B), stored transposed. */
static void quant_col(void* ctx, int c) {
    gemm_ctx* g = (gemm_ctx*)ctx;
    float m = 0.0f;
    for (int k = 0; k < g->K; ++k) m = fmaxf(m, fabsf(b_at(g, k, c)));
    int e = oracle_scale_exponent(m);
    g->eB[c] = e;
    int32_t* y = g->Y + (size_t)c * g->K;
    for (int k = 0; k < g->K; ++k) y[k] = oracle_fixed_point(b_at(g, k, c), e, g->S);
}

/* repro_gemm_cpu.h:42-50: exact int64 dot products, one rounding per output. */
static void dot_row(void* ctx, int i) {
    gemm_ctx* g = (gemm_ctx*)ctx;
    int r = g->r0 + i;
    const int32_t* x = g->X + (size_t)r * g->K;
    for (int c = 0; c < g->N; ++c) {
        const int32_t* y = g->Y + (size_t)c * g->K;
        int64_t t = 0;
        for (int k = 0; k < g->K; ++k) t += (int64_t)x[k] * y[k];
        g->C[(size_t)i * g->N + c] = oracle_round_to_float(t, g->eA[r] + g->eB[c] - 14 * (g->S - 1));
    }
}

static void exact_row(void* ctx, int r) {
    gemm_ctx* g = (gemm_ctx*)ctx;
    const int32_t* x = g->X + (size_t)r * g->K;
    for (int c = 0; c < g->N; ++c) {
        const int32_t* y = g->Y + (size_t)c * g->K;
        int64_t t = 0;
        for (int k = 0; k < g->K; ++k) t += (int64_t)x[k] * y[k];
        g->T[(size_t)r * g->N + c] = t;
    }
}

void oracle_quantize(const float* A, const float* B, int M, int N, int K, int ta, int tb, int S,
                     int32_t* X, int32_t* Y, int* eA, int* eB, int nthreads) {
    gemm_ctx g;
    memset(&g, 0, sizeof g);
    g.A = A; g.B = B; g.M = M; g.N = N; g.K = K; g.ta = ta; g.tb = tb; g.S = S;
    g.X = X; g.Y = Y; g.eA = eA; g.eB = eB;
    int nt = resolve_threads(nthreads);
    par_for(M, nt, quant_row, &g);
    par_for(N, nt, quant_col, &g);
}

void oracle_exact_products(const int32_t* X, const int32_t* Y, int64_t* T, int M, int N, int K,
                           int nthreads) {
    gemm_ctx g;
    memset(&g, 0, sizeof g);
    g.M = M; g.N = N; g.K = K;
    g.X = (int32_t*)X; g.Y = (int32_t*)Y; g.T = T;
    par_for(M, resolve_threads(nthreads), exact_row, &g);
}

static void quant_row_off(void* ctx, int i) { quant_row(ctx, ((gemm_ctx*)ctx)->r0 + i); }

int oracle_cpu_gemm_rows(const float* A, const float* B, float* C, int M, int N, int K, int ta,
                         int tb, int S, int r0, int r1, int nthreads) {
    int nt = resolve_threads(nthreads);
    if (M <= 0 || N <= 0 || K <= 0 || r0 < 0 || r1 > M || r0 >= r1) return nt;
    gemm_ctx g;
    memset(&g, 0, sizeof g);
    g.A = A; g.B = B; g.C = C; g.M = M; g.N = N; g.K = K; g.ta = ta; g.tb = tb; g.S = S;
    g.r0 = r0;
    g.X = (int32_t*)malloc(sizeof(int32_t) * (size_t)M * (size_t)K);
    g.Y = (int32_t*)malloc(sizeof(int32_t) * (size_t)N * (size_t)K);
    g.eA = (int*)malloc(sizeof(int) * (size_t)M);
    g.eB = (int*)malloc(sizeof(int) * (size_t)N);
    if (g.X && g.Y && g.eA && g.eB) {
        par_for(r1 - r0, nt, quant_row_off, &g); /* only the rows that are computed */
        par_for(N, nt, quant_col, &g);
        par_for(r1 - r0, nt, dot_row, &g);
    }
    free(g.X); free(g.Y); free(g.eA); free(g.eB);
    return nt;
}

int oracle_cpu_gemm(const float* A, const float* B, float* C, int M, int N, int K, int ta, int tb,
                    int S, int nthreads) {
    return oracle_cpu_gemm_rows(A, B, C, M, N, K, ta, tb, S, 0, M, nthreads);
}

/* ------------------------------------------------------------------------- */
/* Portable inputs and hashing                                               */
/* ------------------------------------------------------------------------- */

/* SplitMix64 (repro_test_util.h:30-37): the generator adds the golden gamma to its state
 * and mixes; draw i of the stream seeded with s is therefore mix(s + (i+1) * gamma), which
 * lets the generators below fill disjoint ranges in parallel with identical bits. */
static uint64_t sm_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static uint64_t sm_draw(uint64_t seed, uint64_t i) { return sm_mix(seed + (i + 1) * 0x9e3779b97f4a7c15ull); }

/* 24 random bits scaled to [0, 1): exact in double (repro_test_util.h:38). */
static double sm_u01_at(uint64_t seed, uint64_t i) { return (double)(sm_draw(seed, i) >> 40) * (1.0 / 16777216.0); }

void oracle_splitmix64(uint64_t* out, size_t n, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) out[i] = sm_draw(seed, i);
}

enum { GEN_NORMAL, GEN_UNIFORM, GEN_UNIFORM_PM, GEN_ADVERSARIAL };

typedef struct {
    float* out;
    size_t n;
    double scale;
    uint64_t seed, first;
    int kind;
    int chunks;
    int cols;      /* adversarial: row length */
    int pair_rows; /* adversarial: pairs are (r, r^1) instead of (c, c^1) */
    int negate;    /* adversarial: second of a pair is negated */
} gen_ctx;

/* Adversarial base element: 5% exact zeros, 1% subnormals, otherwise +-2^e with e uniform
 * in [-60, 60]. */
static float adversarial_base(uint64_t seed, uint64_t idx) {
    uint64_t u = sm_draw(seed, 2 * idx);
    uint64_t v = sm_draw(seed, 2 * idx + 1);
    unsigned pct = (unsigned)(u % 100u);
    uint32_t sign = (uint32_t)((v >> 63) & 1u) << 31;
    uint32_t bits;
    if (pct < 5) {
        bits = 0;
    } else if (pct < 6) {
        uint32_t f = (uint32_t)((v >> 8) & 0x7FFFFFu);
        bits = f ? f : 1u;
    } else {
        int e = (int)((v >> 16) % 121u) - 60;
        bits = (uint32_t)(e + 127) << 23;
    }
    uint32_t b = sign | bits;
    float x;
    memcpy(&x, &b, 4);
    return x;
}

static void gen_body(void* vctx, int c) {
    gen_ctx* g = (gen_ctx*)vctx;
    size_t a = g->n * (size_t)c / (size_t)g->chunks, b = g->n * (size_t)(c + 1) / (size_t)g->chunks;
    for (size_t i = a; i < b; ++i) {
        uint64_t idx = g->first + i;
        switch (g->kind) {
            case GEN_NORMAL: {
                double t = 0.0;
                for (int j = 0; j < 12; ++j) t += sm_u01_at(g->seed, 12 * idx + (uint64_t)j);
                g->out[i] = (float)(g->scale * (t - 6.0));
                break;
            }
            case GEN_UNIFORM:
                g->out[i] = (float)(g->scale * sm_u01_at(g->seed, idx));
                break;
            case GEN_UNIFORM_PM: {
                /* float32 arithmetic as repro_torch/utils.py:23-29: u = bits * 2^-24 (exact),
                 * v = u * (2 * bound) - bound, each a single float32 rounding. */
                float bound = (float)g->scale;
                float u = (float)(sm_draw(g->seed, idx) >> 40) * (1.0f / 16777216.0f);
                float two_b = 2.0f * bound;
                float t = u * two_b;
                g->out[i] = t - bound;
                break;
            }
            case GEN_ADVERSARIAL: {
                /* Elements come in pairs along k: the second of a pair is the first times
                 * (1 + 2^-20 t), t in {-1, 0, 1}, and negated when g->negate is set. An
                 * operand with negated pairs times one with plain pairs cancels almost
                 * exactly in every dot product. */
                size_t r = i / (size_t)g->cols, c = i % (size_t)g->cols;
                size_t base, second;
                if (g->pair_rows) {
                    base = (r & ~(size_t)1) * (size_t)g->cols + c;
                    second = r & 1;
                } else {
                    base = r * (size_t)g->cols + (c & ~(size_t)1);
                    second = c & 1;
                }
                float x = adversarial_base(g->seed, base);
                if (second) {
                    uint64_t w = sm_draw(g->seed ^ 0x5bd1e995ull, base);
                    int t = (int)(w % 3u) - 1;
                    float f = 1.0f + (float)t * (1.0f / 1048576.0f);
                    x = x * f;
                    if (g->negate) x = -x;
                }
                g->out[i] = x;
                break;
            }
        }
    }
}

static void gen_run(float* out, size_t n, double scale, uint64_t seed, uint64_t first, int kind, int cols) {
    gen_ctx g;
    memset(&g, 0, sizeof g);
    g.out = out; g.n = n; g.scale = scale; g.seed = seed; g.first = first; g.kind = kind;
    g.cols = cols > 0 ? cols : 1;
    g.chunks = n < 65536 ? 1 : 256;
    par_for(g.chunks, g.chunks == 1 ? 1 : resolve_threads(0), gen_body, &g);
}

/* Irwin-Hall: sum of twelve U[0,1) minus 6, exact in double (repro_test_util.h:41). */
void oracle_gen_normal(float* out, size_t n, double scale, uint64_t seed) {
    gen_run(out, n, scale, seed, 0, GEN_NORMAL, 0);
}
void oracle_gen_normal_at(float* out, size_t n, double scale, uint64_t seed, uint64_t first_elem) {
    gen_run(out, n, scale, seed, first_elem, GEN_NORMAL, 0);
}
void oracle_gen_uniform(float* out, size_t n, double scale, uint64_t seed) {
    gen_run(out, n, scale, seed, 0, GEN_UNIFORM, 0);
}
void oracle_gen_uniform_pm(float* out, size_t n, float bound, uint64_t seed, uint64_t first_elem) {
    gen_run(out, n, (double)bound, seed, first_elem, GEN_UNIFORM_PM, 0);
}
/* The input distributions of the reference's hash tool (repro_gemm_cuda/hash_repro_gemm.cu:20-56),
 * drawn in its order from one sequential SplitMix64 stream with the Rng helpers of
 * repro_test_util.h:29-47: u01 = (next >> 40) 2^-24; normal = sum of 12 u01 - 6 in double;
 * range(lo, hi) = lo + next % (hi - lo + 1); wide(lo, hi) = +-(1 + u01) 2^range(lo, hi), the
 * sign from the next draw's low bit. A is MxK, B is KxN, row-major. dist: 0 uniform U[-1,1),
 * 1 normal, 2 weights (0.02 normal, x100 when the following draw % 1000 == 0), 3 wide
 * (2^[-40,40]), 4 stress (normal, then rows of A by r % 8 and columns of B by c % 6 replaced by
 * zeros, subnormals, 1e30-scaled values, one 1e6 outlier, signed zeros, 2^[-60,60] values or
 * 2^-120-scaled values). */
typedef struct { uint64_t s; } seq_rng;
static uint64_t seq_next(seq_rng* g) { g->s += 0x9e3779b97f4a7c15ull; return sm_mix(g->s); }
static double seq_u01(seq_rng* g) { return (double)(seq_next(g) >> 40) * (1.0 / 16777216.0); }
static double seq_normal(seq_rng* g) {
    double t = 0.0;
    for (int i = 0; i < 12; ++i) t += seq_u01(g);
    return t - 6.0;
}
static int seq_range(seq_rng* g, int lo, int hi) { return lo + (int)(seq_next(g) % (uint64_t)(hi - lo + 1)); }
static float seq_wide(seq_rng* g, int lo, int hi) {
    double mant = 1.0 + seq_u01(g);
    double v = ldexp(mant, seq_range(g, lo, hi));
    return (float)((seq_next(g) & 1) ? -v : v);
}
static float seq_dist(seq_rng* g, int dist) {
    switch (dist) {
        case 0: return (float)(2.0 * seq_u01(g) - 1.0);
        case 2: {
            double v = 0.02 * seq_normal(g);
            return (float)((seq_next(g) % 1000 == 0) ? v * 100.0 : v);
        }
        case 3: return seq_wide(g, -40, 40);
        default: return (float)seq_normal(g);
    }
}

int oracle_gen_hash_inputs(float* A, float* B, int M, int N, int K, uint64_t seed, int dist) {
    if (dist < 0 || dist > 4 || M <= 0 || N <= 0 || K <= 0) return 1;
    seq_rng g = {seed};
    size_t nA = (size_t)M * K, nB = (size_t)K * N;
    for (size_t i = 0; i < nA; ++i) A[i] = seq_dist(&g, dist);
    for (size_t i = 0; i < nB; ++i) B[i] = seq_dist(&g, dist);
    if (dist != 4) return 0;
    for (int r = 0; r < M; ++r) {
        float* row = A + (size_t)r * K;
        switch (r % 8) {
            case 1: for (int k = 0; k < K; ++k) row[k] = 0.0f; break;
            case 2: for (int k = 0; k < K; ++k) row[k] = (float)ldexp(seq_normal(&g), -140); break;
            case 3: for (int k = 0; k < K; ++k) row[k] = (float)(1e30 * seq_normal(&g)); break;
            case 4: row[seq_range(&g, 0, K - 1)] = 1e6f; break;
            case 5: for (int k = 0; k < K; ++k) row[k] = (k & 1) ? -0.0f : 0.0f; break;
            default: break;
        }
    }
    for (int c = 0; c < N; ++c) {
        switch (c % 6) {
            case 1: for (int k = 0; k < K; ++k) B[(size_t)k * N + c] = 0.0f; break;
            case 2: for (int k = 0; k < K; ++k) B[(size_t)k * N + c] = seq_wide(&g, -60, 60); break;
            case 3: for (int k = 0; k < K; ++k) B[(size_t)k * N + c] = (float)ldexp(seq_normal(&g), -120); break;
            default: break;
        }
    }
    return 0;
}

void oracle_gen_adversarial(float* out, int rows, int cols, uint64_t seed, int pair_rows, int negate) {
    gen_ctx g;
    memset(&g, 0, sizeof g);
    g.out = out; g.n = (size_t)rows * (size_t)cols; g.scale = 1.0; g.seed = seed;
    g.kind = GEN_ADVERSARIAL; g.cols = cols; g.pair_rows = pair_rows; g.negate = negate;
    g.chunks = g.n < 65536 ? 1 : 256;
    par_for(g.chunks, g.chunks == 1 ? 1 : resolve_threads(0), gen_body, &g);
}

uint64_t oracle_fnv1a64(const void* data, size_t n, uint64_t h) {
    const unsigned char* p = (const unsigned char*)data;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

/* ------------------------------------------------------------------------- */
/* Exact sum (superaccumulator), repro_sum_cuda/repro_sum_math.cuh            */
/* ------------------------------------------------------------------------- */

#define SUM_LIMBS 10

/* Adds x as two integer addends at its limb pair; 0 for NaN/Inf
 * (repro_sum_math.cuh:66-91). Limb l weighs 2^(32 l - 149). */
static int sum_add(int64_t* acc, float x) {
    uint32_t b = f2u(x), e = (b >> 23) & 0xFFu, f = b & 0x7FFFFFu;
    if (e == 0xFFu) return 0;
    uint64_t m = e ? (uint64_t)(f | 0x800000u) : (uint64_t)f;
    int sh = e ? (int)e - 1 : 0;
    uint64_t v = m << (sh & 31);
    int64_t lo = (int64_t)(v & 0xFFFFFFFFull), hi = (int64_t)(v >> 32);
    if (b >> 31) { lo = -lo; hi = -hi; }
    acc[sh >> 5] += lo;
    acc[(sh >> 5) + 1] += hi;
    return 1;
}

/* Carries with floor division by 2^32 (repro_sum_math.cuh:93-100). */
static void sum_normalize(int64_t* t) {
    for (int l = 0; l < SUM_LIMBS - 1; ++l) {
        int64_t c = t[l] >> 32;
        t[l] -= c * 4294967296LL;
        t[l + 1] += c;
    }
}

/* Exact value / divisor rounded once, nearest-even, by long division and guard/sticky
 * bits (repro_sum_math.cuh:102-157). */
static float sum_finalize(int64_t* t, uint32_t divisor, int nonfinite) {
    if (nonfinite) return u2f(0x7FC00000u);
    sum_normalize(t);
    int neg = t[SUM_LIMBS - 1] < 0;
    if (neg) {
        for (int l = 0; l < SUM_LIMBS; ++l) t[l] = -t[l];
        sum_normalize(t);
    }
    uint32_t q[SUM_LIMBS];
    uint64_t rem = 0;
    for (int l = SUM_LIMBS - 1; l >= 0; --l) {
        uint64_t cur = (rem << 32) | (uint64_t)(uint32_t)t[l];
        q[l] = (uint32_t)(cur / divisor);
        rem = cur % divisor;
    }
    int top = SUM_LIMBS - 1;
    while (top >= 0 && q[top] == 0) --top;
    float r;
    if (top < 0) {
        if (rem == 0) return 0.0f;
        r = (2 * rem > divisor) ? u2f(1u) : 0.0f;       /* 2^-149 or 0 (a tie is even: 0) */
        return neg ? -r : r;
    }
    int p = 32 * top + 31 - __builtin_clz(q[top]);
    int shift = p > 23 ? p - 23 : 0;
    int kl = shift >> 5;
    uint64_t two = (uint64_t)q[kl] | (kl + 1 < SUM_LIMBS ? (uint64_t)q[kl + 1] << 32 : 0u);
    uint32_t kept = (uint32_t)(two >> (shift & 31)) & 0xFFFFFFu;
    int up;
    if (shift > 0) {
        int g = shift - 1;
        int guard = (q[g >> 5] >> (g & 31)) & 1u;
        int lower = rem != 0;
        for (int l = 0; l < (g >> 5); ++l) lower = lower || q[l] != 0;
        lower = lower || (q[g >> 5] & ((1u << (g & 31)) - 1u)) != 0;
        up = guard && (lower || (kept & 1u));
    } else {
        up = 2 * rem > divisor || (2 * rem == divisor && (kept & 1u));
    }
    kept += (uint32_t)up;
    r = ldexpf((float)kept, shift - 149);
    return neg ? -r : r;
}

/* out[b] = exact sum over a, c of x[a][b][c], rounded once; divided exactly by A*C when
 * mean (repro_torch/src/bindings.cpp:69-91, CPU branch). */
void oracle_exact_sum(const float* x, float* out, int A, int B, int C, int mean) {
    uint32_t divisor = mean ? (uint32_t)((int64_t)A * C) : 1u;
    for (int b = 0; b < B; ++b) {
        int64_t acc[SUM_LIMBS] = {0};
        int nonfinite = 0;
        for (int a = 0; a < A; ++a)
            for (int c = 0; c < C; ++c)
                if (!sum_add(acc, x[((size_t)a * B + b) * C + c])) nonfinite = 1;
        out[b] = sum_finalize(acc, divisor, nonfinite);
    }
}

/* 1 if x holds a NaN or infinity (exponent field all ones), else 0
 * (the test of repro_torch/src/kernels.cu:10-14). */
int oracle_has_nonfinite(const float* x, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if ((f2u(x[i]) & 0x7F800000u) == 0x7F800000u) return 1;
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Convolution, repro_conv_cuda/repro_conv_math.cuh and repro_conv_cpu.h      */
/* ------------------------------------------------------------------------- */

/* Input value at position (c, ky, kx) of window (n, oy, ox), zero in the padding
 * (repro_conv_math.cuh:46-52). */
static float conv_window_value(const float* x, const oracle_conv_shape* g, int n, int oy, int ox,
                               int c, int ky, int kx) {
    int y = oy * g->SY - g->PY + ky, xx = ox * g->SX - g->PX + kx;
    if (y < 0 || y >= g->H || xx < 0 || xx >= g->W) return 0.0f;
    return x[(((size_t)n * g->C + c) * g->H + y) * g->W + xx];
}

static int conv_oh(const oracle_conv_shape* g) { return (g->H + 2 * g->PY - g->KH) / g->SY + 1; }
static int conv_ow(const oracle_conv_shape* g) { return (g->W + 2 * g->PX - g->KW) / g->SX + 1; }

/* Largest magnitude bit pattern of m and x: the window and position maxima of the reference's
 * convolution compare raw magnitude bits (repro_conv_math.cuh:73-86, 121-130), so a NaN (whose
 * bits exceed +inf's) wins them and its window or position gets exponent 0; the filter and dY
 * maxima use std::max on values, which skips a NaN (repro_conv_cpu.h:29, 48, 77, 82). */
static uint32_t conv_bits_max(uint32_t m, float x) {
    uint32_t a = f2u(x) & 0x7FFFFFFFu;
    return a > m ? a : m;
}

/* Forward (repro_conv_cpu.h:23-38, repro_conv_math.cuh:68-99): weights quantised per filter,
 * each window per window, Y[n][f][oy][ox] = round(sum_k X * W, e_window + e_filter + e0). */
void oracle_conv2d(const float* x, const float* w, float* out, const oracle_conv_shape* g, int S) {
    int K = g->C * g->KH * g->KW, oh = conv_oh(g), ow = conv_ow(g), e0 = -14 * (S - 1);
    int* Wq = (int*)malloc(sizeof(int) * (size_t)g->F * K);
    int* eF = (int*)malloc(sizeof(int) * (size_t)g->F);
    int* q = (int*)malloc(sizeof(int) * (size_t)K);
    float* v = (float*)malloc(sizeof(float) * (size_t)K);
    for (int f = 0; f < g->F; ++f) {
        float m = 0.0f;
        for (int k = 0; k < K; ++k) m = fmaxf(m, fabsf(w[(size_t)f * K + k]));
        eF[f] = oracle_scale_exponent(m);
        for (int k = 0; k < K; ++k) Wq[(size_t)f * K + k] = oracle_fixed_point(w[(size_t)f * K + k], eF[f], S);
    }
    for (int n = 0; n < g->N; ++n)
        for (int oy = 0; oy < oh; ++oy)
            for (int ox = 0; ox < ow; ++ox) {
                uint32_t mb = 0;
                for (int k = 0; k < K; ++k) {
                    int c = k / (g->KH * g->KW), r = k % (g->KH * g->KW);
                    v[k] = conv_window_value(x, g, n, oy, ox, c, r / g->KW, r % g->KW);
                    mb = conv_bits_max(mb, v[k]);
                }
                int e = oracle_scale_exponent(u2f(mb));
                for (int k = 0; k < K; ++k) q[k] = oracle_fixed_point(v[k], e, S);
                for (int f = 0; f < g->F; ++f) {
                    int64_t t = 0;
                    for (int k = 0; k < K; ++k) t += (int64_t)q[k] * Wq[(size_t)f * K + k];
                    out[(((size_t)n * g->F + f) * oh + oy) * ow + ox] =
                        oracle_round_to_float(t, e + eF[f] + e0);
                }
            }
    free(Wq); free(eF); free(q); free(v);
}

/* Weight gradient (repro_conv_cpu.h:40-70, repro_conv_math.cuh:101-130): dY quantised per
 * filter, x per window position over all windows, dW[f][k] = round(sum_w D * X,
 * e_filter + e_position + e0). */
void oracle_conv2d_grad_weight(const float* dy, const float* x, float* dw,
                               const oracle_conv_shape* g, int S) {
    int K = g->C * g->KH * g->KW, oh = conv_oh(g), ow = conv_ow(g), e0 = -14 * (S - 1);
    size_t P = (size_t)oh * ow, outn = (size_t)g->N * g->F * P;
    int* eF = (int*)malloc(sizeof(int) * (size_t)g->F);
    int* D = (int*)malloc(sizeof(int) * outn);
    int* X = (int*)malloc(sizeof(int) * (size_t)g->N * P);
    int64_t* t = (int64_t*)malloc(sizeof(int64_t) * (size_t)g->F);
    for (int f = 0; f < g->F; ++f) {
        float m = 0.0f;
        for (int n = 0; n < g->N; ++n)
            for (size_t p = 0; p < P; ++p) m = fmaxf(m, fabsf(dy[((size_t)n * g->F + f) * P + p]));
        eF[f] = oracle_scale_exponent(m);
    }
    for (size_t i = 0; i < outn; ++i) D[i] = oracle_fixed_point(dy[i], eF[(i / P) % g->F], S);
    for (int k = 0; k < K; ++k) {
        int c = k / (g->KH * g->KW), r = k % (g->KH * g->KW), ky = r / g->KW, kx = r % g->KW;
        uint32_t mb = 0;
        for (int n = 0; n < g->N; ++n)
            for (size_t p = 0; p < P; ++p)
                mb = conv_bits_max(mb, conv_window_value(x, g, n, (int)(p / ow), (int)(p % ow), c, ky, kx));
        int eX = oracle_scale_exponent(u2f(mb));
        for (int n = 0; n < g->N; ++n)
            for (size_t p = 0; p < P; ++p)
                X[(size_t)n * P + p] = oracle_fixed_point(
                    conv_window_value(x, g, n, (int)(p / ow), (int)(p % ow), c, ky, kx), eX, S);
        for (int f = 0; f < g->F; ++f) t[f] = 0;
        for (int n = 0; n < g->N; ++n)
            for (int f = 0; f < g->F; ++f) {
                const int* d = D + ((size_t)n * g->F + f) * P;
                const int* xv = X + (size_t)n * P;
                int64_t s = 0;
                for (size_t p = 0; p < P; ++p) s += (int64_t)d[p] * xv[p];
                t[f] += s;
            }
        for (int f = 0; f < g->F; ++f) dw[(size_t)f * K + k] = oracle_round_to_float(t[f], eF[f] + eX + e0);
    }
    free(eF); free(D); free(X); free(t);
}

/* Input gradient (repro_conv_cpu.h:72-91, repro_conv_math.cuh:132-157): dY quantised with one
 * scale per image, all weights with one scale; dX[n][c][y][x] = round(sum over the windows
 * covering the pixel and all filters of D * Wq, e_image + e_weights + e0). */
void oracle_conv2d_grad_input(const float* dy, const float* w, float* dx, const oracle_conv_shape* g,
                              int S) {
    int oh = conv_oh(g), ow = conv_ow(g), e0 = -14 * (S - 1);
    size_t per = (size_t)g->F * oh * ow, wn = (size_t)g->F * g->C * g->KH * g->KW;
    int* eI = (int*)malloc(sizeof(int) * (size_t)g->N);
    int* D = (int*)malloc(sizeof(int) * (size_t)g->N * per);
    int* Wq = (int*)malloc(sizeof(int) * wn);
    for (int n = 0; n < g->N; ++n) {
        float m = 0.0f;
        for (size_t i = 0; i < per; ++i) m = fmaxf(m, fabsf(dy[(size_t)n * per + i]));
        eI[n] = oracle_scale_exponent(m);
        for (size_t i = 0; i < per; ++i) D[(size_t)n * per + i] = oracle_fixed_point(dy[(size_t)n * per + i], eI[n], S);
    }
    float mw = 0.0f;
    for (size_t i = 0; i < wn; ++i) mw = fmaxf(mw, fabsf(w[i]));
    int eW = oracle_scale_exponent(mw);
    for (size_t i = 0; i < wn; ++i) Wq[i] = oracle_fixed_point(w[i], eW, S);
    for (int n = 0; n < g->N; ++n)
        for (int c = 0; c < g->C; ++c)
            for (int y = 0; y < g->H; ++y)
                for (int xx = 0; xx < g->W; ++xx) {
                    int64_t t = 0;
                    for (int ky = 0; ky < g->KH; ++ky) {
                        int ry = y + g->PY - ky;
                        if (ry < 0 || ry % g->SY) continue;
                        int oy = ry / g->SY;
                        if (oy >= oh) continue;
                        for (int kx = 0; kx < g->KW; ++kx) {
                            int rx = xx + g->PX - kx;
                            if (rx < 0 || rx % g->SX) continue;
                            int ox = rx / g->SX;
                            if (ox >= ow) continue;
                            for (int f = 0; f < g->F; ++f)
                                t += (int64_t)D[(((size_t)n * g->F + f) * oh + oy) * ow + ox] *
                                     Wq[(((size_t)f * g->C + c) * g->KH + ky) * g->KW + kx];
                        }
                    }
                    dx[(((size_t)n * g->C + c) * g->H + y) * g->W + xx] =
                        oracle_round_to_float(t, eI[n] + eW + e0);
                }
    free(eI); free(D); free(Wq);
}
