/*
 * kt_oracle_layers.c -- TEST INFRASTRUCTURE ONLY. CPU restatements of the layers that benchmark configs 3-5 build
 * around the 12-bit GEMM, used as the checker of the GPU path and as the timed CPU figure of those configs. Never
 * part of the product; only tests/, __graft_entry__.smoke() and bench.py's CPU legs load it (through oracle.py).
 *
 * The reference runs these layers in its 12-trit domain with per-tensor dynamic requant; the benchmark configs ask
 * for int8 activations, 12-bit weight codes and per-channel integer requant instead. The structure each function
 * follows is the reference's (file:line given per function); the int8 epilogues are this build's definitions,
 * written out in full in each function's comment so the GPU path and this file implement one stated rule.
 *
 * Integer arithmetic only. The lookup tables (SiLU, sigmoid, GELU codes) are inputs: they are built once from
 * closed forms by the workload generator and handed to the GPU path and to this file alike.
 *
 * Pinning (tests/test_oracle.py, tests/test_layers.py):
 *   - dot16 / the blocked GEMM: equal to kt_linear_cpu (the reference's linear_cpu restatement) on random shapes;
 *   - route: brute-force Python sort with the reference's tie rule (layers.rs:800-805);
 *   - bucket + experts + combine (expert-major, what the GPU computes): equal to kt_moe_forward_token, the
 *     reference's per-token loop order (layers.rs:928-936, 988-1020) evaluated token by token with rows = 1;
 *   - the requant epilogues: kt_requant_sat, pinned in kt_oracle.c.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kt_oracle.h"

static inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* clamp(requant(acc, mant, shift), -127, 127): the int8 epilogue of every GEMM below (kt-int/src/lib.rs:78-86 per
 * output channel, saturating instead of wrapping). */
static inline int8_t rq8(int64_t acc, int64_t mant, int32_t shift) {
    return (int8_t)clamp64(kt_requant_sat(acc, mant, shift), -127, 127);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Generators (integer-only, on the reference LCG of apps/kt-demo/src/main.rs:19-22)                              */
/* ------------------------------------------------------------------------------------------------------------ */

/* kt_gen_w12's stream (uniform codes in [-2048, 2047]) written as int16. */
void kt_gen_w12_i16(uint64_t seed, size_t n, int16_t* out) {
    uint64_t s = seed ^ 0x9E3779B97F4A7C15ULL;
    for (size_t i = 0; i < n; i++) out[i] = (int16_t)((int32_t)((kt_lcg_next(&s) >> 33) % 4096) - 2048);
}

/* round(N(0, sigma)) without a clip, on kt_gen_act_gauss's stream (the same Irwin-Hall sum of 12 uniforms):
 * t = 2 * sum - 12 * 65535, v = sign(t) * ((|t| * sigma + 2^16) >> 17). Router logits of config 4. */
void kt_gen_gauss_i32(uint64_t seed, int64_t sigma, size_t n, int32_t* out) {
    uint64_t s = seed ^ 0xD1B54A32D192ED03ULL;
    for (size_t i = 0; i < n; i++) {
        int64_t sum = 0;
        for (int j = 0; j < 12; j++) sum += (int64_t)((kt_lcg_next(&s) >> 33) & 0xFFFF);
        int64_t t = 2 * sum - 12 * 65535;
        int64_t mag = ((t < 0 ? -t : t) * sigma + 65536) >> 17;
        out[i] = (int32_t)(t < 0 ? -mag : mag);
    }
}

/* kt_channel_scales over int16 codes: scale_n = to_i32(from_ratio(127, 4 * sigma * isqrt(sum_k w[n,k]^2))). */
void kt_channel_scales_i16(const int16_t* w, size_t n, size_t k, int64_t sigma, int32_t* mant, int32_t* shift) {
    for (size_t o = 0; o < n; o++) {
        uint64_t ss = 0;
        for (size_t c = 0; c < k; c++) ss += (uint64_t)((int64_t)w[o * k + c] * w[o * k + c]);
        uint64_t root = kt_isqrt_u128(0, ss);
        if (root == 0) {
            mant[o] = 0;
            shift[o] = 0;
            continue;
        }
        kt_scale s = kt_scale_to_i32(kt_scale_from_ratio(0, 127, 0, 4 * (uint64_t)sigma * root));
        mant[o] = (int32_t)s.mant;
        shift[o] = s.shift;
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* The int8 x int16 dot and a task pool                                                                           */
/* ------------------------------------------------------------------------------------------------------------ */

/* sum_i a[i] * b[i] exactly: |a| <= 128, |b| <= 2048 and n <= 8128 keep every partial sum inside int32 (callers
 * check n). The avx512bw copy is the same loop under a target attribute, chosen once by CPUID. */
static inline __attribute__((always_inline)) int32_t dot16_loop(const int16_t* a, const int16_t* b, size_t n) {
    int32_t s = 0;
    for (size_t i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}
static int32_t dot16_portable(const int16_t* a, const int16_t* b, size_t n) { return dot16_loop(a, b, n); }
__attribute__((target("avx2"))) static int32_t dot16_avx2(const int16_t* a, const int16_t* b, size_t n) {
    return dot16_loop(a, b, n);
}
__attribute__((target("avx512f,avx512bw"))) static int32_t dot16_avx512(const int16_t* a, const int16_t* b,
                                                                         size_t n) {
    return dot16_loop(a, b, n);
}
typedef int32_t (*dot16_fn)(const int16_t*, const int16_t*, size_t);
static dot16_fn dot16_pick(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512bw")) return dot16_avx512;
    if (__builtin_cpu_supports("avx2")) return dot16_avx2;
    return dot16_portable;
}

#define KT_DOT16_MAX_K 8128

typedef struct {
    void (*fn)(void* ctx, size_t task);
    void* ctx;
    size_t ntasks;
    size_t next; /* atomic */
} pool_t;

static void* pool_worker(void* p) {
    pool_t* pl = (pool_t*)p;
    for (;;) {
        size_t t = __atomic_fetch_add(&pl->next, 1, __ATOMIC_RELAXED);
        if (t >= pl->ntasks) return NULL;
        pl->fn(pl->ctx, t);
    }
}

/* Run fn(ctx, 0 .. ntasks-1) on up to `threads` threads (0 = the TRITIFY_THREADS cap, kt_resolve_threads). */
static void pool_run(void (*fn)(void*, size_t), void* ctx, size_t ntasks, size_t threads) {
    if (ntasks == 0) return;
    size_t t = threads ? threads : kt_resolve_threads(ntasks);
    if (t > ntasks) t = ntasks;
    pool_t pl = {fn, ctx, ntasks, 0};
    pthread_t* th = (pthread_t*)calloc(t, sizeof(pthread_t));
    for (size_t i = 1; i < t; i++) pthread_create(&th[i], NULL, pool_worker, &pl);
    pool_worker(&pl);
    for (size_t i = 1; i < t; i++) pthread_join(th[i], NULL);
    free(th);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* A plain exact GEMM with the int8 per-channel epilogue (the checker of every dense W12 product in configs 3-5)  */
/* ------------------------------------------------------------------------------------------------------------ */

typedef struct {
    const int8_t* x;
    const int16_t* w;
    size_t m, n, k;
    const int32_t *mant, *shift;
    int64_t* acc;
    int8_t* y8;
    int32_t* y32;
    int add32;
    dot16_fn dot;
    size_t ncb; /* column blocks per row block */
} gemm_ctx;

#define GEMM_ROWS 32
#define GEMM_COLS 256

static inline int32_t sat32(int64_t v) { return (int32_t)clamp64(v, INT32_MIN, INT32_MAX); }

static void gemm_task(void* p, size_t task) {
    gemm_ctx* c = (gemm_ctx*)p;
    size_t rb = task / c->ncb, cb = task % c->ncb;
    size_t r0 = rb * GEMM_ROWS, r1 = r0 + GEMM_ROWS < c->m ? r0 + GEMM_ROWS : c->m;
    size_t o0 = cb * GEMM_COLS, o1 = o0 + GEMM_COLS < c->n ? o0 + GEMM_COLS : c->n;
    int16_t* a = (int16_t*)malloc((r1 - r0) * c->k * sizeof(int16_t) + 1);
    for (size_t r = r0; r < r1; r++)
        for (size_t i = 0; i < c->k; i++) a[(r - r0) * c->k + i] = c->x[r * c->k + i];
    for (size_t o = o0; o < o1; o++)
        for (size_t r = r0; r < r1; r++) {
            int64_t v = c->dot(a + (r - r0) * c->k, c->w + o * c->k, c->k);
            if (c->acc) c->acc[r * c->n + o] = v;
            if (c->y8) c->y8[r * c->n + o] = rq8(v, c->mant[o], c->shift[o]);
            if (c->y32) {
                int64_t q = kt_requant_sat(v, c->mant[o], c->shift[o]);
                c->y32[r * c->n + o] = c->add32 ? sat32((int64_t)c->y32[r * c->n + o] + sat32(q)) : sat32(q);
            }
        }
    free(a);
}

static int gemm_run(const int8_t* x, const int16_t* w, size_t m, size_t n, size_t k, const int32_t* mant,
                    const int32_t* shift, int64_t* acc, int8_t* y8, int32_t* y32, int add32, size_t threads) {
    if (k > KT_DOT16_MAX_K) return -1;
    size_t ncb = (n + GEMM_COLS - 1) / GEMM_COLS;
    gemm_ctx c = {x, w, m, n, k, mant, shift, acc, y8, y32, add32, dot16_pick(), ncb};
    pool_run(gemm_task, &c, (m + GEMM_ROWS - 1) / GEMM_ROWS * ncb, threads);
    return 0;
}

/* acc (m x n i64, optional) = x (m x k int8) . w^T (n x k int16 codes), and y8 (optional) = rq8(acc, mant[o],
 * shift[o]). Returns -1 when k exceeds the int32-exact bound. */
int kt_gemm_i8w16(const int8_t* x, const int16_t* w, size_t m, size_t n, size_t k, const int32_t* mant,
                  const int32_t* shift, int64_t* acc, int8_t* y8, size_t threads) {
    return gemm_run(x, w, m, n, k, mant, shift, acc, y8, NULL, 0, threads);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Config 4: one MoE layer (GLM-4.5-Air shape), this build's int8 definition of the reference's MoeMlp            */
/* ------------------------------------------------------------------------------------------------------------ */
/*
 * Shapes: T tokens of H int8 activations; E routed experts, top_k of them per token, plus one shared expert,
 * numbered E ("group" g in 0..E); expert g has a gate/up matrix WGU[g] (2F x H codes: rows 0..F-1 gate,
 * F..2F-1 up) and a down matrix WD[g] (H x F codes), with per-channel scales (gm, gs) over its 2F gate/up rows
 * and (dm, ds) over its H down rows.
 *
 *   route (MoeMlp::topk / route, crates/01-engine/kt-core/src/layers.rs:800-805, 826-851): the top_k experts of
 *     token t by router code r[t, e], descending, ties to the lower index; the weight of a selected expert is
 *     cw = SIG[clamp(round_half_away(r / 16), -127, 127) + 127] (a sigmoid code table, GLM-4.5's score).
 *   expert g on row x (SwiGluMlp::forward_int, layers.rs:609-640, int8 epilogues):
 *     gq[c] = rq8(x . WGU[g][c], gm[c], gs[c]),  uq[c] = rq8(x . WGU[g][F + c], gm[F + c], gs[F + c]),
 *     h[c]  = clamp(requant(SILU[gq[c] + 127] * uq[c], 1, h_shift), -127, 127)             (c < F)
 *     d[o]  = rq8(h . WD[g][o], dm[o], ds[o])                                             (o < H)
 *   combine (MoeMlp::combine, layers.rs:893-923, as a fixed-point weighted sum; the shared expert is added with
 *     weight 2^12, the shared-expert add of layers.rs:757-780):
 *     out[t, o] = clamp(requant(sum_i cw_i d_{e_i}[o] + 4096 d_E[o], 1, out_shift), -127, 127).
 *
 * The GPU computes the experts expert-major ("bucket" order: the rows of group g are its tokens in increasing
 * token order, group E is every token); integer sums do not depend on the order, so this equals the per-token
 * evaluation the reference does, which kt_moe_forward_token restates.
 */

static inline int32_t sig_index(int32_t r) {
    int64_t a = r < 0 ? -(int64_t)r : (int64_t)r, q = (a + 8) >> 4;
    if (q > 127) q = 127;
    return (int32_t)(r < 0 ? -q : q);
}

/* MoeMlp::topk (layers.rs:800-805) over one token's codes, then the sigmoid-table weight of each choice. */
static void route_one(const int32_t* r, size_t E, size_t top_k, const int16_t* sig, int32_t* sel, int32_t* cw) {
    uint8_t* taken = (uint8_t*)calloc(E, 1);
    for (size_t i = 0; i < top_k; i++) {
        size_t best = E;
        for (size_t e = 0; e < E; e++)
            if (!taken[e] && (best == E || r[e] > r[best])) best = e; /* strict: ties keep the lower index */
        taken[best] = 1;
        sel[i] = (int32_t)best;
        cw[i] = sig[sig_index(r[best]) + 127];
    }
    free(taken);
}

void kt_moe_route(const int32_t* logits, size_t T, size_t E, size_t top_k, const int16_t* sig, int32_t* sel,
                  int32_t* cw) {
    for (size_t t = 0; t < T; t++) route_one(logits + t * E, E, top_k, sig, sel + t * top_k, cw + t * top_k);
}

/* Bucket order: list[g * T + j] = the j-th token (increasing) that chose expert g, pos[t * top_k + i] = the j of
 * (t, its i-th choice), count[g] = group sizes; group E lists every token. */
void kt_moe_bucket(const int32_t* sel, size_t T, size_t E, size_t top_k, int32_t* list, int32_t* pos,
                   int32_t* count) {
    for (size_t g = 0; g <= E; g++) count[g] = 0;
    for (size_t t = 0; t < T; t++) {
        for (size_t i = 0; i < top_k; i++) {
            size_t g = (size_t)sel[t * top_k + i];
            pos[t * top_k + i] = count[g];
            list[g * T + (size_t)count[g]++] = (int32_t)t;
        }
        list[E * T + t] = (int32_t)t;
    }
    count[E] = (int32_t)T;
}

typedef struct {
    const int8_t* x;
    size_t T, H, F, G;
    const int32_t *list, *count;
    const int64_t* off; /* exclusive prefix of count */
    const int16_t *wgu, *wd;
    const int32_t *gm, *gs, *dm, *ds;
    const int16_t* silu;
    int h_shift;
    int8_t *h, *d;
    const size_t* task_g; /* task -> group, first row */
    const size_t* task_r;
    dot16_fn dot;
} moe_ctx;

#define MOE_ROWS 64

/* One expert on rows [r0, r0 + MOE_ROWS) of its group: gate/up, the SwiGLU epilogue, down. */
static void moe_task(void* p, size_t task) {
    moe_ctx* c = (moe_ctx*)p;
    size_t g = c->task_g[task], r0 = c->task_r[task], cnt = (size_t)c->count[g];
    size_t r1 = r0 + MOE_ROWS < cnt ? r0 + MOE_ROWS : cnt, nr = r1 - r0, H = c->H, F = c->F;
    const int16_t* wgu = c->wgu + g * 2 * F * H;
    const int16_t* wd = c->wd + g * H * F;
    const int32_t *gm = c->gm + g * 2 * F, *gs = c->gs + g * 2 * F, *dm = c->dm + g * H, *ds = c->ds + g * H;
    int16_t* a = (int16_t*)malloc(nr * H * sizeof(int16_t) + 1);
    int16_t* hh = (int16_t*)malloc(nr * F * sizeof(int16_t) + 1);
    for (size_t r = 0; r < nr; r++) {
        const int8_t* xr = c->x + (size_t)c->list[g * c->T + r0 + r] * H;
        for (size_t i = 0; i < H; i++) a[r * H + i] = xr[i];
    }
    for (size_t ch = 0; ch < F; ch++)
        for (size_t r = 0; r < nr; r++) {
            int8_t gq = rq8(c->dot(a + r * H, wgu + ch * H, H), gm[ch], gs[ch]);
            int8_t uq = rq8(c->dot(a + r * H, wgu + (F + ch) * H, H), gm[F + ch], gs[F + ch]);
            int64_t hv = (int64_t)c->silu[gq + 127] * uq;
            int8_t h8 = (int8_t)clamp64(kt_requant_sat(hv, 1, c->h_shift), -127, 127);
            hh[r * F + ch] = h8;
            c->h[((size_t)c->off[g] + r0 + r) * F + ch] = h8;
        }
    for (size_t o = 0; o < H; o++)
        for (size_t r = 0; r < nr; r++)
            c->d[((size_t)c->off[g] + r0 + r) * H + o] = rq8(c->dot(hh + r * F, wd + o * F, F), dm[o], ds[o]);
    free(a);
    free(hh);
}

/* Every expert on its bucket (groups 0..E, G = E + 1): h (P x F) and d (P x H) in bucket order, P = sum count. */
int kt_moe_experts(const int8_t* x, size_t T, size_t H, size_t F, size_t G, const int32_t* list,
                   const int32_t* count, const int16_t* wgu, const int16_t* wd, const int32_t* gm, const int32_t* gs,
                   const int32_t* dm, const int32_t* ds, const int16_t* silu, int h_shift, int8_t* h, int8_t* d,
                   size_t threads) {
    if (H > KT_DOT16_MAX_K || F > KT_DOT16_MAX_K) return -1;
    int64_t* off = (int64_t*)malloc(G * sizeof(int64_t));
    size_t ntasks = 0;
    int64_t acc = 0;
    for (size_t g = 0; g < G; g++) {
        off[g] = acc;
        acc += count[g];
        ntasks += ((size_t)count[g] + MOE_ROWS - 1) / MOE_ROWS;
    }
    size_t* tg = (size_t*)malloc((ntasks + 1) * sizeof(size_t));
    size_t* tr = (size_t*)malloc((ntasks + 1) * sizeof(size_t));
    size_t n = 0;
    for (size_t g = 0; g < G; g++)
        for (size_t r = 0; r < (size_t)count[g]; r += MOE_ROWS) tg[n] = g, tr[n] = r, n++;
    moe_ctx c = {x, T, H, F, G, list, count, off, wgu, wd, gm, gs, dm, ds, silu, h_shift, h, d, tg, tr, dot16_pick()};
    pool_run(moe_task, &c, ntasks, threads);
    free(tg);
    free(tr);
    free(off);
    return 0;
}

/* The weighted sum of each token's expert outputs (rows of d in bucket order) and the shared expert's. */
void kt_moe_combine(const int8_t* d, const int32_t* sel, const int32_t* cw, const int32_t* pos, const int32_t* count,
                    size_t T, size_t H, size_t E, size_t top_k, int out_shift, int8_t* out) {
    int64_t* off = (int64_t*)malloc((E + 1) * sizeof(int64_t));
    int64_t acc = 0;
    for (size_t g = 0; g <= E; g++) off[g] = acc, acc += count[g];
    int64_t* y = (int64_t*)malloc(H * sizeof(int64_t));
    for (size_t t = 0; t < T; t++) {
        const int8_t* ds = d + ((size_t)off[E] + t) * H;
        for (size_t o = 0; o < H; o++) y[o] = 4096 * (int64_t)ds[o];
        for (size_t i = 0; i < top_k; i++) {
            size_t g = (size_t)sel[t * top_k + i];
            const int8_t* dr = d + ((size_t)off[g] + (size_t)pos[t * top_k + i]) * H;
            for (size_t o = 0; o < H; o++) y[o] += (int64_t)cw[t * top_k + i] * dr[o];
        }
        for (size_t o = 0; o < H; o++) out[t * H + o] = (int8_t)clamp64(kt_requant_sat(y[o], 1, out_shift), -127, 127);
    }
    free(y);
    free(off);
}

/* The reference's loop order (MoeMlp::forward_routed / forward_one_int, layers.rs:928-936, 988-1020, and the
 * shared-expert add of 757-780): token by token, each selected expert called on that one row, then combined.
 * Straight loops with i64 sums; slow, for small shapes only. */
void kt_moe_forward_token(const int8_t* x, const int32_t* logits, size_t T, size_t H, size_t F, size_t E,
                          size_t top_k, const int16_t* wgu, const int16_t* wd, const int32_t* gm, const int32_t* gs,
                          const int32_t* dm, const int32_t* ds, const int16_t* silu, const int16_t* sig, int h_shift,
                          int out_shift, int8_t* out) {
    int32_t* sel = (int32_t*)malloc((top_k + 1) * sizeof(int32_t));
    int32_t* cw = (int32_t*)malloc((top_k + 1) * sizeof(int32_t));
    int8_t* h = (int8_t*)malloc(F + 1);
    int8_t* dd = (int8_t*)malloc(H + 1);
    int64_t* y = (int64_t*)malloc(H * sizeof(int64_t));
    for (size_t t = 0; t < T; t++) {
        const int8_t* xr = x + t * H;
        route_one(logits + t * E, E, top_k, sig, sel, cw);
        for (size_t o = 0; o < H; o++) y[o] = 0;
        for (size_t i = 0; i <= top_k; i++) {
            size_t g = i < top_k ? (size_t)sel[i] : E; /* the shared expert last */
            int64_t wgt = i < top_k ? cw[i] : 4096;
            const int16_t* wg = wgu + g * 2 * F * H;
            for (size_t ch = 0; ch < F; ch++) {
                int64_t sg = 0, su = 0;
                for (size_t k = 0; k < H; k++) {
                    sg += (int64_t)xr[k] * wg[ch * H + k];
                    su += (int64_t)xr[k] * wg[(F + ch) * H + k];
                }
                int64_t gq = rq8(sg, gm[g * 2 * F + ch], gs[g * 2 * F + ch]);
                int64_t uq = rq8(su, gm[g * 2 * F + F + ch], gs[g * 2 * F + F + ch]);
                h[ch] = (int8_t)clamp64(kt_requant_sat(silu[gq + 127] * uq, 1, h_shift), -127, 127);
            }
            const int16_t* wdg = wd + g * H * F;
            for (size_t o = 0; o < H; o++) {
                int64_t s = 0;
                for (size_t c = 0; c < F; c++) s += (int64_t)h[c] * wdg[o * F + c];
                dd[o] = rq8(s, dm[g * H + o], ds[g * H + o]);
            }
            for (size_t o = 0; o < H; o++) y[o] += wgt * dd[o];
        }
        for (size_t o = 0; o < H; o++) out[t * H + o] = (int8_t)clamp64(kt_requant_sat(y[o], 1, out_shift), -127, 127);
    }
    free(sel);
    free(cw);
    free(h);
    free(dd);
    free(y);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Config 5: SAM 2.1 Hiera-B+ image-encoder GEMMs (this build's int8 definition)                                   */
/* ------------------------------------------------------------------------------------------------------------ */
/*
 * Entry (IntTensor::from_reals of the normalized image, crates/03-models/kt-model-vision/src/plugin.rs:38, with
 * preprocess.rs's ImageNet normalization): pixel p of channel c -> q = lut[c * 256 + p], an int8 code table built
 * once from the closed form round(48 * (p / 255 - mean_c) / std_c).
 * Patch embed (Conv2d::forward_int, crates/01-engine/kt-core/src/conv.rs:68-130): per output channel oc and
 * position (oy, ox), acc = sum over (ic, ky, kx) of q[ic][iy][ix] * w[oc][ic][ky][kx] with iy = oy*stride + ky - pad,
 * ix = ox*stride + kx - pad, taps outside the image skipped; out[oc][oy][ox] = rq8(acc + bias[oc], mant[oc],
 * shift[oc]) (the reference adds the bias in accumulator units, then requantizes).
 */
void kt_sam_entry(const uint8_t* img, size_t C, size_t HW, const int8_t* lut, int8_t* q) {
    for (size_t c = 0; c < C; c++)
        for (size_t i = 0; i < HW; i++) q[c * HW + i] = lut[c * 256 + img[c * HW + i]];
}

typedef struct {
    const int8_t* q;
    size_t ci, h, w, co, kh, kw, stride, pad, oh, ow;
    const int16_t* wt;
    const int32_t *bias, *mant, *shift;
    int8_t* out;
    int64_t* acc_out;
} conv_ctx;

static void conv_task(void* p, size_t oc) {
    conv_ctx* c = (conv_ctx*)p;
    const int16_t* wb = c->wt + oc * c->ci * c->kh * c->kw;
    for (size_t oy = 0; oy < c->oh; oy++)
        for (size_t ox = 0; ox < c->ow; ox++) {
            int64_t acc = 0;
            for (size_t ic = 0; ic < c->ci; ic++)
                for (size_t ky = 0; ky < c->kh; ky++) {
                    size_t iy = oy * c->stride + ky;
                    if (iy < c->pad || iy - c->pad >= c->h) continue;
                    iy -= c->pad;
                    for (size_t kx = 0; kx < c->kw; kx++) {
                        size_t ix = ox * c->stride + kx;
                        if (ix < c->pad || ix - c->pad >= c->w) continue;
                        ix -= c->pad;
                        acc += (int64_t)c->q[(ic * c->h + iy) * c->w + ix] * wb[(ic * c->kh + ky) * c->kw + kx];
                    }
                }
            acc += c->bias ? c->bias[oc] : 0;
            size_t o = (oc * c->oh + oy) * c->ow + ox;
            if (c->acc_out) c->acc_out[o] = acc;
            c->out[o] = rq8(acc, c->mant[oc], c->shift[oc]);
        }
}

/* The patch-embed conv on the int8 entry codes q ([ci][h][w]); out is [co][oh][ow] int8, acc_out (optional) the
 * i64 sums including the bias. Output channels run in parallel (each a disjoint plane, as par_blocks does). */
void kt_conv2d_i8w16(const int8_t* q, size_t ci, size_t h, size_t w, const int16_t* wt, size_t co, size_t kh,
                     size_t kw, size_t stride, size_t pad, const int32_t* bias, const int32_t* mant,
                     const int32_t* shift, int8_t* out, int64_t* acc_out, size_t threads) {
    size_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1;
    conv_ctx c = {q, ci, h, w, co, kh, kw, stride, pad, oh, ow, wt, bias, mant, shift, out, acc_out};
    pool_run(conv_task, &c, co, threads);
}

/* Hiera's stage MLP (FeedForward::forward_int, crates/03-models/kt-model-vision/src/hiera.rs:336-340, with the
 * GELU of nonlin.rs:30-47 as an int8 code table): h = gelu[rq8(x . Wi^T) + 127], y = rq8(h . Wo^T). */
int kt_mlp_gelu(const int8_t* x, size_t m, size_t d, size_t dh, const int16_t* wi, const int32_t* im,
                const int32_t* is, const int8_t* gelu, const int16_t* wo, const int32_t* om, const int32_t* os,
                int8_t* h, int8_t* y, size_t threads) {
    if (kt_gemm_i8w16(x, wi, m, dh, d, im, is, NULL, h, threads)) return -1;
    for (size_t i = 0; i < m * dh; i++) h[i] = gelu[h[i] + 127];
    return kt_gemm_i8w16(h, wo, m, d, dh, om, os, NULL, y, threads);
}

/* n values uniform in [lo, hi]: ((s >> 33) % (hi - lo + 1)) + lo on the stream seed ^ 0x9E3779B97F4A7C15 (the image
 * pixels of config 5 with lo = 0, hi = 255). */
void kt_gen_uniform_i32(uint64_t seed, int64_t lo, int64_t hi, size_t n, int32_t* out) {
    uint64_t s = seed ^ 0x9E3779B97F4A7C15ULL, range = (uint64_t)(hi - lo + 1);
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)((int64_t)((kt_lcg_next(&s) >> 33) % range) + lo);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Config 3: a Qwen2.5-0.5B-shape decoder (this build's int8 definition of the reference's DecoderModel)           */
/* ------------------------------------------------------------------------------------------------------------ */
/*
 * The reference's decoder (DecoderModel::embed_int / blocks_int / head_int / decode_step,
 * crates/01-engine/kt-core/src/model.rs:168-188, 290-353; Attention, attention.rs; SwiGluMlp, layers.rs:609-640;
 * generate_greedy_by, generate.rs:82-111) with int8 activations, W12 weights and per-channel requant:
 *   residual r: int32 per hidden unit; embed: r = emb[token] (the 12-bit codes of the tied embedding row);
 *   rmsnorm(r) -> int8: rms = isqrt(floor(sum r^2 / d)), q = clamp(div_round(32 r, rms), +-127) (0 when rms = 0),
 *     div_round = round half away from zero;
 *   attention block: qkv = rq8(rmsnorm(r) . Wqkv^T) (q: nh heads, then k, v: nkv heads, each hd wide);
 *     rope at position p (rotate-half pairs i, i + hd/2): a' = sr(a C - b S, 14), b' = sr(b C + a S, 14) with the
 *     int16 tables C = cos[p][i], S = sin[p][i] (2^14 scale), sr = round-half-away shift, clamped to +-127;
 *     the rotated k and v are appended to the caches at p; head h (kv head g = h / (nh / nkv)) attends positions
 *     j <= p: s_j = q . k_j, m = max s_j, e_j = EXP[(m - s_j + 64) >> 7] (0 past the 1024-entry table),
 *     o = div_round(sum_j e_j v_j, sum_j e_j); r = sat32(r + sat32(requant(o . Wo^T, o scales)));
 *   mlp block: g, u = rq8(rmsnorm(r) . Wgu^T) (gate rows 0..ffn-1, up ffn..2ffn-1); h = clamp(sr(SILU[g + 127] u,
 *     h_shift)); r = sat32(r + sat32(requant(h . Wd^T, down scales)));
 *   head: logits = sat32(requant(rmsnorm(r) . emb^T, lm scales)) (int32); greedy: the first maximum
 *     (argmax_codes, generate.rs:48-56).
 * Every operation is per row except attention, whose row t sees only positions <= its own: feeding a prompt as one
 * batch or position by position (the reference's generate_greedy_by) gives the same integers.
 */
typedef struct {
    int64_t d, ffn, nh, nkv, hd, layers, vocab, max_pos, h_shift;
    const int16_t* emb;                    /* vocab x d codes; the lm_head is tied */
    const int32_t *lm_mant, *lm_shift;     /* vocab */
    const int16_t* wqkv;                   /* layers x (nh + 2 nkv) hd x d */
    const int32_t *qkv_mant, *qkv_shift;   /* layers x (nh + 2 nkv) hd */
    const int16_t* wo;                     /* layers x d x nh hd */
    const int32_t *o_mant, *o_shift;       /* layers x d */
    const int16_t* wgu;                    /* layers x 2 ffn x d */
    const int32_t *gu_mant, *gu_shift;     /* layers x 2 ffn */
    const int16_t* wd;                     /* layers x d x ffn */
    const int32_t *d_mant, *d_shift;       /* layers x d */
    const int16_t *rope_cos, *rope_sin;    /* max_pos x hd / 2 */
    const int32_t* exp_tab;                /* 1024 */
    const int16_t* silu;                   /* 255 */
} kt_dec_model;

static inline int64_t div_round(int64_t a, int64_t b) { /* b > 0, round half away from zero */
    int64_t q = (2 * (a < 0 ? -a : a) + b) / (2 * b);
    return a < 0 ? -q : q;
}
static inline int64_t shift_round(int64_t v, int s) {
    int64_t q = ((v < 0 ? -v : v) + ((int64_t)1 << (s - 1))) >> s;
    return v < 0 ? -q : q;
}

/* The decoder's RMSNorm to int8 codes (this build's rule): rms = isqrt(floor(sum r^2 / d)),
 * q = clamp(div_round(32 r, rms), +-127), 0 when rms = 0. */
void kt_dec_rmsnorm_rows(const int32_t* r, size_t rows, size_t d, int8_t* q) {
    for (size_t t = 0; t < rows; t++) {
        const int32_t* x = r + t * d;
        unsigned __int128 ss = 0; /* exact: d values of at most 2^62 */
        for (size_t i = 0; i < d; i++) ss += (unsigned __int128)(uint64_t)((int64_t)x[i] * x[i]);
        int64_t rms = (int64_t)kt_isqrt_u128(0, (uint64_t)(ss / d)); /* the mean of squares is at most 2^62 */
        for (size_t i = 0; i < d; i++) q[t * d + i] = rms == 0 ? 0 : (int8_t)clamp64(div_round(32 * (int64_t)x[i], rms), -127, 127);
    }
}

/* Rotate-half RoPE of `heads` heads of hd int8 values in place at position p: pairs (i, i + hd/2) rotated by the
 * int16 tables C = cos[p][i], S = sin[p][i] at 2^14: a' = clamp(sr(a C - b S, 14)), b' = clamp(sr(b C + a S, 14)). */
void kt_dec_rope_row(int8_t* x, size_t heads, size_t hd, size_t p, const int16_t* cos_t, const int16_t* sin_t) {
    const size_t hh = hd / 2;
    for (size_t hv = 0; hv < heads; hv++) {
        int8_t* y = x + hv * hd;
        for (size_t i = 0; i < hh; i++) {
            int64_t a = y[i], b = y[i + hh], C = cos_t[p * hh + i], S = sin_t[p * hh + i];
            y[i] = (int8_t)clamp64(shift_round(a * C - b * S, 14), -127, 127);
            y[i + hh] = (int8_t)clamp64(shift_round(b * C + a * S, 14), -127, 127);
        }
    }
}

/* One head's attention (this build's integer softmax) over positions 0..p of one kv head g of the caches kl / vl
 * ([pos][nkv][hd] int8): s_j = q . k_j, m = max s_j, e_j = exp_tab[(m - s_j + 64) >> 7] (0 past 1024 entries),
 * o = clamp(div_round(sum_j e_j v_j, sum_j e_j)). sc: scratch of p + 1 values. */
void kt_dec_attend(const int8_t* q, const int8_t* kl, const int8_t* vl, size_t p, size_t nkv, size_t g, size_t hd,
                   const int32_t* exp_tab, int64_t* sc, int8_t* o) {
    int64_t m = INT64_MIN;
    for (size_t j = 0; j <= p; j++) {
        const int8_t* k = kl + (j * nkv + g) * hd;
        int64_t s = 0;
        for (size_t i = 0; i < hd; i++) s += (int64_t)q[i] * k[i];
        sc[j] = s;
        if (s > m) m = s;
    }
    int64_t den = 0;
    for (size_t j = 0; j <= p; j++) {
        int64_t idx = (m - sc[j] + 64) >> 7;
        sc[j] = idx < 1024 ? exp_tab[idx] : 0;
        den += sc[j];
    }
    for (size_t i = 0; i < hd; i++) {
        int64_t acc = 0;
        for (size_t j = 0; j <= p; j++) acc += sc[j] * vl[(j * nkv + g) * hd + i];
        o[i] = (int8_t)clamp64(div_round(acc, den), -127, 127);
    }
}

/* kt_dec_forward: rows tokens[0 .. T) at positions pos0 .. pos0 + T - 1 through every layer, appending k and v to the
 * caches (layers x max_pos x nkv x hd int8 each); logits (vocab int32, optional) of the last row. r is scratch of
 * T x d int32. */
void kt_dec_forward(const kt_dec_model* M, const int32_t* tokens, size_t T, size_t pos0, int8_t* kc, int8_t* vc,
                    int32_t* logits, size_t threads) {
    const size_t d = (size_t)M->d, ffn = (size_t)M->ffn, nh = (size_t)M->nh, nkv = (size_t)M->nkv, hd = (size_t)M->hd;
    const size_t nq = (nh + 2 * nkv) * hd, maxp = (size_t)M->max_pos, rep = nh / nkv;
    int32_t* r = (int32_t*)malloc(T * d * sizeof(int32_t));
    int8_t* xn = (int8_t*)malloc(T * (d > ffn ? ffn : d) * 2 + T * ffn);
    int8_t* qkv = (int8_t*)malloc(T * nq);
    int8_t* o = (int8_t*)malloc(T * nh * hd);
    int8_t* gu = (int8_t*)malloc(T * 2 * ffn);
    int8_t* h = (int8_t*)malloc(T * ffn);
    int64_t* sc = (int64_t*)malloc(maxp * sizeof(int64_t));
    for (size_t t = 0; t < T; t++)
        for (size_t i = 0; i < d; i++) r[t * d + i] = M->emb[(size_t)tokens[t] * d + i];
    for (size_t l = 0; l < (size_t)M->layers; l++) {
        int8_t* kl = kc + l * maxp * nkv * hd;
        int8_t* vl = vc + l * maxp * nkv * hd;
        kt_dec_rmsnorm_rows(r, T, d, xn);
        gemm_run(xn, M->wqkv + l * nq * d, T, nq, d, M->qkv_mant + l * nq, M->qkv_shift + l * nq, NULL, qkv, NULL, 0,
                 threads);
        for (size_t t = 0; t < T; t++) {
            size_t p = pos0 + t;
            int8_t* row = qkv + t * nq;
            kt_dec_rope_row(row, nh + nkv, hd, p, M->rope_cos, M->rope_sin); /* q heads then k heads */
            memcpy(kl + p * nkv * hd, row + nh * hd, nkv * hd);
            memcpy(vl + p * nkv * hd, row + (nh + nkv) * hd, nkv * hd);
        }
        for (size_t t = 0; t < T; t++)
            for (size_t hq = 0; hq < nh; hq++)
                kt_dec_attend(qkv + t * nq + hq * hd, kl, vl, pos0 + t, nkv, hq / rep, hd, M->exp_tab, sc,
                              o + t * nh * hd + hq * hd);
        gemm_run(o, M->wo + l * d * nh * hd, T, d, nh * hd, M->o_mant + l * d, M->o_shift + l * d, NULL, NULL, r, 1,
                 threads);
        kt_dec_rmsnorm_rows(r, T, d, xn);
        gemm_run(xn, M->wgu + l * 2 * ffn * d, T, 2 * ffn, d, M->gu_mant + l * 2 * ffn, M->gu_shift + l * 2 * ffn,
                 NULL, gu, NULL, 0, threads);
        for (size_t t = 0; t < T; t++)
            for (size_t c = 0; c < ffn; c++) {
                int64_t g = gu[t * 2 * ffn + c], u = gu[t * 2 * ffn + ffn + c];
                h[t * ffn + c] = (int8_t)clamp64(shift_round(M->silu[g + 127] * u, (int)M->h_shift), -127, 127);
            }
        gemm_run(h, M->wd + l * d * ffn, T, d, ffn, M->d_mant + l * d, M->d_shift + l * d, NULL, NULL, r, 1, threads);
    }
    if (logits) {
        kt_dec_rmsnorm_rows(r + (T - 1) * d, 1, d, xn);
        gemm_run(xn, M->emb, 1, (size_t)M->vocab, d, M->lm_mant, M->lm_shift, NULL, NULL, logits, 0, threads);
    }
    free(r);
    free(xn);
    free(qkv);
    free(o);
    free(gu);
    free(h);
    free(sc);
}

/* argmax_codes (generate.rs:48-56): the first index of the maximum. */
int64_t kt_argmax_i32(const int32_t* v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (int64_t)best;
}

/* generate_greedy_by (generate.rs:82-111) with no stop tokens: the prompt (P tokens) as one batch when `batched`,
 * else position by position as the reference feeds it; then max_new tokens, hashing (here: returning) the logits of
 * every step before its argmax. tokens_out: max_new ids; logits_out: max_new x vocab int32. The caches must hold
 * P + max_new - 1 positions (max_pos). */
int kt_dec_generate(const kt_dec_model* M, const int32_t* prompt, size_t P, size_t max_new, int batched,
                    int32_t* tokens_out, int32_t* logits_out, size_t threads) {
    if (P == 0 || P + max_new - 1 > (size_t)M->max_pos || M->d > KT_DOT16_MAX_K || M->ffn > KT_DOT16_MAX_K) return -1;
    size_t cache = (size_t)M->layers * (size_t)M->max_pos * (size_t)M->nkv * (size_t)M->hd;
    int8_t* kc = (int8_t*)calloc(cache, 1);
    int8_t* vc = (int8_t*)calloc(cache, 1);
    size_t V = (size_t)M->vocab;
    if (batched) {
        kt_dec_forward(M, prompt, P, 0, kc, vc, logits_out, threads);
    } else {
        for (size_t p = 0; p < P; p++) kt_dec_forward(M, prompt + p, 1, p, kc, vc, p + 1 == P ? logits_out : NULL, threads);
    }
    size_t pos = P;
    for (size_t n = 0; n < max_new; n++) {
        int32_t next = (int32_t)kt_argmax_i32(logits_out + n * V, V);
        tokens_out[n] = next;
        if (n + 1 < max_new) {
            kt_dec_forward(M, &next, 1, pos, kc, vc, logits_out + (n + 1) * V, threads);
            pos++;
        }
    }
    free(kc);
    free(vc);
    return 0;
}

/* Per-output-channel 12-bit codes of a Gaussian matrix (config 3's "N(0, 0.02) quantized to 12-bit codes per output
 * channel", in integers): v = round(N(0, 2^20)) on kt_gen_gauss_i32's stream, then per row
 * code = div_round(2047 v, max_row |v|) (a zero row stays zero). */
void kt_gen_quant_rows(uint64_t seed, size_t rows, size_t cols, int16_t* out) {
    int32_t* v = (int32_t*)malloc(cols * sizeof(int32_t));
    uint64_t s = seed ^ 0xD1B54A32D192ED03ULL;
    for (size_t r = 0; r < rows; r++) {
        int64_t mx = 0;
        for (size_t c = 0; c < cols; c++) {
            int64_t sum = 0;
            for (int j = 0; j < 12; j++) sum += (int64_t)((kt_lcg_next(&s) >> 33) & 0xFFFF);
            int64_t t = 2 * sum - 12 * 65535;
            int64_t mag = ((t < 0 ? -t : t) * (1 << 20) + 65536) >> 17;
            v[c] = (int32_t)(t < 0 ? -mag : mag);
            if (mag > mx) mx = mag;
        }
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = mx == 0 ? 0 : (int16_t)div_round(2047 * (int64_t)v[c], mx);
    }
    free(v);
}

/* kt_channel_scales_i16 with the accumulator's 4 sigma mapped to `target` instead of 127. */
void kt_channel_scales_target_i16(const int16_t* w, size_t n, size_t k, int64_t sigma, int64_t target, int32_t* mant,
                                  int32_t* shift) {
    for (size_t o = 0; o < n; o++) {
        uint64_t ss = 0;
        for (size_t c = 0; c < k; c++) ss += (uint64_t)((int64_t)w[o * k + c] * w[o * k + c]);
        uint64_t root = kt_isqrt_u128(0, ss);
        if (root == 0) {
            mant[o] = 0;
            shift[o] = 0;
            continue;
        }
        kt_scale s = kt_scale_to_i32(kt_scale_from_ratio(0, (uint64_t)target, 0, 4 * (uint64_t)sigma * root));
        mant[o] = (int32_t)s.mant;
        shift[o] = s.shift;
    }
}
