/*
 * kt_oracle_refdec.c -- TEST INFRASTRUCTURE ONLY (the CPU oracle; never part of the product). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * A C restatement of the reference's integer decoder engine, at the reference's own semantics: 12-trit weight codes
 * (|w| <= WLEVELS) with per-tensor Scales, activations as i32 codes at the 2^28 level quantized dynamically per
 * tensor, every op composed with kt-int's integer Scale arithmetic (restated in kt_oracle.c). Paths are relative to
 * the tritify repository root.
 *
 *   model build (offline, f64): QuantLinear::from_weights, RmsNorm::new, Embedding::from_weights
 *     (crates/01-engine/kt-core/src/layers.rs:212-232, 380-390, 1110-1125), Attention::new's RoPE tables, 1/sqrt(hd)
 *     and exp CodeLut (attention.rs:64-140), SwiGluMlp::new's SiLU CodeLut (layers.rs:591-601),
 *     CodeLut::build / index / code_at (crates/00-kernels/kt-int/src/lib.rs:346-396);
 *   run time (integers only): RmsNorm::forward_int (layers.rs:392-434), add (layers.rs:121-136),
 *     QuantLinear::forward_int (kt_oracle.c, layers.rs:275-328), Attention::rope_int (attention.rs:222-246),
 *     Attention::decode_step (attention.rs:340-459), SwiGluMlp::forward_int (layers.rs:609-640),
 *     DecoderModel::decode_step (model.rs:290-294, 338-353), generate_greedy_by / argmax_codes / hash_step
 *     (generate.rs:48-111) and repro::run's per-position logits_hash (crates/04-ingest/kt-convert/src/repro.rs:
 *     34-42, 60-84);
 *   the seeded model of repro::synthetic_model (repro.rs:260-300).
 *
 * Pinning: verify_repro --synthetic (seed 7, prompt [3,14,15,9,26,5,35,8,9,7,9,3], 32 greedy tokens) prints
 * logits_hash 8109ebad0a2883838a9d133351ce421f676e8d66dbcaffc5cde000272b748d03 (REPRODUCE.md:17); the same run here
 * must give it (tests/test_refdec.py), which pins every function below through the whole decoder. The offline tables
 * call the C library's exp / pow / cos / sin, as the reference's f64 methods call the platform libm.
 *
 * Built with -ffp-contract=off: no float expression is contracted into a fused multiply-add.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kt_oracle.h"

typedef __int128 i128;
typedef unsigned __int128 u128;

#define WLEVELS 265720LL
#define ACT_LEVELS (1LL << 28)

/* kt-int restated in kt_oracle.c */
kt_scale kt_scale_from_f64(double x);
int kt_scale_ge(kt_scale a, kt_scale o);
kt_scale kt_scale_mul(kt_scale a, kt_scale o);
int64_t kt_scale_apply(kt_scale a, int64_t value);
kt_scale kt_scale_recip(kt_scale a);
kt_scale kt_scale_add(kt_scale a, kt_scale o);
kt_scale kt_scale_rsqrt(kt_scale a);
int32_t kt_requant_dyn(int64_t v, int64_t num_level, int64_t den);
void kt_quant_linear_forward(const int32_t* x, size_t rows, size_t in, kt_scale xs, const int32_t* w, size_t out,
                             kt_scale ws, const int64_t* bias, kt_scale bs, size_t threads, int32_t* y, kt_scale* os,
                             int64_t* xmax_out, int64_t* ymax_out);
size_t kt_sha256_ctx_size(void);
void kt_sha256_init(void* c);
void kt_sha256_update(void* c, const void* data, size_t n);
void kt_sha256_final(void* c, uint8_t out[32]);

static const kt_scale ZERO = {0, 0};

static kt_scale ratio(u128 num, u128 den) {
    return kt_scale_from_ratio((uint64_t)(num >> 64), (uint64_t)num, (uint64_t)(den >> 64), (uint64_t)den);
}
/* The engine's "largest scale" fold, |a, b| if b.ge(a) { b } else { a } from Scale::ZERO: of equal values the last
 * one wins. */
static kt_scale fold_max(kt_scale a, kt_scale b) { return kt_scale_ge(b, a) ? b : a; }
static int64_t abs_w(int64_t v) { return v < 0 ? (int64_t)(0 - (uint64_t)v) : v; } /* i64::abs, release build */
static int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
static int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }

/* ------------------------------------------------------------------------------------------------------------ */
/* CodeLut (kt-int/src/lib.rs:346-396)                                                                          */
/* ------------------------------------------------------------------------------------------------------------ */
typedef struct {
    int64_t* codes;
    size_t n;
    kt_scale inv_step_scale;
    int64_t lo_index;
    kt_scale code_scale;
    int right_identity;
} rd_lut;

enum { LUT_EXP = 0, LUT_SILU = 1 };

static double lut_f(int kind, double x) { return kind == LUT_EXP ? exp(x) : x / (1.0 + exp(-x)); }

static void lut_build_f(rd_lut* L, double (*f)(double), double lo, double hi, unsigned idx_bits, unsigned code_bits,
                        int right_id) {
    const size_t n = (size_t)1 << idx_bits;
    const double k = (double)(1ULL << code_bits);
    L->codes = (int64_t*)malloc(n * sizeof(int64_t));
    for (size_t i = 0; i < n; i++) {
        const double x = lo + (hi - lo) * ((double)i / (double)(n - 1));
        L->codes[i] = (int64_t)round(f(x) * k);
    }
    const double inv_step = (double)(n - 1) / (hi - lo);
    L->inv_step_scale = kt_scale_from_f64(inv_step);
    L->lo_index = (int64_t)round(lo * inv_step);
    L->n = n;
    L->code_scale = kt_scale_from_f64(1.0 / k);
    L->right_identity = right_id;
}

static double f_exp(double x) { return lut_f(LUT_EXP, x); }
static double f_silu(double x) { return lut_f(LUT_SILU, x); }
static void lut_build(rd_lut* L, int kind, double lo, double hi, unsigned idx_bits, unsigned code_bits, int right_id) {
    lut_build_f(L, kind == LUT_EXP ? f_exp : f_silu, lo, hi, idx_bits, code_bits, right_id);
}

/* CodeLut::index: round((data * scale - lo) * inv_step) with the build-time constants. */
static int64_t lut_index(const rd_lut* L, int64_t data, kt_scale scale) {
    return kt_scale_apply(kt_scale_mul(scale, L->inv_step_scale), data) - L->lo_index;
}
static int64_t lut_code_at(const rd_lut* L, int64_t idx) {
    if (idx < 0) idx = 0;
    if (idx > (int64_t)L->n - 1) idx = (int64_t)L->n - 1;
    return L->codes[idx];
}

/* ------------------------------------------------------------------------------------------------------------ */
/* The model                                                                                                    */
/* ------------------------------------------------------------------------------------------------------------ */
typedef struct {
    int32_t* w;
    kt_scale s;
    size_t out, in;
} rd_ql;
typedef struct {
    int32_t* w;
    kt_scale s, eps;
    size_t dim;
} rd_norm;
typedef struct {
    rd_norm in_norm, post_norm;
    rd_ql wq, wk, wv, wo, gate, up, down;
} rd_layer;

typedef struct {
    size_t dim, layers, nh, nkv, hd, hidden, vocab, max_seq;
    double eps, theta;
    int32_t* emb;
    kt_scale emb_scale;
    rd_layer* L;
    rd_norm final_norm;
    rd_ql lm_head;
    kt_scale *cos_mag, *sin_mag; /* max_seq x hd/2 */
    int8_t *cos_sign, *sin_sign;
    kt_scale inv_sqrt;
    rd_lut exp_code, silu;
} kt_refdec;

/* One step's KV cache of one layer (LayerKv, attention.rs:251-265): post-RoPE k codes and v codes, each step with
 * its own Scale. */
typedef struct {
    int32_t *k, *v;
    kt_scale *ks, *vs;
    size_t steps, kstride, cap;
} rd_cache;

/* An IntTensor: codes and one Scale. */
typedef struct {
    int32_t* d;
    size_t n;
    kt_scale s;
} rd_t;

static rd_t t_new(size_t n) {
    rd_t t = {(int32_t*)calloc(n ? n : 1, sizeof(int32_t)), n, {0, 0}};
    return t;
}
static void t_free(rd_t* t) {
    free(t->d);
    t->d = NULL;
}

/* QuantLinear::from_weights / RmsNorm::new / Embedding::from_weights: codes = clamp(round(w / step)), step =
 * peak / WLEVELS, scale = Scale::from_f64(step) (layers.rs:212-232, 380-390, 1110-1125). */
static kt_scale quant_weights(const float* w, size_t n, int32_t* codes) {
    double peak = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double a = fabs((double)w[i]);
        peak = a > peak ? a : peak;
    }
    if (peak == 0.0) {
        memset(codes, 0, n * sizeof(int32_t));
        return ZERO;
    }
    const double step = peak / (double)WLEVELS;
    for (size_t i = 0; i < n; i++) {
        int64_t c = (int64_t)round((double)w[i] / step);
        codes[i] = (int32_t)(c < -WLEVELS ? -WLEVELS : c > WLEVELS ? WLEVELS : c);
    }
    return kt_scale_from_f64(step);
}

static void ql_build(rd_ql* q, const float* w, size_t out, size_t in) {
    q->w = (int32_t*)malloc(out * in * sizeof(int32_t));
    q->s = quant_weights(w, out * in, q->w);
    q->out = out, q->in = in;
}
static void norm_build(rd_norm* nm, const float* w, size_t dim, double eps) {
    nm->w = (int32_t*)malloc(dim * sizeof(int32_t));
    nm->s = quant_weights(w, dim, nm->w);
    nm->eps = kt_scale_from_f64(eps);
    nm->dim = dim;
}

/* Attention::new's tables (attention.rs:64-90, 100-140): per (position p, pair j < hd/2) the angle
 * p * theta^(-2j/hd) as signed Scales of its cosine and sine; 1/sqrt(hd); the exp CodeLut over [-30, 0]. SwiGLU's
 * SiLU CodeLut over [-30, 30] with the identity right tail (layers.rs:599). */
static void tables_build(kt_refdec* M) {
    const size_t half = M->hd / 2, n = M->max_seq * half;
    M->cos_mag = (kt_scale*)malloc(n * sizeof(kt_scale));
    M->sin_mag = (kt_scale*)malloc(n * sizeof(kt_scale));
    M->cos_sign = (int8_t*)malloc(n);
    M->sin_sign = (int8_t*)malloc(n);
    for (size_t p = 0; p < M->max_seq; p++)
        for (size_t j = 0; j < half; j++) {
            const double inv_freq = pow(M->theta, -(2.0 * (double)j) / (double)M->hd);
            const double ang = (double)p * inv_freq;
            const double c = cos(ang), s = sin(ang);
            const size_t idx = p * half + j;
            M->cos_mag[idx] = kt_scale_from_f64(fabs(c));
            M->cos_sign[idx] = c < 0.0 ? -1 : 1;
            M->sin_mag[idx] = kt_scale_from_f64(fabs(s));
            M->sin_sign[idx] = s < 0.0 ? -1 : 1;
        }
    M->inv_sqrt = kt_scale_from_f64(1.0 / sqrt((double)M->hd));
    lut_build(&M->exp_code, LUT_EXP, -30.0, 0.0, 16, 20, 0);
    lut_build(&M->silu, LUT_SILU, -30.0, 30.0, 16, 20, 1);
}

/* repro::synthetic_model (repro.rs:260-300): weights uniform in [-1, 1) from the LCG, ((s >> 40) / 2^24) * 2 - 1 as
 * f32, drawn per layer in the field order of LayerWeights, then the embedding, the final norm and the lm_head. */
kt_refdec* kt_rd_synthetic(uint64_t seed, size_t dim, size_t layers, size_t nh, size_t nkv, size_t hd, size_t hidden,
                           size_t vocab, double eps, double theta, size_t max_seq) {
    kt_refdec* M = (kt_refdec*)calloc(1, sizeof(kt_refdec));
    M->dim = dim, M->layers = layers, M->nh = nh, M->nkv = nkv, M->hd = hd, M->hidden = hidden, M->vocab = vocab;
    M->eps = eps, M->theta = theta, M->max_seq = max_seq;
    const size_t qd = nh * hd, kvd = nkv * hd;
    size_t big = vocab * dim;
    const size_t cand[4] = {qd * dim, hidden * dim, dim * hidden, kvd * dim};
    for (int i = 0; i < 4; i++) big = cand[i] > big ? cand[i] : big;
    float* buf = (float*)malloc(big * sizeof(float));
    uint64_t s = seed;
#define DRAW(n)                                                                                     \
    for (size_t i_ = 0; i_ < (n); i_++) {                                                           \
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;                                    \
        buf[i_] = (float)((double)(s >> 40) / (double)(1ULL << 24) * 2.0 - 1.0);                    \
    }
    M->L = (rd_layer*)calloc(layers, sizeof(rd_layer));
    for (size_t l = 0; l < layers; l++) {
        rd_layer* L = &M->L[l];
        DRAW(dim);
        norm_build(&L->in_norm, buf, dim, eps);
        DRAW(qd * dim);
        ql_build(&L->wq, buf, qd, dim);
        DRAW(kvd * dim);
        ql_build(&L->wk, buf, kvd, dim);
        DRAW(kvd * dim);
        ql_build(&L->wv, buf, kvd, dim);
        DRAW(dim * qd);
        ql_build(&L->wo, buf, dim, qd);
        DRAW(dim);
        norm_build(&L->post_norm, buf, dim, eps);
        DRAW(hidden * dim);
        ql_build(&L->gate, buf, hidden, dim);
        DRAW(hidden * dim);
        ql_build(&L->up, buf, hidden, dim);
        DRAW(dim * hidden);
        ql_build(&L->down, buf, dim, hidden);
    }
    DRAW(vocab * dim);
    M->emb = (int32_t*)malloc(vocab * dim * sizeof(int32_t));
    M->emb_scale = quant_weights(buf, vocab * dim, M->emb);
    DRAW(dim);
    norm_build(&M->final_norm, buf, dim, eps);
    DRAW(vocab * dim);
    ql_build(&M->lm_head, buf, vocab, dim);
#undef DRAW
    free(buf);
    tables_build(M);
    return M;
}

/* A DecoderModel of the given shape whose codes and Scales the caller sets (kt_rd_set_*), with Attention::new's and
 * SwiGluMlp::new's tables built here: the checker of a device model built from other inputs. */
kt_refdec* kt_rd_new(size_t dim, size_t layers, size_t nh, size_t nkv, size_t hd, size_t hidden, size_t vocab,
                     double eps, double theta, size_t max_seq) {
    kt_refdec* M = (kt_refdec*)calloc(1, sizeof(kt_refdec));
    M->dim = dim, M->layers = layers, M->nh = nh, M->nkv = nkv, M->hd = hd, M->hidden = hidden, M->vocab = vocab;
    M->eps = eps, M->theta = theta, M->max_seq = max_seq;
    M->L = (rd_layer*)calloc(layers, sizeof(rd_layer));
    M->emb = (int32_t*)calloc(vocab * dim, sizeof(int32_t));
    tables_build(M);
    return M;
}

static rd_ql* ql_at(kt_refdec* M, size_t layer, int which) {
    if (which == 7) return &M->lm_head;
    rd_layer* L = &M->L[layer];
    rd_ql* all[7] = {&L->wq, &L->wk, &L->wv, &L->wo, &L->gate, &L->up, &L->down};
    return all[which];
}

/* Codes (out x in) and Scale of wq wk wv wo gate up down (0..6) of a layer, or the lm_head (7). */
void kt_rd_set_ql(kt_refdec* M, size_t layer, int which, const int32_t* codes, size_t out, size_t in, kt_scale s) {
    rd_ql* q = ql_at(M, layer, which);
    free(q->w);
    q->w = (int32_t*)malloc(out * in * sizeof(int32_t));
    memcpy(q->w, codes, out * in * sizeof(int32_t));
    q->out = out, q->in = in, q->s = s;
}

/* Gamma codes and Scale of in_norm (0) / post_norm (1) of a layer, or the final norm (2); eps from the model. */
void kt_rd_set_norm(kt_refdec* M, size_t layer, int which, const int32_t* codes, kt_scale s) {
    rd_norm* nm = which == 2 ? &M->final_norm : which == 0 ? &M->L[layer].in_norm : &M->L[layer].post_norm;
    free(nm->w);
    nm->w = (int32_t*)malloc(M->dim * sizeof(int32_t));
    memcpy(nm->w, codes, M->dim * sizeof(int32_t));
    nm->s = s, nm->eps = kt_scale_from_f64(M->eps), nm->dim = M->dim;
}

void kt_rd_set_emb(kt_refdec* M, const int32_t* codes, kt_scale s) {
    memcpy(M->emb, codes, M->vocab * M->dim * sizeof(int32_t));
    M->emb_scale = s;
}

static void ql_free(rd_ql* q) { free(q->w); }
void kt_rd_free(kt_refdec* M) {
    if (!M) return;
    for (size_t l = 0; l < M->layers; l++) {
        rd_layer* L = &M->L[l];
        free(L->in_norm.w), free(L->post_norm.w);
        ql_free(&L->wq), ql_free(&L->wk), ql_free(&L->wv), ql_free(&L->wo);
        ql_free(&L->gate), ql_free(&L->up), ql_free(&L->down);
    }
    free(M->L);
    free(M->emb);
    free(M->final_norm.w);
    ql_free(&M->lm_head);
    free(M->cos_mag), free(M->sin_mag), free(M->cos_sign), free(M->sin_sign);
    free(M->exp_code.codes), free(M->silu.codes);
    free(M);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* The run-time ops (integers only)                                                                             */
/* ------------------------------------------------------------------------------------------------------------ */

/* requant_dyn of v[0..n) to ACT_LEVELS by its largest magnitude, the engine's closing step of every op: zeros at
 * Scale::ZERO when that is 0, else codes at from_ratio(gmax, ACT_LEVELS) * c. */
static void close_dyn(const int64_t* v, size_t n, kt_scale c, rd_t* y) {
    int64_t gmax = 0;
    for (size_t i = 0; i < n; i++) {
        const int64_t a = abs_w(v[i]);
        gmax = a > gmax ? a : gmax;
    }
    if (gmax == 0) {
        memset(y->d, 0, n * sizeof(int32_t));
        y->s = ZERO;
        return;
    }
    for (size_t i = 0; i < n; i++) y->d[i] = kt_requant_dyn(v[i], ACT_LEVELS, gmax);
    y->s = kt_scale_mul(ratio((u128)gmax, ACT_LEVELS), c);
}

/* RmsNorm::forward_int (layers.rs:392-434) over rows of dim. */
void kt_rd_rmsnorm(const int32_t* x, size_t rows, size_t dim, kt_scale xs, const int32_t* g, kt_scale gs,
                   kt_scale eps, int32_t* y, kt_scale* ys) {
    const size_t n = rows * dim;
    int64_t* p = (int64_t*)malloc(n * sizeof(int64_t) + 8);
    kt_scale* c_rows = (kt_scale*)malloc(rows * sizeof(kt_scale) + 8);
    for (size_t r = 0; r < rows; r++) {
        const int32_t* xr = x + r * dim;
        u128 ss = 0;
        for (size_t i = 0; i < dim; i++) ss += (u128)((i128)xr[i] * (i128)xr[i]);
        const kt_scale mean_sq = kt_scale_mul(kt_scale_mul(ratio(ss, dim), xs), xs);
        const kt_scale denom = kt_scale_add(mean_sq, eps);
        const kt_scale inv = denom.mant == 0 ? ZERO : kt_scale_rsqrt(denom);
        c_rows[r] = kt_scale_mul(kt_scale_mul(xs, inv), gs);
        for (size_t i = 0; i < dim; i++) p[r * dim + i] = (int64_t)xr[i] * (int64_t)g[i];
    }
    kt_scale cc = ZERO;
    for (size_t r = 0; r < rows; r++) cc = fold_max(cc, c_rows[r]);
    rd_t out = {y, n, ZERO};
    if (cc.mant == 0) {
        memset(y, 0, n * sizeof(int32_t));
    } else {
        const kt_scale cinv = kt_scale_recip(cc);
        for (size_t r = 0; r < rows; r++) {
            const kt_scale f = kt_scale_mul(c_rows[r], cinv);
            for (size_t i = 0; i < dim; i++) p[r * dim + i] = kt_scale_apply(f, p[r * dim + i]);
        }
        close_dyn(p, n, cc, &out);
    }
    *ys = out.s;
    free(p), free(c_rows);
}

/* add (layers.rs:121-136): both tensors to the larger scale, summed, requantized dynamically. */
void kt_rd_add(const int32_t* a, kt_scale as, const int32_t* b, kt_scale bs, size_t n, int32_t* y, kt_scale* ys) {
    const kt_scale common = kt_scale_ge(as, bs) ? as : bs;
    rd_t out = {y, n, ZERO};
    if (common.mant == 0) {
        memset(y, 0, n * sizeof(int32_t));
    } else {
        const kt_scale cinv = kt_scale_recip(common), fa = kt_scale_mul(as, cinv), fb = kt_scale_mul(bs, cinv);
        int64_t* sum = (int64_t*)malloc(n * sizeof(int64_t) + 8);
        for (size_t i = 0; i < n; i++) sum[i] = wadd(kt_scale_apply(fa, a[i]), kt_scale_apply(fb, b[i]));
        close_dyn(sum, n, common, &out);
        free(sum);
    }
    *ys = out.s;
}

static void ql(const rd_ql* q, const rd_t* x, rd_t* y) {
    int64_t xm, ym;
    /* threads 0: linear_cpu's own plan_threads workers (backend.rs:89-94); any split gives the same integers */
    kt_quant_linear_forward(x->d, x->n / q->in, q->in, x->s, q->w, q->out, q->s, NULL, ZERO, 0, y->d, &y->s, &xm,
                            &ym);
}

/* The SwiGLU activation between the gate/up and down products (SwiGluMlp::forward_int, layers.rs:615-637):
 * h = silu_code(g) * u with the CodeLut's index, its clamp and its identity right tail, then requant_dyn at
 * code_scale * u.scale. */
void kt_rd_swiglu_act(const void* model, const int32_t* g, kt_scale gs, const int32_t* u, kt_scale us, size_t n,
                      int32_t* h, kt_scale* hs) {
    const rd_lut* L = &((const kt_refdec*)model)->silu;
    const kt_scale id_factor = kt_scale_mul(gs, kt_scale_recip(L->code_scale));
    int64_t* hv = (int64_t*)malloc(n * sizeof(int64_t) + 8);
    for (size_t k = 0; k < n; k++) {
        const int64_t gd = g[k], idx = lut_index(L, gd, gs);
        const int64_t code = idx < 0 ? 0 : idx >= (int64_t)L->n ? kt_scale_apply(id_factor, gd) : lut_code_at(L, idx);
        hv[k] = wmul(code, u[k]);
    }
    rd_t out = {h, n, ZERO};
    close_dyn(hv, n, kt_scale_mul(L->code_scale, us), &out);
    *hs = out.s;
    free(hv);
}

/* Attention::rope_int (attention.rs:222-246): rotate_half pairs (j, j + hd/2) by the signed cos/sin Scales of
 * position p. */
static void rope(const kt_refdec* M, int32_t* v, size_t p) {
    const size_t half = M->hd / 2;
    for (size_t j = 0; j < half; j++) {
        const size_t idx = p * half + j;
        const int64_t cs = M->cos_sign[idx], ss = M->sin_sign[idx];
        const kt_scale cm = M->cos_mag[idx], sm = M->sin_mag[idx];
        const int64_t a = v[j], b = v[j + half];
        v[j] = (int32_t)(cs * kt_scale_apply(cm, a) - ss * kt_scale_apply(sm, b));
        v[j + half] = (int32_t)(cs * kt_scale_apply(cm, b) + ss * kt_scale_apply(sm, a));
    }
}

/* The cache append of Attention::decode_step (attention.rs:366-384): k rotated at pos, k and v and their scales
 * pushed. */
void kt_rd_attention_append(const void* model, void* cache, const int32_t* k, kt_scale ks, const int32_t* v,
                            kt_scale vs, size_t pos) {
    const kt_refdec* M = (const kt_refdec*)model;
    rd_cache* C = (rd_cache*)cache;
    const size_t hd = M->hd, kstride = M->nkv * hd;
    int32_t* kd = C->k + C->steps * kstride;
    memcpy(kd, k, kstride * sizeof(int32_t));
    for (size_t h = 0; h < M->nkv; h++) rope(M, kd + h * hd, pos);
    memcpy(C->v + C->steps * kstride, v, kstride * sizeof(int32_t));
    C->ks[C->steps] = ks;
    C->vs[C->steps] = vs;
    C->steps++;
}

/* The core of Attention::decode_step (attention.rs:358-458) after the q/k/v projections: RoPE at pos, append k and
 * v with their scales, the integer-code softmax per head over every cached step at a common score scale, the
 * heads brought to a common scale and requantized. Returns the concatenated head outputs (the wo input). */
void kt_rd_attention_core(const void* model, void* cache, const int32_t* q, kt_scale qs, const int32_t* k,
                          kt_scale ks, const int32_t* v, kt_scale vs, size_t pos, int32_t* o, kt_scale* os) {
    const kt_refdec* M = (const kt_refdec*)model;
    rd_cache* C = (rd_cache*)cache;
    const size_t hd = M->hd, nh = M->nh, nkv = M->nkv, group = nh / nkv, qstride = nh * hd, kstride = nkv * hd;
    int32_t* qd = (int32_t*)malloc(qstride * sizeof(int32_t));
    memcpy(qd, q, qstride * sizeof(int32_t));
    for (size_t h = 0; h < nh; h++) rope(M, qd + h * hd, pos);
    kt_rd_attention_append(model, cache, k, ks, v, vs, pos);
    const size_t steps = C->steps;

    kt_scale v_ref = ZERO;
    for (size_t j = 0; j < steps; j++) v_ref = fold_max(v_ref, C->vs[j]);
    kt_scale* vf = (kt_scale*)malloc(steps * sizeof(kt_scale));
    if (v_ref.mant == 0) {
        for (size_t j = 0; j < steps; j++) vf[j] = ZERO;
    } else {
        const kt_scale vinv = kt_scale_recip(v_ref);
        for (size_t j = 0; j < steps; j++) vf[j] = kt_scale_mul(C->vs[j], vinv);
    }
    int64_t* head_out = (int64_t*)calloc(qstride, sizeof(int64_t));
    kt_scale* scale_h = (kt_scale*)calloc(nh, sizeof(kt_scale));
    int64_t *dots = (int64_t*)malloc(steps * 8), *score = (int64_t*)malloc(steps * 8), *ec = (int64_t*)malloc(steps * 8);
    kt_scale* sj = (kt_scale*)malloc(steps * sizeof(kt_scale));
    for (size_t h = 0; h < nh; h++) {
        const size_t kv = h / group;
        for (size_t j = 0; j < steps; j++) {
            const int32_t* kr = C->k + j * kstride + kv * hd;
            int64_t dot = 0;
            for (size_t d = 0; d < hd; d++) dot = wadd(dot, wmul(qd[h * hd + d], kr[d]));
            dots[j] = dot;
            sj[j] = kt_scale_mul(kt_scale_mul(qs, C->ks[j]), M->inv_sqrt);
        }
        kt_scale s_ref = ZERO;
        for (size_t j = 0; j < steps; j++) s_ref = fold_max(s_ref, sj[j]);
        if (s_ref.mant == 0) continue;
        const kt_scale sref_inv = kt_scale_recip(s_ref);
        int64_t dmax = INT64_MIN;
        for (size_t j = 0; j < steps; j++) {
            score[j] = kt_scale_apply(kt_scale_mul(sj[j], sref_inv), dots[j]);
            if (score[j] > dmax) dmax = score[j];
        }
        int64_t sumc = 0;
        for (size_t j = 0; j < steps; j++) {
            const int64_t idx = lut_index(&M->exp_code, score[j] - dmax, s_ref);
            ec[j] = idx < 0 ? 0 : lut_code_at(&M->exp_code, idx);
            sumc += ec[j];
        }
        if (sumc <= 0) continue;
        for (size_t d = 0; d < hd; d++) {
            int64_t acc = 0;
            for (size_t j = 0; j < steps; j++)
                acc = wadd(acc, wmul(ec[j], kt_scale_apply(vf[j], C->v[j * kstride + kv * hd + d])));
            head_out[h * hd + d] = acc;
        }
        scale_h[h] = kt_scale_mul(v_ref, ratio(1, (u128)sumc));
    }
    kt_scale common = ZERO;
    for (size_t h = 0; h < nh; h++) common = fold_max(common, scale_h[h]);
    rd_t out = {o, qstride, ZERO};
    if (common.mant == 0) {
        memset(o, 0, qstride * sizeof(int32_t));
    } else {
        const kt_scale cinv = kt_scale_recip(common);
        for (size_t h = 0; h < nh; h++) {
            const kt_scale f = kt_scale_mul(scale_h[h], cinv);
            for (size_t d = 0; d < hd; d++) head_out[h * hd + d] = kt_scale_apply(f, head_out[h * hd + d]);
        }
        close_dyn(head_out, qstride, common, &out);
    }
    *os = out.s;
    free(qd), free(vf), free(head_out), free(scale_h), free(dots), free(score), free(ec), free(sj);
}

void* kt_rd_cache_new(const void* model) {
    const kt_refdec* M = (const kt_refdec*)model;
    rd_cache* C = (rd_cache*)calloc(1, sizeof(rd_cache));
    C->kstride = M->nkv * M->hd;
    C->cap = M->max_seq;
    C->k = (int32_t*)calloc(C->cap * C->kstride, sizeof(int32_t));
    C->v = (int32_t*)calloc(C->cap * C->kstride, sizeof(int32_t));
    C->ks = (kt_scale*)calloc(C->cap, sizeof(kt_scale));
    C->vs = (kt_scale*)calloc(C->cap, sizeof(kt_scale));
    return C;
}
void kt_rd_cache_free(void* cache) {
    rd_cache* C = (rd_cache*)cache;
    if (!C) return;
    free(C->k), free(C->v), free(C->ks), free(C->vs), free(C);
}

/* DecoderModel::decode_step (model.rs:290-294, 338-353) of one token at position pos: embed, every block
 * (input_norm -> attention decode step -> add; post_norm -> SwiGLU -> add), final norm, lm_head. caches: one per
 * layer. logits: vocab codes, *ls their Scale. */
void kt_rd_decode_step(const void* model, void** caches, int64_t token, size_t pos, int32_t* logits, kt_scale* ls) {
    const kt_refdec* M = (const kt_refdec*)model;
    const size_t dim = M->dim, qd = M->nh * M->hd, kvd = M->nkv * M->hd, hid = M->hidden;
    rd_t x = t_new(dim), h = t_new(dim), a = t_new(dim), q = t_new(qd), k = t_new(kvd), v = t_new(kvd);
    rd_t cat = t_new(qd), g = t_new(hid), u = t_new(hid), hh = t_new(hid), m = t_new(dim), x2 = t_new(dim);
    memcpy(x.d, M->emb + (size_t)token * dim, dim * sizeof(int32_t));
    x.s = M->emb_scale;
    for (size_t l = 0; l < M->layers; l++) {
        const rd_layer* L = &M->L[l];
        kt_rd_rmsnorm(x.d, 1, dim, x.s, L->in_norm.w, L->in_norm.s, L->in_norm.eps, h.d, &h.s);
        ql(&L->wq, &h, &q);
        ql(&L->wk, &h, &k);
        ql(&L->wv, &h, &v);
        kt_rd_attention_core(M, caches[l], q.d, q.s, k.d, k.s, v.d, v.s, pos, cat.d, &cat.s);
        ql(&L->wo, &cat, &a);
        kt_rd_add(x.d, x.s, a.d, a.s, dim, x2.d, &x2.s);
        kt_rd_rmsnorm(x2.d, 1, dim, x2.s, L->post_norm.w, L->post_norm.s, L->post_norm.eps, h.d, &h.s);
        ql(&L->gate, &h, &g);
        ql(&L->up, &h, &u);
        kt_rd_swiglu_act(M, g.d, g.s, u.d, u.s, hid, hh.d, &hh.s);
        ql(&L->down, &hh, &m);
        kt_rd_add(x2.d, x2.s, m.d, m.s, dim, x.d, &x.s);
    }
    kt_rd_rmsnorm(x.d, 1, dim, x.s, M->final_norm.w, M->final_norm.s, M->final_norm.eps, h.d, &h.s);
    rd_t lg = {logits, M->vocab, ZERO};
    ql(&M->lm_head, &h, &lg);
    *ls = lg.s;
    rd_t* all[] = {&x, &h, &a, &q, &k, &v, &cat, &g, &u, &hh, &m, &x2};
    for (size_t i = 0; i < sizeof all / sizeof all[0]; i++) t_free(all[i]);
}

/* Attention::forward_int between its projections over a whole sequence (attention.rs:467-598): rows i = 0..T-1 of
 * q (nh heads) and k (nkv heads) rotated at position i; per head and row the causal scores j <= i (exact i64 dots)
 * at the one score scale q.scale * k.scale * inv_sqrt, the exp-CodeLut numerators of (dot - max), their sum and
 * the sum of numerator * v over the rows (v at its one scale); per (row, head) the scale v.scale / sumc; their
 * largest (the engine's fold over the [row][head] order), every output brought to it, then requant_dyn. q: T x
 * nh*hd, k and v: T x nkv*hd codes; o: T x nh*hd. Sums wrap as the reference's release build does. */
void kt_rd_attention_prefill(const void* model, size_t T, const int32_t* q, kt_scale qs, const int32_t* k,
                             kt_scale ks, const int32_t* v, kt_scale vs, int32_t* o, kt_scale* os) {
    const kt_refdec* M = (const kt_refdec*)model;
    const size_t hd = M->hd, nh = M->nh, nkv = M->nkv, group = nh / nkv, qs_ = nh * hd, ks_ = nkv * hd;
    const kt_scale s_score = kt_scale_mul(kt_scale_mul(qs, ks), M->inv_sqrt);
    int32_t* qd = (int32_t*)malloc(T * qs_ * sizeof(int32_t) + 4);
    int32_t* kd = (int32_t*)malloc(T * ks_ * sizeof(int32_t) + 4);
    memcpy(qd, q, T * qs_ * sizeof(int32_t));
    memcpy(kd, k, T * ks_ * sizeof(int32_t));
    for (size_t i = 0; i < T; i++) {
        for (size_t h = 0; h < nh; h++) rope(M, qd + i * qs_ + h * hd, i);
        for (size_t h = 0; h < nkv; h++) rope(M, kd + i * ks_ + h * hd, i);
    }
    int64_t* head_out = (int64_t*)calloc(nh * T * hd + 1, sizeof(int64_t));
    int64_t* head_sum = (int64_t*)calloc(nh * T + 1, sizeof(int64_t));
    int64_t* dots = (int64_t*)malloc((T + 1) * sizeof(int64_t));
    int64_t* ec = (int64_t*)malloc((T + 1) * sizeof(int64_t));
    for (size_t h = 0; h < nh; h++) {
        const size_t kv = h / group;
        for (size_t i = 0; i < T; i++) {
            int64_t dmax = INT64_MIN;
            for (size_t j = 0; j <= i; j++) {
                int64_t dot = 0;
                for (size_t d = 0; d < hd; d++) dot = wadd(dot, wmul(qd[i * qs_ + h * hd + d], kd[j * ks_ + kv * hd + d]));
                dots[j] = dot;
                dmax = dot > dmax ? dot : dmax;
            }
            int64_t sumc = 0;
            for (size_t j = 0; j <= i; j++) {
                const int64_t idx = lut_index(&M->exp_code, wadd(dots[j], 0 - (uint64_t)dmax), s_score);
                ec[j] = idx < 0 ? 0 : lut_code_at(&M->exp_code, idx);
                sumc += ec[j];
            }
            if (sumc > 0) {
                for (size_t d = 0; d < hd; d++) {
                    int64_t acc = 0;
                    for (size_t j = 0; j <= i; j++) acc = wadd(acc, wmul(ec[j], v[j * ks_ + kv * hd + d]));
                    head_out[(h * T + i) * hd + d] = acc;
                }
                head_sum[h * T + i] = sumc;
            }
        }
    }
    kt_scale* sc = (kt_scale*)malloc((T * nh + 1) * sizeof(kt_scale));
    kt_scale common = ZERO;
    for (size_t i = 0; i < T; i++)
        for (size_t h = 0; h < nh; h++) {
            const int64_t sumc = head_sum[h * T + i];
            sc[i * nh + h] = sumc > 0 ? kt_scale_mul(vs, ratio(1, (u128)sumc)) : ZERO;
            common = fold_max(common, sc[i * nh + h]);
        }
    const size_t n = T * qs_;
    if (common.mant == 0) {
        memset(o, 0, n * sizeof(int32_t));
        *os = ZERO;
    } else {
        const kt_scale cinv = kt_scale_recip(common);
        int64_t* vv = (int64_t*)malloc((n + 1) * sizeof(int64_t));
        for (size_t i = 0; i < T; i++)
            for (size_t h = 0; h < nh; h++) {
                const kt_scale f = kt_scale_mul(sc[i * nh + h], cinv);
                for (size_t d = 0; d < hd; d++)
                    vv[i * qs_ + h * hd + d] = kt_scale_apply(f, head_out[(h * T + i) * hd + d]);
            }
        rd_t out = {o, n, ZERO};
        close_dyn(vv, n, common, &out);
        *os = out.s;
        free(vv);
    }
    free(qd), free(kd), free(head_out), free(head_sum), free(dots), free(ec), free(sc);
}

/* CausalLM::forward_int of DecoderModel (model.rs:361-367 = embed_int, blocks_int, head_int; model.rs:168-189):
 * the T tokens' embedding rows as one tensor, per block input_norm -> Attention::forward_int -> add, post_norm ->
 * SwiGluMlp::forward_int -> add, every op over the whole T-row tensor (one dynamic quantization per tensor), then
 * the final norm and the lm_head: logits T x vocab at *ls. T must not exceed max_seq (the reference asserts). */
int kt_rd_forward(const void* model, const int32_t* tokens, size_t T, int32_t* logits, kt_scale* ls) {
    const kt_refdec* M = (const kt_refdec*)model;
    if (T == 0 || T > M->max_seq) return -1;
    for (size_t i = 0; i < T; i++)
        if (tokens[i] < 0 || (size_t)tokens[i] >= M->vocab) return -1;
    const size_t dim = M->dim, qd = M->nh * M->hd, kvd = M->nkv * M->hd, hid = M->hidden;
    rd_t x = t_new(T * dim), h = t_new(T * dim), a = t_new(T * dim), q = t_new(T * qd), k = t_new(T * kvd);
    rd_t v = t_new(T * kvd), cat = t_new(T * qd), g = t_new(T * hid), u = t_new(T * hid), hh = t_new(T * hid);
    rd_t m = t_new(T * dim), x2 = t_new(T * dim);
    for (size_t i = 0; i < T; i++) memcpy(x.d + i * dim, M->emb + (size_t)tokens[i] * dim, dim * sizeof(int32_t));
    x.s = M->emb_scale;
    for (size_t l = 0; l < M->layers; l++) {
        const rd_layer* L = &M->L[l];
        kt_rd_rmsnorm(x.d, T, dim, x.s, L->in_norm.w, L->in_norm.s, L->in_norm.eps, h.d, &h.s);
        ql(&L->wq, &h, &q);
        ql(&L->wk, &h, &k);
        ql(&L->wv, &h, &v);
        kt_rd_attention_prefill(M, T, q.d, q.s, k.d, k.s, v.d, v.s, cat.d, &cat.s);
        ql(&L->wo, &cat, &a);
        kt_rd_add(x.d, x.s, a.d, a.s, T * dim, x2.d, &x2.s);
        kt_rd_rmsnorm(x2.d, T, dim, x2.s, L->post_norm.w, L->post_norm.s, L->post_norm.eps, h.d, &h.s);
        ql(&L->gate, &h, &g);
        ql(&L->up, &h, &u);
        kt_rd_swiglu_act(M, g.d, g.s, u.d, u.s, T * hid, hh.d, &hh.s);
        ql(&L->down, &hh, &m);
        kt_rd_add(x2.d, x2.s, m.d, m.s, T * dim, x.d, &x.s);
    }
    kt_rd_rmsnorm(x.d, T, dim, x.s, M->final_norm.w, M->final_norm.s, M->final_norm.eps, h.d, &h.s);
    rd_t lg = {logits, T * M->vocab, ZERO};
    ql(&M->lm_head, &h, &lg);
    *ls = lg.s;
    rd_t* all[] = {&x, &h, &a, &q, &k, &v, &cat, &g, &u, &hh, &m, &x2};
    for (size_t i = 0; i < sizeof all / sizeof all[0]; i++) t_free(all[i]);
    return 0;
}

/* hash_step (generate.rs:58-64): the scale's mant (i64 LE) and shift (i32 LE), then every code (i32 LE). */
static void hash_step(void* ctx, const int32_t* codes, size_t n, kt_scale s) {
    kt_sha256_update(ctx, &s.mant, 8);
    kt_sha256_update(ctx, &s.shift, 4);
    kt_sha256_update(ctx, codes, n * sizeof(int32_t));
}

/* generate_greedy_by (generate.rs:82-111) with no stop ids, as repro::run drives it (repro.rs:60-84): the prompt
 * position by position, then up to max_new greedy tokens (argmax_codes: the first maximum). tokens_out: max_new
 * ids; run_hash: the Generation's logits_hash (every step that chose a token); pos_hashes (optional):
 * P + max_new - 1 per-position logits_hash values (repro.rs:34-42), 32 bytes each. Returns 0, or -1 when the
 * prompt is empty or the run needs more positions than the tables hold. */
int kt_rd_generate(const void* model, const int32_t* prompt, size_t P, size_t max_new, int32_t* tokens_out,
                   uint8_t run_hash[32], uint8_t* pos_hashes) {
    const kt_refdec* M = (const kt_refdec*)model;
    if (P == 0 || P + (max_new ? max_new - 1 : 0) > M->max_seq) return -1;
    void** caches = (void**)malloc(M->layers * sizeof(void*));
    for (size_t l = 0; l < M->layers; l++) caches[l] = kt_rd_cache_new(M);
    int32_t* logits = (int32_t*)malloc(M->vocab * sizeof(int32_t));
    kt_scale ls = ZERO;
    const size_t ctx_bytes = kt_sha256_ctx_size();
    void* run = malloc(ctx_bytes);
    void* one = malloc(ctx_bytes);
    size_t npos = 0;
#define STEP(tok, p)                                                          \
    do {                                                                      \
        kt_rd_decode_step(M, caches, (tok), (p), logits, &ls);                \
        if (pos_hashes) {                                                     \
            kt_sha256_init(one);                                              \
            hash_step(one, logits, M->vocab, ls);                             \
            kt_sha256_final(one, pos_hashes + 32 * npos);                     \
        }                                                                     \
        npos++;                                                               \
    } while (0)
    for (size_t p = 0; p < P; p++) STEP(prompt[p], p);
    kt_sha256_init(run);
    size_t pos = P, n = 0;
    while (n < max_new) {
        hash_step(run, logits, M->vocab, ls);
        size_t best = 0;
        for (size_t i = 1; i < M->vocab; i++)
            if (logits[i] > logits[best]) best = i;
        tokens_out[n++] = (int32_t)best;
        if (n < max_new) {
            STEP((int64_t)best, pos);
            pos++;
        }
    }
#undef STEP
    kt_sha256_final(run, run_hash);
    for (size_t l = 0; l < M->layers; l++) kt_rd_cache_free(caches[l]);
    free(caches), free(logits), free(run), free(one);
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Accessors: the model's integers, for loading the same model on the device and for the table checks           */
/* ------------------------------------------------------------------------------------------------------------ */

/* which: 0 wq, 1 wk, 2 wv, 3 wo, 4 gate, 5 up, 6 down, 7 lm_head (layer ignored). Copies out x in codes when
 * codes is non-null; returns the scale and the shape. */
kt_scale kt_rd_get_ql(const void* model, size_t layer, int which, int32_t* codes, size_t* out, size_t* in) {
    const kt_refdec* M = (const kt_refdec*)model;
    const rd_ql* q = NULL;
    if (which == 7) {
        q = &M->lm_head;
    } else {
        const rd_layer* L = &M->L[layer];
        const rd_ql* all[7] = {&L->wq, &L->wk, &L->wv, &L->wo, &L->gate, &L->up, &L->down};
        q = all[which];
    }
    if (codes) memcpy(codes, q->w, q->out * q->in * sizeof(int32_t));
    *out = q->out, *in = q->in;
    return q->s;
}
/* which: 0 input_norm, 1 post_norm, 2 final_norm (layer ignored). */
kt_scale kt_rd_get_norm(const void* model, size_t layer, int which, int32_t* codes, kt_scale* eps) {
    const kt_refdec* M = (const kt_refdec*)model;
    const rd_norm* nm = which == 2 ? &M->final_norm : which == 0 ? &M->L[layer].in_norm : &M->L[layer].post_norm;
    if (codes) memcpy(codes, nm->w, nm->dim * sizeof(int32_t));
    *eps = nm->eps;
    return nm->s;
}
kt_scale kt_rd_get_emb(const void* model, int32_t* codes) {
    const kt_refdec* M = (const kt_refdec*)model;
    if (codes) memcpy(codes, M->emb, M->vocab * M->dim * sizeof(int32_t));
    return M->emb_scale;
}
/* The run-time tables: which 0 exp, 1 silu -> codes (2^16 entries), inv_step scale, lo_index, code scale. */
void kt_rd_get_lut(const void* model, int which, int64_t* codes, kt_scale* inv_step, int64_t* lo_index,
                   kt_scale* code_scale) {
    const kt_refdec* M = (const kt_refdec*)model;
    const rd_lut* L = which == 0 ? &M->exp_code : &M->silu;
    if (codes) memcpy(codes, L->codes, L->n * sizeof(int64_t));
    *inv_step = L->inv_step_scale, *lo_index = L->lo_index, *code_scale = L->code_scale;
}
/* RoPE tables: max_seq x hd/2 each of cos/sin magnitudes (mant, shift) and signs; and 1/sqrt(hd). */
kt_scale kt_rd_get_rope(const void* model, int64_t* cos_mant, int32_t* cos_shift, int8_t* cos_sign,
                        int64_t* sin_mant, int32_t* sin_shift, int8_t* sin_sign) {
    const kt_refdec* M = (const kt_refdec*)model;
    const size_t n = M->max_seq * (M->hd / 2);
    for (size_t i = 0; i < n; i++) {
        cos_mant[i] = M->cos_mag[i].mant, cos_shift[i] = M->cos_mag[i].shift, cos_sign[i] = M->cos_sign[i];
        sin_mant[i] = M->sin_mag[i].mant, sin_shift[i] = M->sin_mag[i].shift, sin_sign[i] = M->sin_sign[i];
    }
    return M->inv_sqrt;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* MoeMlp at the reference's semantics (crates/01-engine/kt-core/src/layers.rs:652-1020, router.rs:29-79)        */
/* ------------------------------------------------------------------------------------------------------------ */
typedef struct {
    rd_ql gate, up, down;
} rd_mlp;

typedef struct {
    size_t dim, E, top_k, hidden, shared_hidden;
    int norm_topk, sigmoid, has_shared;
    rd_ql router;
    rd_mlp* experts;
    rd_mlp shared;
    rd_lut exp_code, sig, silu;
    int64_t* bias; /* the sigmoid router's coded selection bias, round(b * 2^20) */
} kt_refmoe;

#define ROUTER_CODE_BITS 20

enum { LUT_SIGMOID = 2 };

static double lut_f2(int kind, double x) { return kind == LUT_SIGMOID ? 1.0 / (1.0 + exp(-x)) : lut_f(kind, x); }

static double f_sigmoid(double x) { return lut_f2(LUT_SIGMOID, x); }
static void lut_build2(rd_lut* L, int kind, double lo, double hi, unsigned idx_bits, unsigned code_bits,
                       int right_id) {
    if (kind != LUT_SIGMOID)
        lut_build(L, kind, lo, hi, idx_bits, code_bits, right_id);
    else
        lut_build_f(L, f_sigmoid, lo, hi, idx_bits, code_bits, right_id);
}

static float unif_f32(uint64_t* s) {
    *s = *s * 6364136223846793005ULL + 1442695040888963407ULL;
    return (float)((double)(*s >> 40) / (double)(1ULL << 24) * 2.0 - 1.0);
}
static void draw(uint64_t* s, float* buf, size_t n) {
    for (size_t i = 0; i < n; i++) buf[i] = unif_f32(s);
}
/* tests_glm.rs:20-29: a SwiGluMlp drawing gate, up (hidden x dim) and down (dim x hidden) from the stream. */
static void mlp_build(rd_mlp* m, uint64_t* s, size_t dim, size_t hidden, float* buf) {
    draw(s, buf, hidden * dim);
    ql_build(&m->gate, buf, hidden, dim);
    draw(s, buf, hidden * dim);
    ql_build(&m->up, buf, hidden, dim);
    draw(s, buf, dim * hidden);
    ql_build(&m->down, buf, dim, hidden);
}

/* The MoE of the reference's GLM tests (tests_glm.rs:31-43, 224-228), generalized: the stream from `seed` draws the
 * router (E x dim) and then each expert's gate / up / down (hidden 24 there); norm_topk_prob as given; with
 * sigmoid != 0 a sigmoid router whose bias is vecf(bias_seed, E) * 0.05 (as f32); with shared_hidden > 0 a shared
 * expert drawn from the stream seed ^ 0xA5. The tables are MoeMlp::new's exp CodeLut, SigmoidScore::new's table
 * (router.rs:38-49) and SwiGluMlp::new's SiLU. */
void* kt_rm_synthetic(uint64_t seed, size_t dim, size_t E, size_t top_k, size_t hidden, int norm_topk, int sigmoid,
                      uint64_t bias_seed, size_t shared_hidden) {
    kt_refmoe* M = (kt_refmoe*)calloc(1, sizeof(kt_refmoe));
    M->dim = dim, M->E = E, M->top_k = top_k, M->hidden = hidden, M->shared_hidden = shared_hidden;
    M->norm_topk = norm_topk, M->sigmoid = sigmoid, M->has_shared = shared_hidden > 0;
    size_t big = E * dim;
    const size_t h2 = hidden > shared_hidden ? hidden : shared_hidden;
    if (h2 * dim > big) big = h2 * dim;
    float* buf = (float*)malloc(big * sizeof(float));
    uint64_t s = seed;
    draw(&s, buf, E * dim);
    ql_build(&M->router, buf, E, dim);
    M->experts = (rd_mlp*)calloc(E, sizeof(rd_mlp));
    for (size_t e = 0; e < E; e++) mlp_build(&M->experts[e], &s, dim, hidden, buf);
    if (M->has_shared) {
        uint64_t s2 = seed ^ 0xA5;
        mlp_build(&M->shared, &s2, dim, shared_hidden, buf);
    }
    M->bias = (int64_t*)calloc(E, sizeof(int64_t));
    if (sigmoid) {
        uint64_t sb = bias_seed;
        const double k = (double)(1ULL << ROUTER_CODE_BITS);
        for (size_t e = 0; e < E; e++) {
            const float b = unif_f32(&sb) * 0.05f;
            M->bias[e] = (int64_t)round((double)b * k);
        }
    }
    lut_build2(&M->exp_code, LUT_EXP, -30.0, 0.0, 16, ROUTER_CODE_BITS, 0);
    lut_build2(&M->sig, LUT_SIGMOID, -16.0, 16.0, 16, ROUTER_CODE_BITS, 0);
    lut_build2(&M->silu, LUT_SILU, -30.0, 30.0, 16, 20, 1);
    free(buf);
    return M;
}

static void mlp_free(rd_mlp* m) { ql_free(&m->gate), ql_free(&m->up), ql_free(&m->down); }
void kt_rm_free(void* p) {
    kt_refmoe* M = (kt_refmoe*)p;
    if (!M) return;
    ql_free(&M->router);
    for (size_t e = 0; e < M->E; e++) mlp_free(&M->experts[e]);
    free(M->experts);
    if (M->has_shared) mlp_free(&M->shared);
    free(M->bias), free(M->exp_code.codes), free(M->sig.codes), free(M->silu.codes);
    free(M);
}

/* SwiGluMlp::forward_int (layers.rs:609-640) on rows x dim codes at xs, with the SiLU table `silu`. */
static void mlp_forward(const rd_mlp* m, const rd_lut* silu, const rd_t* x, rd_t* y) {
    const size_t rows = x->n / m->gate.in, hid = m->gate.out;
    rd_t g = t_new(rows * hid), u = t_new(rows * hid), h = t_new(rows * hid);
    ql(&m->gate, x, &g);
    ql(&m->up, x, &u);
    const kt_scale id_factor = kt_scale_mul(g.s, kt_scale_recip(silu->code_scale));
    int64_t* hv = (int64_t*)malloc(g.n * sizeof(int64_t) + 8);
    for (size_t k = 0; k < g.n; k++) {
        const int64_t gd = g.d[k], idx = lut_index(silu, gd, g.s);
        const int64_t code = idx < 0 ? 0 : idx >= (int64_t)silu->n ? kt_scale_apply(id_factor, gd) : lut_code_at(silu, idx);
        hv[k] = wmul(code, u.d[k]);
    }
    close_dyn(hv, g.n, kt_scale_mul(silu->code_scale, u.s), &h);
    ql(&m->down, &h, y);
    free(hv);
    t_free(&g), t_free(&u), t_free(&h);
}

/* MoeMlp::topk (layers.rs:800-805): the k largest keys, descending, ties to the lower index. */
static void topk_i64(const int64_t* keys, size_t n, size_t k, int32_t* out) {
    char* used = (char*)calloc(n, 1);
    for (size_t i = 0; i < k; i++) {
        size_t best = n;
        for (size_t j = 0; j < n; j++)
            if (!used[j] && (best == n || keys[j] > keys[best])) best = j;
        used[best] = 1;
        out[i] = (int32_t)best;
    }
    free(used);
}

/* MoeMlp::route (layers.rs:826-851) / route_sigmoid (layers.rs:855-870 with router.rs:61-71) for one token row x
 * (dim codes at xs): the router's logits (its QuantLinear), then the softmax numerators exp(l - lmax) from the exp
 * CodeLut and top-k by logit code, or the sigmoid codes and top-k by code + coded bias. sel, ec: top_k each;
 * returns sumc (the top-k codes' sum with norm_topk_prob, else all E codes' sum, or 2^20 for a raw sigmoid). The
 * logits (E codes) and their scale are written when non-null. */
int64_t kt_rm_route(const void* p, const int32_t* x, kt_scale xs, int32_t* sel, int64_t* ec, int32_t* logits_out,
                    kt_scale* ls_out) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    const size_t E = M->E, K = M->top_k;
    rd_t row = {(int32_t*)x, M->dim, xs}, lg = t_new(E);
    ql(&M->router, &row, &lg);
    if (logits_out) memcpy(logits_out, lg.d, E * sizeof(int32_t));
    if (ls_out) *ls_out = lg.s;
    int64_t* codes = (int64_t*)malloc(E * sizeof(int64_t));
    int64_t* keys = (int64_t*)malloc(E * sizeof(int64_t));
    int64_t sumc = 0;
    if (M->sigmoid) {
        for (size_t j = 0; j < E; j++) {
            codes[j] = lut_code_at(&M->sig, lut_index(&M->sig, lg.d[j], lg.s));
            keys[j] = codes[j] + M->bias[j];
        }
        topk_i64(keys, E, K, sel);
        for (size_t i = 0; i < K; i++) ec[i] = codes[sel[i]];
        if (M->norm_topk)
            for (size_t i = 0; i < K; i++) sumc += ec[i];
        else
            sumc = (int64_t)1 << ROUTER_CODE_BITS;
    } else {
        int32_t lmax = INT32_MIN;
        for (size_t j = 0; j < E; j++) lmax = lg.d[j] > lmax ? lg.d[j] : lmax;
        int64_t all = 0;
        for (size_t j = 0; j < E; j++) {
            const int64_t idx = lut_index(&M->exp_code, (int64_t)lg.d[j] - lmax, lg.s);
            codes[j] = idx < 0 ? 0 : lut_code_at(&M->exp_code, idx);
            all += codes[j];
            keys[j] = lg.d[j];
        }
        topk_i64(keys, E, K, sel);
        for (size_t i = 0; i < K; i++) ec[i] = codes[sel[i]];
        if (M->norm_topk)
            for (size_t i = 0; i < K; i++) sumc += ec[i];
        else
            sumc = all;
    }
    free(codes), free(keys);
    t_free(&lg);
    return sumc;
}

/* MoeMlp::combine (layers.rs:893-923): the k expert outputs (out_dim codes each, scales ys) brought to their largest
 * scale, summed with the numerators ec, requantized; the scale folds in 1/sumc. */
void kt_rm_combine(const int32_t* ys, const kt_scale* ys_s, size_t k, size_t out_dim, const int64_t* ec,
                   int64_t sumc, int32_t* out, kt_scale* os) {
    rd_t o = {out, out_dim, ZERO};
    if (sumc <= 0 || k == 0) {
        memset(out, 0, out_dim * sizeof(int32_t));
        *os = ZERO;
        return;
    }
    kt_scale common = ZERO;
    for (size_t i = 0; i < k; i++) common = fold_max(common, ys_s[i]);
    if (common.mant == 0) {
        memset(out, 0, out_dim * sizeof(int32_t));
        *os = ZERO;
        return;
    }
    const kt_scale cinv = kt_scale_recip(common);
    int64_t* acc = (int64_t*)calloc(out_dim, sizeof(int64_t));
    for (size_t i = 0; i < k; i++) {
        const kt_scale f = kt_scale_mul(ys_s[i], cinv);
        for (size_t d = 0; d < out_dim; d++) acc[d] = wadd(acc[d], wmul(ec[i], kt_scale_apply(f, ys[i * out_dim + d])));
    }
    close_dyn(acc, out_dim, common, &o);
    *os = o.s.mant ? kt_scale_mul(o.s, ratio(1, (u128)sumc)) : ZERO;
    free(acc);
}

/* merge_rows (layers.rs:873-891; forward_routed's inline copy, 1000-1015): per-row outputs brought to the largest
 * row scale, requantized together. */
void kt_rm_merge_rows(const int32_t* rows, const kt_scale* rs, size_t T, size_t dim, int32_t* out, kt_scale* os) {
    kt_scale common = ZERO;
    for (size_t t = 0; t < T; t++) common = fold_max(common, rs[t]);
    rd_t o = {out, T * dim, ZERO};
    if (common.mant == 0) {
        memset(out, 0, T * dim * sizeof(int32_t));
        *os = ZERO;
        return;
    }
    const kt_scale cinv = kt_scale_recip(common);
    int64_t* a = (int64_t*)malloc(T * dim * sizeof(int64_t) + 8);
    for (size_t t = 0; t < T; t++) {
        const kt_scale f = kt_scale_mul(rs[t], cinv);
        for (size_t d = 0; d < dim; d++) a[t * dim + d] = kt_scale_apply(f, rows[t * dim + d]);
    }
    close_dyn(a, T * dim, common, &o);
    *os = o.s;
    free(a);
}

/* MoeMlp::forward_int (layers.rs:1031-1034): forward_routed (one token: forward_one_int; a sequence: token by token,
 * merged) then add_shared (the shared expert over the whole input, added by `add`). x: T x dim codes at xs. */
void kt_rm_forward(const void* p, const int32_t* x, size_t T, kt_scale xs, int32_t* out, kt_scale* os) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    const size_t dim = M->dim, K = M->top_k;
    int32_t* rows = (int32_t*)malloc(T * dim * sizeof(int32_t));
    kt_scale* rs = (kt_scale*)malloc(T * sizeof(kt_scale));
    int32_t* ys = (int32_t*)malloc(K * dim * sizeof(int32_t));
    kt_scale* ys_s = (kt_scale*)malloc(K * sizeof(kt_scale));
    int32_t sel[64];
    int64_t ec[64];
    for (size_t t = 0; t < T; t++) {
        const int64_t sumc = kt_rm_route(M, x + t * dim, xs, sel, ec, NULL, NULL);
        if (sumc <= 0) {
            memset(rows + t * dim, 0, dim * sizeof(int32_t));
            rs[t] = ZERO;
            continue;
        }
        rd_t row = {(int32_t*)x + t * dim, dim, xs};
        for (size_t i = 0; i < K; i++) {
            rd_t y = {ys + i * dim, dim, ZERO};
            mlp_forward(&M->experts[sel[i]], &M->silu, &row, &y);
            ys_s[i] = y.s;
        }
        kt_rm_combine(ys, ys_s, K, dim, ec, sumc, rows + t * dim, &rs[t]);
    }
    rd_t routed = t_new(T * dim);
    if (T <= 1) {
        memcpy(routed.d, rows, T * dim * sizeof(int32_t));
        routed.s = T ? rs[0] : ZERO;
    } else {
        kt_rm_merge_rows(rows, rs, T, dim, routed.d, &routed.s);
    }
    if (M->has_shared) {
        rd_t xin = {(int32_t*)x, T * dim, xs}, sh = t_new(T * dim);
        mlp_forward(&M->shared, &M->silu, &xin, &sh);
        kt_rd_add(routed.d, routed.s, sh.d, sh.s, T * dim, out, os);
        t_free(&sh);
    } else {
        memcpy(out, routed.d, T * dim * sizeof(int32_t));
        *os = routed.s;
    }
    t_free(&routed);
    free(rows), free(rs), free(ys), free(ys_s);
}

/* SwiGluMlp::forward_int of one expert (e < E) or the shared expert (e == E) on rows x dim codes at xs. */
void kt_rm_expert(const void* p, size_t e, const int32_t* x, size_t rows, kt_scale xs, int32_t* y, kt_scale* ys) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    rd_t xin = {(int32_t*)x, rows * M->dim, xs}, out = {y, rows * M->dim, ZERO};
    mlp_forward(e < M->E ? &M->experts[e] : &M->shared, &M->silu, &xin, &out);
    *ys = out.s;
}

/* Accessors for loading the same layer on the device. which: 0 router; for experts e (e == E: shared) 1 gate,
 * 2 up, 3 down. */
kt_scale kt_rm_get_ql(const void* p, size_t e, int which, int32_t* codes, size_t* out, size_t* in) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    const rd_ql* q;
    if (which == 0) {
        q = &M->router;
    } else {
        const rd_mlp* m = e < M->E ? &M->experts[e] : &M->shared;
        q = which == 1 ? &m->gate : which == 2 ? &m->up : &m->down;
    }
    if (codes) memcpy(codes, q->w, q->out * q->in * sizeof(int32_t));
    *out = q->out, *in = q->in;
    return q->s;
}
/* The run-time tables: which 0 exp, 1 sigmoid, 2 silu (as kt_rd_get_lut); and the coded bias (E values). */
void kt_rm_get_lut(const void* p, int which, int64_t* codes, kt_scale* inv_step, int64_t* lo_index,
                   kt_scale* code_scale) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    const rd_lut* L = which == 0 ? &M->exp_code : which == 1 ? &M->sig : &M->silu;
    if (codes) memcpy(codes, L->codes, L->n * sizeof(int64_t));
    *inv_step = L->inv_step_scale, *lo_index = L->lo_index, *code_scale = L->code_scale;
}
void kt_rm_get_bias(const void* p, int64_t* bias) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    memcpy(bias, M->bias, M->E * sizeof(int64_t));
}

/* IntTensor::from_reals (tensor.rs:106-117) of the reference tests' probe (tests.rs:29-32): rows x cols reals
 * uniform in [-1, 1) from the stream s, quantized to ACT_LEVELS by their largest magnitude. */
kt_scale kt_rm_probe(uint64_t* s, size_t n, int32_t* out) {
    double* real = (double*)malloc(n * sizeof(double) + 8);
    double mx = 0.0;
    for (size_t i = 0; i < n; i++) {
        real[i] = (double)unif_f32(s);
        const double a = fabs(real[i]);
        mx = a > mx ? a : mx;
    }
    kt_scale sc = ZERO;
    if (mx == 0.0) {
        memset(out, 0, n * sizeof(int32_t));
    } else {
        const double step = mx / (double)ACT_LEVELS, inv = (double)ACT_LEVELS / mx;
        sc = kt_scale_from_f64(step);
        for (size_t i = 0; i < n; i++) out[i] = (int32_t)round(real[i] * inv);
    }
    free(real);
    return sc;
}

/* The sigmoid router's selection bias: set expert e's to round(b * 2^20) for the f32 value b (SigmoidScore::new,
 * router.rs:38-49); the reference tests plant one (tests_glm.rs:183-200) or use all zeros. */
void kt_rm_set_bias(void* p, size_t e, float b) {
    kt_refmoe* M = (kt_refmoe*)p;
    M->bias[e] = (int64_t)round((double)b * (double)(1ULL << ROUTER_CODE_BITS));
}
/* The same MoeMlp with its QuantLinears given rather than drawn from seeded floats (MoeMlp::new over loaded
 * weights, layers.rs:652-700): every matrix zero at scale zero until kt_rm_set_ql fills it, the selection bias zero
 * until kt_rm_set_bias_code sets it, MoeMlp::new's and SigmoidScore::new's tables. For workloads at model size,
 * where the seeded float draw of the reference tests would take minutes. */
void* kt_rm_empty(size_t dim, size_t E, size_t top_k, size_t hidden, int norm_topk, int sigmoid,
                  size_t shared_hidden) {
    kt_refmoe* M = (kt_refmoe*)calloc(1, sizeof(kt_refmoe));
    M->dim = dim, M->E = E, M->top_k = top_k, M->hidden = hidden, M->shared_hidden = shared_hidden;
    M->norm_topk = norm_topk, M->sigmoid = sigmoid, M->has_shared = shared_hidden > 0;
    const kt_scale z = ZERO;
    M->router = (rd_ql){(int32_t*)calloc(E * dim, sizeof(int32_t)), z, E, dim};
    M->experts = (rd_mlp*)calloc(E, sizeof(rd_mlp));
    for (size_t e = 0; e <= E; e++) {
        const size_t h = e < E ? hidden : shared_hidden;
        if (e == E && !M->has_shared) break;
        rd_mlp* m = e < E ? &M->experts[e] : &M->shared;
        m->gate = (rd_ql){(int32_t*)calloc(h * dim, sizeof(int32_t)), z, h, dim};
        m->up = (rd_ql){(int32_t*)calloc(h * dim, sizeof(int32_t)), z, h, dim};
        m->down = (rd_ql){(int32_t*)calloc(dim * h, sizeof(int32_t)), z, dim, h};
    }
    M->bias = (int64_t*)calloc(E, sizeof(int64_t));
    lut_build2(&M->exp_code, LUT_EXP, -30.0, 0.0, 16, ROUTER_CODE_BITS, 0);
    lut_build2(&M->sig, LUT_SIGMOID, -16.0, 16.0, 16, ROUTER_CODE_BITS, 0);
    lut_build2(&M->silu, LUT_SILU, -30.0, 30.0, 16, 20, 1);
    return M;
}
/* Fill one QuantLinear (which as kt_rm_get_ql: 0 router; 1 gate, 2 up, 3 down of expert e, e == E the shared
 * expert) with out x in codes at scale s. */
void kt_rm_set_ql(void* p, size_t e, int which, const int32_t* codes, kt_scale s) {
    kt_refmoe* M = (kt_refmoe*)p;
    rd_ql* q;
    if (which == 0) {
        q = &M->router;
    } else {
        rd_mlp* m = e < M->E ? &M->experts[e] : &M->shared;
        q = which == 1 ? &m->gate : which == 2 ? &m->up : &m->down;
    }
    memcpy(q->w, codes, q->out * q->in * sizeof(int32_t));
    q->s = s;
}
/* The sigmoid router's coded selection bias of expert e, as SigmoidScore holds it (round(b * 2^20)). */
void kt_rm_set_bias_code(void* p, size_t e, int64_t code) { ((kt_refmoe*)p)->bias[e] = code; }
/* SigmoidScore::codes (router.rs:61-63): n logits codes at scale ls -> sigma codes. */
void kt_rm_sigmoid_codes(const void* p, const int32_t* logits, size_t n, kt_scale ls, int64_t* out) {
    const kt_refmoe* M = (const kt_refmoe*)p;
    for (size_t j = 0; j < n; j++) out[j] = lut_code_at(&M->sig, lut_index(&M->sig, logits[j], ls));
}

/* ------------------------------------------------------------------------------------------------------------ */
/* The SAM 2.1 image path at the reference's semantics: Conv2d (crates/01-engine/kt-core/src/conv.rs:22-130),     */
/* the pixel entry IntTensor::from_reals (tensor.rs:106-117), the GELU CodeLut and apply_gelu                      */
/* (crates/03-models/kt-model-vision/src/nonlin.rs:7-47), FeedForward (hiera.rs:321-345)                           */
/* ------------------------------------------------------------------------------------------------------------ */

/* IntTensor::from_reals (tensor.rs:106-117): codes round(v * levels / max) at Scale::from_f64(max / levels). */
kt_scale kt_rc_from_reals(const double* real, size_t n, int64_t levels, int32_t* out) {
    double mx = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double a = fabs(real[i]);
        mx = a > mx ? a : mx;
    }
    if (mx == 0.0) {
        memset(out, 0, n * sizeof(int32_t));
        return ZERO;
    }
    const double step = mx / (double)levels, inv = (double)levels / mx;
    for (size_t i = 0; i < n; i++) out[i] = (int32_t)round(real[i] * inv);
    return kt_scale_from_f64(step);
}

/* Conv2d::from_weights / QuantLinear::from_weights (conv.rs:25-47, layers.rs:212-232): b = 12 weight codes. */
kt_scale kt_rc_quant_weights(const float* w, size_t n, int32_t* codes) { return quant_weights(w, n, codes); }

/* Conv2d::with_bias / QuantLinear::with_bias (conv.rs:49-60, layers.rs:234-245): codes round(b / step), step =
 * max |b| / ACT_LEVELS (no clamp), Scale::from_f64(step); a zero bias gives no bias (returns 0). */
int kt_rc_quant_bias(const float* b, size_t n, int64_t* codes, kt_scale* bs) {
    double mx = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double a = fabs((double)b[i]);
        mx = a > mx ? a : mx;
    }
    if (!(mx > 0.0)) return 0;
    const double step = mx / (double)ACT_LEVELS;
    for (size_t i = 0; i < n; i++) codes[i] = (int64_t)round((double)b[i] / step);
    *bs = kt_scale_from_f64(step);
    return 1;
}

/* Conv2d::forward_int (conv.rs:68-130): x [ci][h][w] codes at xs, quant_to by its whole-tensor max, the direct
 * convolution (accumulation order (ic, ky, kx), taps outside the image skipped) against w [co][ci][kh][kw] at ws, the
 * bias in units of c, then requant_dyn by the whole output's max. out [co][oh][ow]. bias may be NULL. */
/* One block of output channels [oc0, oc1) of the direct convolution (conv.rs:91-120), accumulation order
 * (ic, ky, kx); the bias in units of c added last. */
typedef struct {
    const int32_t *qx, *wc;
    const int64_t* bias;
    kt_scale f;
    size_t ci, h, w, kh, kw, stride, pad, oh, ow, oc0, oc1;
    int64_t* acc;
} rc_block;
static void* rc_conv_block(void* p) {
    const rc_block* B = (const rc_block*)p;
    for (size_t oc = B->oc0; oc < B->oc1; oc++) {
        const int64_t b = B->bias ? kt_scale_apply(B->f, B->bias[oc]) : 0;
        for (size_t oy = 0; oy < B->oh; oy++)
            for (size_t ox = 0; ox < B->ow; ox++) {
                int64_t a = 0;
                for (size_t ic = 0; ic < B->ci; ic++)
                    for (size_t ky = 0; ky < B->kh; ky++) {
                        const size_t iy = oy * B->stride + ky;
                        if (iy < B->pad || iy - B->pad >= B->h) continue;
                        for (size_t kx = 0; kx < B->kw; kx++) {
                            const size_t ix = ox * B->stride + kx;
                            if (ix < B->pad || ix - B->pad >= B->w) continue;
                            a = wadd(a, wmul(B->qx[(ic * B->h + iy - B->pad) * B->w + ix - B->pad],
                                             B->wc[((oc * B->ci + ic) * B->kh + ky) * B->kw + kx]));
                        }
                    }
                B->acc[(oc * B->oh + oy) * B->ow + ox] = wadd(a, b);
            }
    }
    return NULL;
}

void kt_rc_conv2d(const int32_t* x, kt_scale xs, size_t ci, size_t h, size_t w, const int32_t* wc, kt_scale ws,
                  size_t co, size_t kh, size_t kw, size_t stride, size_t pad, const int64_t* bias, kt_scale bs,
                  int32_t* out, kt_scale* os) {
    const size_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1, n = co * oh * ow;
    const size_t nx = ci * h * w;
    int64_t xmax = 0;
    for (size_t i = 0; i < nx; i++) {
        const int64_t a = abs_w((int64_t)x[i]);
        xmax = a > xmax ? a : xmax;
    }
    *os = ZERO;
    if (xmax == 0) {
        memset(out, 0, n * sizeof(int32_t));
        return;
    }
    int32_t* qx = (int32_t*)malloc(nx * sizeof(int32_t));
    for (size_t i = 0; i < nx; i++) { /* quant_to (layers.rs:23-31) */
        const int64_t num = (int64_t)x[i] * WLEVELS, half = xmax / 2;
        qx[i] = (int32_t)(num >= 0 ? (num + half) / xmax : -((-num + half) / xmax));
    }
    const kt_scale c = kt_scale_mul(kt_scale_mul(ratio((u128)xmax, WLEVELS), xs), ws);
    if (c.mant == 0) {
        memset(out, 0, n * sizeof(int32_t));
        free(qx);
        return;
    }
    kt_scale f = ZERO;
    if (bias) f = kt_scale_mul(bs, kt_scale_recip(c));
    int64_t* acc = (int64_t*)malloc(n * sizeof(int64_t));
    /* par_blocks (layers.rs:88-115): the output channels in contiguous blocks, one per worker, when the work is at
     * least 2^20 MAC; the calling thread takes the first block. Disjoint writes: the same integers for any split. */
    const size_t work = n * ci * kh * kw;
    size_t nt = work >= ((size_t)1 << 20) ? kt_resolve_threads(co) : 1;
    nt = nt < 1 ? 1 : (nt > co ? co : nt);
    const size_t chunk = (co + nt - 1) / nt, nb = (co + chunk - 1) / chunk;
    rc_block* blk = (rc_block*)calloc(nb ? nb : 1, sizeof(rc_block));
    pthread_t* th = (pthread_t*)calloc(nb ? nb : 1, sizeof(pthread_t));
    for (size_t i = 0; i < nb; i++) {
        const size_t a0 = i * chunk, a1 = a0 + chunk < co ? a0 + chunk : co;
        blk[i] = (rc_block){qx, wc, bias, f, ci, h, w, kh, kw, stride, pad, oh, ow, a0, a1, acc};
    }
    for (size_t i = 1; i < nb; i++) pthread_create(&th[i], NULL, rc_conv_block, &blk[i]);
    if (nb) rc_conv_block(&blk[0]);
    for (size_t i = 1; i < nb; i++) pthread_join(th[i], NULL);
    free(blk), free(th);
    rd_t o = {out, n, ZERO};
    close_dyn(acc, n, c, &o);
    *os = o.s;
    free(qx), free(acc);
}

/* nonlin.rs:7-21: erf by Abramowitz & Stegun 7.1.26, and the exact GELU 0.5 x (1 + erf(x / sqrt 2)). */
static double as_erf(double x) {
    const double sign = x < 0.0 ? -1.0 : 1.0;
    x = fabs(x);
    const double t = 1.0 / (1.0 + 0.3275911 * x);
    const double y =
        1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t *
                  exp(-x * x);
    return sign * y;
}
static double gelu_f64(double x) { return 0.5 * x * (1.0 + as_erf(x / 1.4142135623730951)); }

static rd_lut* gelu_lut(void) {
    static rd_lut L;
    static int built = 0;
    if (!built) {
        lut_build_f(&L, gelu_f64, -10.0, 10.0, 16, 20, 1);
        built = 1;
    }
    return &L;
}

/* build_gelu_lut (nonlin.rs:24-26): CodeLut(gelu, -10, 10, 2^16 entries, 20 code bits, identity right tail). */
void kt_rc_gelu_table(int64_t* codes, kt_scale* inv_step, int64_t* lo_index, kt_scale* code_scale) {
    const rd_lut* L = gelu_lut();
    if (codes) memcpy(codes, L->codes, L->n * sizeof(int64_t));
    *inv_step = L->inv_step_scale, *lo_index = L->lo_index, *code_scale = L->code_scale;
}

/* apply_gelu (nonlin.rs:30-45): each code -> the table's code (0 below it, the identity factor above), as i32, at
 * the table's code scale (no requantization). */
void kt_rc_apply_gelu(const int32_t* x, size_t n, kt_scale xs, int32_t* y, kt_scale* ys) {
    const rd_lut* L = gelu_lut();
    const kt_scale id_factor = kt_scale_mul(xs, kt_scale_recip(L->code_scale));
    for (size_t i = 0; i < n; i++) {
        const int64_t d = x[i], idx = lut_index(L, d, xs);
        const int64_t code = idx < 0 ? 0 : idx >= (int64_t)L->n ? kt_scale_apply(id_factor, d) : lut_code_at(L, idx);
        y[i] = (int32_t)code;
    }
    *ys = L->code_scale;
}

/* FeedForward::forward_int (hiera.rs:336-340): proj_in (+ bias) -> apply_gelu -> proj_out (+ bias). bi / bo may be
 * NULL (no bias). */
void kt_rc_feedforward(const int32_t* x, size_t rows, size_t dim, kt_scale xs, const int32_t* wi, kt_scale wis,
                       const int64_t* bi, kt_scale bis, size_t hidden, const int32_t* wo, kt_scale wos,
                       const int64_t* bo, kt_scale bos, int32_t* y, kt_scale* ys) {
    int64_t xm, ym;
    int32_t* h = (int32_t*)malloc(rows * hidden * sizeof(int32_t));
    int32_t* g = (int32_t*)malloc(rows * hidden * sizeof(int32_t));
    kt_scale hs, gs;
    kt_quant_linear_forward(x, rows, dim, xs, wi, hidden, wis, bi, bis, 0, h, &hs, &xm, &ym);
    kt_rc_apply_gelu(h, rows * hidden, hs, g, &gs);
    kt_quant_linear_forward(g, rows, hidden, gs, wo, dim, wos, bo, bos, 0, y, ys, &xm, &ym);
    free(h), free(g);
}
