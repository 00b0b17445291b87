// The reference decoder's own layers on the device, at the reference's integer semantics: activations are i32 codes
// at the 2^28 level with one kt-int Scale per tensor (a kt_hip_qscale record in device memory), every op closes
// with requant_dyn to that level by its own largest magnitude, and scales compose with kt-int's integer Scale
// arithmetic (kt_scale_dev.h). With kt_hip_quant_linear for every projection they run DecoderModel::decode_step
// (crates/01-engine/kt-core/src/model.rs:290-294, 338-353) with no host round trip:
//
//   rd_embed           Embedding::lookup of a token read from device memory              (layers.rs:1127-1140)
//   rd_rmsnorm         RmsNorm::forward_int                                                (layers.rs:392-434)
//   rd_add             add, the residual add                                               (layers.rs:121-136)
//   rd_swiglu          SwiGluMlp::forward_int between the gate/up and down products       (layers.rs:615-637)
//   rd_attention_step  Attention::decode_step between the q/k/v and o products:           (attention.rs:358-458)
//                      RoPE, the KV cache append with per-step scales, the integer-code
//                      softmax at a common score scale, the heads brought to one scale
//   rd_argmax          argmax_codes, the greedy choice, with an optional per-step record  (generate.rs:48-56)
//   rd_gelu            apply_gelu, SAM's GELU by its CodeLut (many CTAs: a whole image's  (kt-model-vision/src/
//                      tokens)                                                             nonlin.rs:30-45)
//
// Each kernel is one CTA of 1024 threads (one token's tensors are at most a few thousand values); the Scale
// arithmetic of a tensor runs in one thread, the per-element work in all of them. The offline tables
// (CodeLut::build, the RoPE Scales, Scale::from_f64) are built on the host with the C library's f64 functions, as
// the reference builds them with its platform's.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "kt_dpp.h"
#include "kt_kernels.h"
#include "kt_scale_dev.h"
#include "kt_w12_core.h"

namespace kt {

namespace {

constexpr int RD_THREADS = 1024;
constexpr int RD_WAVES = RD_THREADS / 64;
constexpr int RD_MAX_ROWS = 1024;  // RMSNorm rows in one call (one factor per thread)
constexpr int RD_PV_GROUP = 8;     // P.V by kv head for groups of up to this many q heads
constexpr int64_t ACT_LEVELS = 1LL << 28;

}  // namespace

// A QuantLinear output left as its exact sums by the one-row product (kt_hip_quant_linear_multi_sums), as the op
// reading it next takes it: the output's sums, its call's state (max |x|, c, mode) and where its record goes (or
// null). That op applies requant_dyn (layers.rs:33-39, 321-327) as ql_requant_kernel would: ymax = max |sum| over
// the output (i64::abs, wrapping, as the product's own maximum); codes requant_dyn(sum, 2^28, ymax) when the mode is
// 0 and ymax > 0, else zeros (x all zero, or c zero; the path carries no bias); the Scale from_ratio(ymax, 2^28) * c.
struct RqSums {
    const int64_t* acc;
    const QlState* st;
    kt_hip_qscale* rec;
};

// The arguments of rd_attention_step_kernel (kt_hip_ref_attention_step).
struct RdAttn {
    const int32_t *q, *k, *v;
    const kt_hip_qscale *qs, *ks, *vs;
    const int32_t* pos;
    int nh, nkv, hd, max_seq;
    int32_t *kc, *vc;                  // [max_seq][nkv * hd]
    kt_hip_sscale *kscale, *vscale;    // [max_seq]
    const kt_hip_sscale *cos, *sin;    // [max_seq][hd / 2]
    int64_t isq_mant;
    int32_t isq_shift;
    const int64_t* exp_codes;
    kt_hip_codelut exp;
    int32_t* o;
    kt_hip_qscale* os;
    unsigned char* ws;                 // the heads kernels' workspace (rd_heads_layout), or null: the one-CTA kernel
    int hb;                            // the one-CTA kernel: heads whose scores LDS holds at once
    int sums;                          // the heads kernels: q, k, v as the product's sums (qsum, ksum, vsum)
    RqSums qsum, ksum, vsum;
};

// Attention::forward_int over a sequence (prefill): the inputs, the tables and the workspace parts.
struct RdPrefill {
    const int32_t *q, *k, *v;          // T x nh*hd, T x nkv*hd, T x nkv*hd
    const kt_hip_qscale *qs, *ks, *vs;
    int T, nh, nkv, hd;
    const kt_hip_sscale *cos, *sin;    // [max_seq][hd / 2]
    int64_t isq_mant;
    int32_t isq_shift;
    const int64_t* exp_codes;
    kt_hip_codelut exp;
    int32_t *qd, *kd;                  // rotated q and k
    int64_t* hout;                     // [nh][T][hd]: the sums of numerator * v, then the outputs at the common scale
    int64_t* hsum;                     // [nh][T]: the numerators' sums
    Sc* fac;                           // [T][nh]: each (row, head)'s scale over the common one
    uint64_t* gmax;                    // the largest |output| at the common scale
    Sc* common;
    int32_t* o;                        // T x nh*hd
    kt_hip_qscale* os;
};

namespace {

__device__ inline Sc rec_sc(const kt_hip_qscale* r) { return Sc{r->mant, r->shift}; }
__device__ inline void put_rec(kt_hip_qscale* r, Sc s) {
    kt_hip_qscale o{};
    o.mant = s.mant, o.shift = s.shift;
    *r = o;
}
__device__ inline int64_t iabs(int64_t v) { return v < 0 ? (int64_t)(0 - (uint64_t)v) : v; }
__device__ inline int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
__device__ inline int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }

// Lane 0's value as a wave-uniform one (scalar registers). The one-thread Scale chains run in all lanes of wave 0 on
// such values, so their integer arithmetic is scalar and their branches are uniform, rather than per-lane code under
// a one-lane exec mask.
__device__ inline int64_t uni64(int64_t v) { return (int64_t)lane64((uint64_t)v, 0); }
__device__ inline Sc uni(Sc s) { return Sc{uni64(s.mant), __builtin_amdgcn_readlane(s.shift, 0)}; }
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }
// Block-wide reductions over the CTA's 1024 threads; every thread gets the result: each wave's result to LDS, one
// barrier, the 16 of them reduced in row 0 of every wave.
__device__ int64_t block_max_i64(int64_t v, int64_t* red) {
    v = wave_max_i64(v);
    const int lane = threadIdx.x & 63;
    if (lane == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = (int64_t)lane64((uint64_t)row_max_i64(lane < RD_WAVES ? red[lane] : INT64_MIN), 0);
    __syncthreads();
    return v;
}
// The same reductions for CTAs of 256 threads (4 waves).
__device__ int64_t block_max_4w(int64_t v, int64_t* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const int64_t u = __shfl_xor(v, o, 64);
        v = u > v ? u : v;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
    for (int w = 1; w < 4; w++) v = red[w] > v ? red[w] : v;
    __syncthreads();
    return v;
}
__device__ int64_t block_sum_4w(int64_t v, int64_t* red) {  // wrapping
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = wadd(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
    for (int w = 1; w < 4; w++) v = wadd(v, red[w]);
    __syncthreads();
    return v;
}

// Block maxima of two or three values at once (one pair of barriers); red holds 3 x RD_WAVES values.
template <int K>
__device__ void block_max_k(int64_t (&v)[K], int64_t* red) {
#pragma unroll
    for (int k = 0; k < K; k++) {
        v[k] = wave_max_i64(v[k]);
        if ((threadIdx.x & 63) == 0) red[k * RD_WAVES + (threadIdx.x >> 6)] = v[k];
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < K; k++)
        v[k] = (int64_t)lane64((uint64_t)row_max_i64(lane < RD_WAVES ? red[k * RD_WAVES + lane] : INT64_MIN), 0);
    __syncthreads();
}

// requant_dyn of a sums output (RqSums): whether its codes are live, the Scale, the record as ql_requant_kernel
// writes it.
__device__ inline bool rqs_live(const QlState* st, int64_t ymax) { return st->mode == 0 && ymax > 0; }
__device__ inline Sc rqs_scale(const QlState* st, int64_t ymax) {
    return rqs_live(st, ymax) ? sc_mul(from_ratio((u128)(uint64_t)ymax, (u128)ACT_LEVELS), Sc{st->c_mant, st->c_shift})
                              : Sc{0, 0};
}
// rqs_scale with the state's fields read as wave-uniform values (wave 0's scalar chains)
__device__ inline Sc rqs_scale_u(const QlState* st, int64_t ymax) {
    const int mode = __builtin_amdgcn_readfirstlane(st->mode);
    const Sc c = uni(Sc{st->c_mant, st->c_shift});
    return mode == 0 && ymax > 0 ? sc_mul(from_ratio((u128)(uint64_t)ymax, (u128)ACT_LEVELS), c) : Sc{0, 0};
}
__device__ inline void rqs_record(const RqSums& r, int64_t ymax, Sc s) {
    if (!r.rec) return;
    kt_hip_qscale o{};
    o.xmax = r.st->xmax;
    if (rqs_live(r.st, ymax)) o.mant = s.mant, o.shift = s.shift, o.ymax = ymax;
    *r.rec = o;
}

// The engine's largest-scale fold (|a, b| if b.ge(a) { b } else { a } from Scale::ZERO, in sequence order) as a
// parallel reduction: of equal values the one latest in the sequence wins, as in the fold. idx < 0: no element.
struct ScIdx {
    Sc s;
    int idx;
};
__device__ inline ScIdx sc_pick(ScIdx a, ScIdx b) {
    if (a.idx < 0) return b;
    if (b.idx < 0) return a;
    const bool ab = sc_ge(a.s, b.s), ba = sc_ge(b.s, a.s);
    if (ab && ba) return a.idx > b.idx ? a : b;
    return ba ? b : a;
}
// The fold's total order as a key of three words per item: each Scale normalized exactly to m * 2^e with m's top bit
// set (e = -shift - clz(mant) lies in [-2^31 - 63, 2^31], stored as e + 2^40 > 0), so comparing values (sc_ge) is
// comparing (e, m) as integers, and the index breaks ties (the fold's later-wins rule). The third word holds the
// index above the item's clz, which the order then ignores (indices are distinct) and from which the winner's own
// (mant, shift) comes back exactly: mant = m >> clz, shift = -e - clz. A dead item (idx < 0 or a zero Scale) is the
// key (0, 0, 0), below every live one.
struct FoldKey {
    uint64_t e, m, i;
};
__device__ inline FoldKey fold_key(const ScIdx& v) {
    const bool live = v.idx >= 0 && v.s.mant != 0;
    const uint64_t a = (uint64_t)v.s.mant;
    const int lz = live ? __builtin_clzll(a) : 0;
    return live ? FoldKey{(uint64_t)(-(int64_t)v.s.shift - lz + (1LL << 40)), a << lz,
                          ((uint64_t)(uint32_t)v.idx << 6) | (uint64_t)lz}
                : FoldKey{0, 0, 0};
}
__device__ inline ScIdx fold_item(const FoldKey& k) {
    if (k.e == 0) return ScIdx{Sc{0, 0}, -1};
    const int lz = (int)(k.i & 63);
    return ScIdx{Sc{(int64_t)(k.m >> lz), (int32_t)(-((int64_t)k.e - (1LL << 40)) - lz)}, (int)(k.i >> 6)};
}
__device__ inline bool fold_gt(const FoldKey& x, const FoldKey& y) {
    return x.e != y.e ? x.e > y.e : (x.m != y.m ? x.m > y.m : x.i > y.i);
}
template <int CTRL>
__device__ inline void fold_dpp(FoldKey& k) {
    const FoldKey u{dpp64<CTRL>(k.e), dpp64<CTRL>(k.m), dpp64<CTRL>(k.i)};
    if (fold_gt(u, k)) k = u;
}
__device__ inline void fold_row(FoldKey& k) {
    fold_dpp<DPP_XOR1>(k);
    fold_dpp<DPP_XOR2>(k);
    fold_dpp<DPP_HALF_MIRROR>(k);
    fold_dpp<DPP_MIRROR>(k);
}
__device__ inline FoldKey fold_lane(const FoldKey& k, int l) { return FoldKey{lane64(k.e, l), lane64(k.m, l), lane64(k.i, l)}; }
// The engine's fold over K sequences at once, one item per thread for each: the largest key of each wave by DPP
// steps, one barrier, the 16 waves' keys folded in row 0 of every wave; the winners (their own Scales and indices)
// are returned. Ends with a barrier. red: at least 3 K RD_WAVES words.
template <int K>
__device__ void block_fold_max_k(ScIdx (&v)[K], ScIdx* red) {
    uint64_t* r64 = reinterpret_cast<uint64_t*>(red);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    FoldKey k[K];
#pragma unroll
    for (int q = 0; q < K; q++) {
        k[q] = fold_key(v[q]);
        fold_row(k[q]);
        FoldKey b = fold_lane(k[q], 0);
#pragma unroll
        for (int l = 16; l < 64; l += 16) {
            const FoldKey c = fold_lane(k[q], l);
            if (fold_gt(c, b)) b = c;
        }
        k[q] = b;
    }
    if (lane == 0)
#pragma unroll
        for (int q = 0; q < K; q++) {
            uint64_t* d = r64 + (q * RD_WAVES + w) * 3;
            d[0] = k[q].e, d[1] = k[q].m, d[2] = k[q].i;
        }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < K; q++) {
        FoldKey b{0, 0, 0};
        if (lane < RD_WAVES) {
            const uint64_t* d = r64 + (q * RD_WAVES + lane) * 3;
            b = FoldKey{d[0], d[1], d[2]};
        }
        fold_row(b);
        v[q] = fold_item(fold_lane(b, 0));
    }
    __syncthreads();
}
// n: how many leading threads hold items (the rest hold idx -1); every thread of the CTA calls it. Ends with a
// barrier.
__device__ ScIdx block_fold_max(ScIdx v, ScIdx* red, int n) {
    (void)n;
    ScIdx a[1] = {v};
    block_fold_max_k<1>(a, red);
    return a[0];
}

// CodeLut::index / code_at (kt-int/src/lib.rs:382-395) with the call's factor m = scale * inv_step.
__device__ inline int64_t lut_index(Sc m, int64_t data, int64_t lo_index) { return sc_apply(m, data) - lo_index; }
// the same for an i32 code, in 64-bit arithmetic where sc_apply32 allows
__device__ inline int64_t lut_index32(Sc m, int32_t data, int64_t lo_index) { return sc_apply32(m, data) - lo_index; }
__device__ inline int64_t lut_code(const int64_t* codes, int n, int64_t idx) {
    return codes[idx < 0 ? 0 : (idx > n - 1 ? n - 1 : idx)];
}

}  // namespace

// Embedding::lookup (layers.rs:1127-1140): y = the token's code row at the table's scale. A token outside
// [0, vocab) gives zeros at Scale::ZERO (the reference panics there; a kernel must not read out of bounds).
__global__ __launch_bounds__(RD_THREADS) void rd_embed_kernel(const int32_t* __restrict__ emb, int64_t e_mant,
                                                              int32_t e_shift, const int32_t* __restrict__ token,
                                                              int vocab, int dim, int32_t* __restrict__ y,
                                                              kt_hip_qscale* __restrict__ ys) {
    const int t = *token;
    const bool ok = t >= 0 && t < vocab;
    for (int i = threadIdx.x; i < dim; i += RD_THREADS) y[i] = ok ? emb[(size_t)t * dim + i] : 0;
    if (threadIdx.x == 0) put_rec(ys, ok ? Sc{e_mant, e_shift} : Sc{0, 0});
}

// RmsNorm::forward_int of one row held in registers (NV values per thread, value i = threadIdx.x + RD_THREADS * k,
// dim <= RD_THREADS * NV; gv the gammas likewise): the exact sum of squares reduced across the CTA, the row factor
// c = xs * rsqrt(mean_sq + eps) * gs by thread 0 (only thread 0 reads xs), the products brought to c and
// requantized by their largest magnitude. The same integers as rd_rmsnorm_kernel's general path for one row.
template <int NV>
__device__ void rd_norm_row(int32_t (&xv)[NV], const int32_t (&gv)[NV], int dim, Sc xs, Sc gs, Sc eps,
                            int32_t* __restrict__ y, kt_hip_qscale* __restrict__ ys, int64_t* red) {
    __shared__ uint64_t sq2[RD_WAVES][2];
    __shared__ Sc cf[2];  // c and its factor over itself
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t hi = 0, lo = 0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if ((int)threadIdx.x + RD_THREADS * k >= dim) xv[k] = 0;
        const int64_t v = xv[k];
        const uint64_t sq = (uint64_t)(v * v), t = lo + sq;
        hi += t < lo, lo = t;
    }
    add128_row(hi, lo);
    {  // the four rows' sums
        u128 w = 0;
#pragma unroll
        for (int l = 0; l < 64; l += 16) w += ((u128)lane64(hi, l) << 64) | lane64(lo, l);
        hi = (uint64_t)(w >> 64), lo = (uint64_t)w;
    }
    if (lane == 0) sq2[wave][0] = hi, sq2[wave][1] = lo;
    __syncthreads();
    const int wv = wave_id();
    Sc cc{0, 0};  // wave 0: the row factor (uniform)
    if (wv == 0) {  // the 16 waves' sums (lane q < 16 reads wave q's), then the row factor's chain on scalars
        uint64_t h2 = lane < RD_WAVES ? sq2[lane][0] : 0, l2 = lane < RD_WAVES ? sq2[lane][1] : 0;
        add128_row(h2, l2);
        const u128 ss = ((u128)lane64(h2, 0) << 64) | lane64(l2, 0);
        const Sc xu = uni(xs);
        const Sc mean_sq = sc_mul(sc_mul(from_ratio(ss, (u128)dim), xu), xu);
        const Sc denom = sc_add(mean_sq, eps);
        const Sc inv = denom.mant == 0 ? Sc{0, 0} : sc_rsqrt(denom);
        cc = sc_mul(sc_mul(xu, inv), gs);  // the largest of one row's factors is that factor
        const Sc f = cc.mant != 0 ? sc_mul(cc, sc_recip(cc)) : Sc{0, 0};
        if (lane == 0) cf[0] = cc, cf[1] = f;
    }
    __syncthreads();
    const Sc f0 = cf[1];
    if (wv != 0) cc = cf[0];
    int64_t hv[NV];
    int64_t m = 0;
#pragma unroll
    for (int k = 0; k < NV; k++) {  // values past dim stay 0 (whole waves skip the 128-bit products)
        hv[k] = 0;
        if (cc.mant != 0 && (int)threadIdx.x + RD_THREADS * k < dim)
            hv[k] = sc_apply(f0, (int64_t)xv[k] * (int64_t)gv[k]);
        m = iabs(hv[k]) > m ? iabs(hv[k]) : m;
    }
    const int64_t gmax = block_max_i64(m, red);
    const RqDen rd_gmax = rq_den(gmax);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int i = threadIdx.x + RD_THREADS * k;
        if (i < dim) y[i] = gmax == 0 ? 0 : rq_apply(rd_gmax, hv[k]);
    }
    if (wv == 0) {
        const Sc r = gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), cc);
        if (lane == 0) put_rec(ys, r);
    }
}

// RmsNorm::forward_int (layers.rs:392-434) over `rows` rows of `dim`: per row the exact sum of squares, its
// mean-square Scale plus eps, the integer inverse square root, the row factor c_r = xs * inv * gs; the products
// x_i * g_i brought to the largest c_r and requantized by the largest magnitude.
__global__ __launch_bounds__(RD_THREADS) void rd_rmsnorm_kernel(const int32_t* __restrict__ x, int rows, int dim,
                                                                const kt_hip_qscale* __restrict__ xs_rec,
                                                                const int32_t* __restrict__ g, int64_t g_mant,
                                                                int32_t g_shift, int64_t e_mant, int32_t e_shift,
                                                                int32_t* __restrict__ y,
                                                                kt_hip_qscale* __restrict__ ys) {
    __shared__ int64_t red[RD_WAVES];
    __shared__ Sc crow[RD_MAX_ROWS], frow[RD_MAX_ROWS];
    __shared__ ScIdx redsc[RD_THREADS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const Sc xs = rec_sc(xs_rec), gs{g_mant, g_shift}, eps{e_mant, e_shift};
    constexpr int RD_NV = 8;
    if (rows == 1 && dim <= RD_THREADS * RD_NV) {
        // one row (the decode step): its values and gammas loaded once by every thread, all in flight together
        int32_t xv[RD_NV], gv[RD_NV];
#pragma unroll
        for (int k = 0; k < RD_NV; k++) {
            const int i = threadIdx.x + RD_THREADS * k, ic = i < dim ? i : dim - 1;
            xv[k] = x[ic], gv[k] = g[ic];
        }
        rd_norm_row<RD_NV>(xv, gv, dim, xs, gs, eps, y, ys, red);
        return;
    }
    // each row's exact sum of squares by one wave, its factor c_r = xs * rsqrt(mean_sq + eps) * gs by that wave's
    // first lane (the rows' Scale arithmetic runs side by side)
    for (int r = wave; r < rows; r += RD_WAVES) {
        uint64_t hi = 0, lo = 0;  // the u128 sum as two words: squares below 2^62, at most 2^26 of them per lane
        for (int i = lane; i < dim; i += 64) {
            const int64_t v = x[(size_t)r * dim + i];
            const uint64_t sq = (uint64_t)(v * v), t = lo + sq;
            hi += t < lo, lo = t;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t ohi = __shfl_xor(hi, o, 64), olo = __shfl_xor(lo, o, 64), t = lo + olo;
            hi += ohi + (t < lo), lo = t;
        }
        if (lane == 0) {
            const u128 ss = ((u128)hi << 64) | lo;
            const Sc mean_sq = sc_mul(sc_mul(from_ratio(ss, (u128)dim), xs), xs);
            const Sc denom = sc_add(mean_sq, eps);
            const Sc inv = denom.mant == 0 ? Sc{0, 0} : sc_rsqrt(denom);
            crow[r] = sc_mul(sc_mul(xs, inv), gs);
        }
    }
    __syncthreads();
    // the largest row factor by the engine's fold (of equal values the latest row's), then each row's share of it
    ScIdx best{Sc{0, 0}, -1};
    for (int r = threadIdx.x; r < rows; r += RD_THREADS) best = sc_pick(best, ScIdx{crow[r], r});
    const Sc cc = block_fold_max(best, redsc, rows).s;
    if (cc.mant != 0) {
        const Sc cinv = sc_recip(cc);  // every thread: one Scale reciprocal, no extra barrier
        for (int r = threadIdx.x; r < rows; r += RD_THREADS) frow[r] = sc_mul(crow[r], cinv);
    }
    __syncthreads();
    const int n = rows * dim;
    int64_t m = 0;
    if (cc.mant != 0)
        for (int i = threadIdx.x; i < n; i += RD_THREADS) {
            const int64_t v = sc_apply(frow[i / dim], (int64_t)x[i] * (int64_t)g[i % dim]);
            m = iabs(v) > m ? iabs(v) : m;
        }
    const int64_t gmax = block_max_i64(m, red);
    const RqDen rd_gmax = rq_den(gmax);
    for (int i = threadIdx.x; i < n; i += RD_THREADS)
        y[i] = gmax == 0 ? 0 : rq_apply(rd_gmax, sc_apply(frow[i / dim], (int64_t)x[i] * (int64_t)g[i % dim]));
    if (threadIdx.x == 0)
        put_rec(ys, gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), cc));
}

// add (layers.rs:121-136): both to the larger scale, summed, requantized. y may alias a or b.
__global__ __launch_bounds__(RD_THREADS) void rd_add_kernel(const int32_t* a, const kt_hip_qscale* as_rec,
                                                            const int32_t* b, const kt_hip_qscale* bs_rec, int n,
                                                            int32_t* y, kt_hip_qscale* ys) {
    __shared__ int64_t red[RD_WAVES];
    __shared__ Sc par[3];  // common, fa, fb
    // up to RD_AV values per thread held in registers, their loads issued before the Scale work of thread 0 so that
    // the two overlap; longer tensors read a and b twice
    constexpr int RD_AV = 4;
    const bool held = n <= RD_THREADS * RD_AV;
    int32_t av[RD_AV], bv[RD_AV];
    if (held) {
#pragma unroll
        for (int k = 0; k < RD_AV; k++) {
            const int i = threadIdx.x + RD_THREADS * k, ic = i < n ? i : n - 1;
            av[k] = a[ic], bv[k] = b[ic];
        }
    }
    if (threadIdx.x == 0) {
        const Sc as = rec_sc(as_rec), bs = rec_sc(bs_rec);
        const Sc common = sc_ge(as, bs) ? as : bs;
        par[0] = common;
        if (common.mant != 0) {
            const Sc cinv = sc_recip(common);
            par[1] = sc_mul(as, cinv), par[2] = sc_mul(bs, cinv);
        }
    }
    __syncthreads();
    const Sc common = par[0], fa = par[1], fb = par[2];
    int64_t m = 0, hv[RD_AV];
    if (held) {
#pragma unroll
        for (int k = 0; k < RD_AV; k++) {  // values past n stay 0 (whole waves skip them)
            hv[k] = 0;
            if (common.mant != 0 && (int)threadIdx.x + RD_THREADS * k < n)
                hv[k] = wadd(sc_apply32(fa, av[k]), sc_apply32(fb, bv[k]));
            m = iabs(hv[k]) > m ? iabs(hv[k]) : m;
        }
    } else if (common.mant != 0) {
        for (int i = threadIdx.x; i < n; i += RD_THREADS) {
            const int64_t v = wadd(sc_apply32(fa, a[i]), sc_apply32(fb, b[i]));
            m = iabs(v) > m ? iabs(v) : m;
        }
    }
    const int64_t gmax = block_max_i64(m, red);  // every read of a, b, and their records, is done past here
    const RqDen rd_gmax = rq_den(gmax);
    if (held) {
#pragma unroll
        for (int k = 0; k < RD_AV; k++) {
            const int i = threadIdx.x + RD_THREADS * k;
            if (i < n) y[i] = gmax == 0 ? 0 : rq_apply(rd_gmax, hv[k]);
        }
    } else {
        for (int i = threadIdx.x; i < n; i += RD_THREADS)
            y[i] = gmax == 0 ? 0 : rq_apply(rd_gmax, wadd(sc_apply32(fa, a[i]), sc_apply32(fb, b[i])));
    }
    if (threadIdx.x == 0)
        put_rec(ys, gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), common));
}

// add (layers.rs:121-136) and then RmsNorm::forward_int (layers.rs:392-434) of the sum, for one row of
// n <= RD_THREADS * RD_AN values: the decode step's residual add followed by the next norm (model.rs:338-353), one
// launch where the two kernels took two. y = add(a, b) with its record ys (y may alias a or b), then h = the norm of
// y from the codes still in registers and the Scale thread 0 formed for ys. The same integers as rd_add_kernel and
// rd_rmsnorm_kernel in sequence. SUMS: b is a QuantLinear's sums (bsum), its requant_dyn and record formed here
// first, as ql_requant_kernel would.
constexpr int RD_AN = 4;
template <bool SUMS>
__global__ __launch_bounds__(RD_THREADS) void rd_add_norm_kernel(const int32_t* a, const kt_hip_qscale* as_rec,
                                                                 const int32_t* b, const kt_hip_qscale* bs_rec,
                                                                 RqSums bsum, int n, int32_t* y, kt_hip_qscale* ys,
                                                                 const int32_t* __restrict__ g, int64_t g_mant,
                                                                 int32_t g_shift, int64_t e_mant, int32_t e_shift,
                                                                 int32_t* __restrict__ h,
                                                                 kt_hip_qscale* __restrict__ hs) {
    __shared__ int64_t red[RD_WAVES];
    __shared__ Sc par[3];  // common, fa, fb
    int32_t av[RD_AN], bv[RD_AN], gv[RD_AN];
    int64_t bacc[RD_AN];
#pragma unroll
    for (int k = 0; k < RD_AN; k++) {
        const int i = threadIdx.x + RD_THREADS * k, ic = i < n ? i : n - 1;
        av[k] = a[ic], gv[k] = g[ic];
        if constexpr (SUMS) bacc[k] = bsum.acc[ic];
        else bv[k] = b[ic];
    }
    int64_t bmax = 0;
    if constexpr (SUMS) {  // b's maximum (the values past n repeat value n - 1), codes and Scale
#pragma unroll
        for (int k = 0; k < RD_AN; k++) bmax = iabs(bacc[k]) > bmax ? iabs(bacc[k]) : bmax;
        bmax = block_max_i64(bmax, red);
        const bool live = rqs_live(bsum.st, bmax);
        const RqDen d = rq_den(bmax);
#pragma unroll
        for (int k = 0; k < RD_AN; k++) bv[k] = live ? rq_apply(d, bacc[k]) : 0;
    }
    const int wv = wave_id(), lane = threadIdx.x & 63;
    Sc common{0, 0};  // wave 0: the common Scale (uniform)
    if (wv == 0) {  // the Scale chain on scalars
        Sc bs;
        if constexpr (SUMS) {
            bs = rqs_scale_u(bsum.st, bmax);
            if (lane == 0) rqs_record(bsum, bmax, bs);
        } else {
            bs = uni(rec_sc(bs_rec));
        }
        const Sc as = uni(rec_sc(as_rec));
        common = sc_ge(as, bs) ? as : bs;
        Sc fa{0, 0}, fb{0, 0};
        if (common.mant != 0) {
            const Sc cinv = sc_recip(common);
            fa = sc_mul(as, cinv), fb = sc_mul(bs, cinv);
        }
        if (lane == 0) par[0] = common, par[1] = fa, par[2] = fb;
    }
    __syncthreads();
    const Sc fa = par[1], fb = par[2];
    if (wv != 0) common = par[0];
    int64_t m = 0, hv[RD_AN];
#pragma unroll
    for (int k = 0; k < RD_AN; k++) {
        hv[k] = 0;
        if (common.mant != 0 && (int)threadIdx.x + RD_THREADS * k < n)
            hv[k] = wadd(sc_apply32(fa, av[k]), sc_apply32(fb, bv[k]));
        m = iabs(hv[k]) > m ? iabs(hv[k]) : m;
    }
    const int64_t gmax = block_max_i64(m, red);  // every read of a and b is done past here
    const RqDen rd_gmax = rq_den(gmax);
    int32_t yv[RD_AN];
#pragma unroll
    for (int k = 0; k < RD_AN; k++) {
        const int i = threadIdx.x + RD_THREADS * k;
        yv[k] = gmax == 0 ? 0 : rq_apply(rd_gmax, hv[k]);
        if (i < n) y[i] = yv[k];
    }
    Sc xs{0, 0};  // the sum's Scale: wave 0 writes the record and carries it into the norm
    if (wv == 0) {
        xs = gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), common);
        if (lane == 0) put_rec(ys, xs);
    }
    rd_norm_row<RD_AN>(yv, gv, n, xs, Sc{g_mant, g_shift}, Sc{e_mant, e_shift}, h, hs, red);
}

// SwiGluMlp::forward_int's activation (layers.rs:615-637): h = silu_code(g) * u, the SiLU code from the CodeLut at
// g's scale (0 below the table, the identity tail g * gs / code_scale above it), requantized at code_scale * us.
// One CTA per row: row r's n values with its own records gs_rec[r], us_rec[r], hs[r] (rows = 1: one tensor).
// SUMS (one row, n <= RD_THREADS * RD_VPT): g and u are QuantLinear sums (gsum, usum), their requant_dyn and records
// formed here first, as ql_requant_kernel would.
template <bool SUMS>
__global__ __launch_bounds__(RD_THREADS) void rd_swiglu_kernel(const int32_t* __restrict__ g,
                                                               const kt_hip_qscale* __restrict__ gs_rec,
                                                               const int32_t* __restrict__ u,
                                                               const kt_hip_qscale* __restrict__ us_rec, RqSums gsum,
                                                               RqSums usum, int n, const int64_t* __restrict__ codes,
                                                               kt_hip_codelut L, int32_t* __restrict__ h,
                                                               kt_hip_qscale* __restrict__ hs) {
    __shared__ int64_t red[3 * RD_WAVES];
    if constexpr (!SUMS) {
        const int64_t r = blockIdx.x;
        g += r * n, u += r * n, h += r * n, gs_rec += r, us_rec += r, hs += r;
    }
    // up to RD_VPT values per thread formed once and held in registers, their loads issued before thread 0's Scale
    // work so that the two overlap (the table reads follow the factors); longer rows form each value twice
    constexpr int RD_VPT = 8;
    const bool held = SUMS || n <= RD_THREADS * RD_VPT;
    int32_t gd[RD_VPT], ud[RD_VPT];
    int64_t gmax = 0, umax = 0;
    if constexpr (SUMS) {  // the sums, their maxima (the values past n repeat value n - 1), codes and Scales
        int64_t ga[RD_VPT], ua[RD_VPT];
#pragma unroll
        for (int i = 0; i < RD_VPT; i++) {
            const int k = threadIdx.x + RD_THREADS * i, kk = k < n ? k : n - 1;
            ga[i] = gsum.acc[kk], ua[i] = usum.acc[kk];
        }
        int64_t mx[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < RD_VPT; i++) {
            mx[0] = iabs(ga[i]) > mx[0] ? iabs(ga[i]) : mx[0];
            mx[1] = iabs(ua[i]) > mx[1] ? iabs(ua[i]) : mx[1];
        }
        block_max_k<2>(mx, red);
        gmax = mx[0], umax = mx[1];
        const bool lg = rqs_live(gsum.st, gmax), lu = rqs_live(usum.st, umax);
        const RqDen dg = rq_den(gmax), du = rq_den(umax);
#pragma unroll
        for (int i = 0; i < RD_VPT; i++) {
            gd[i] = lg ? rq_apply(dg, ga[i]) : 0;
            ud[i] = lu ? rq_apply(du, ua[i]) : 0;
        }
    } else if (held) {
#pragma unroll
        for (int i = 0; i < RD_VPT; i++) {
            const int k = threadIdx.x + RD_THREADS * i, kk = k < n ? k : n - 1;
            gd[i] = g[kk], ud[i] = u[kk];
        }
    }
    __shared__ Sc par[3];  // index factor, identity factor, h scale
    const Sc cs{L.code_mant, L.code_shift};
    if (threadIdx.x == 0) {  // g's factors (and with SUMS its Scale and record first)
        Sc gs;
        if constexpr (SUMS) {
            gs = rqs_scale(gsum.st, gmax);
            rqs_record(gsum, gmax, gs);
        } else {
            gs = rec_sc(gs_rec);
        }
        par[0] = sc_mul(gs, Sc{L.inv_mant, L.inv_shift});
        par[1] = sc_mul(gs, sc_recip(cs));
    }
    if (threadIdx.x == 64) {  // u's side, in another wave
        Sc us;
        if constexpr (SUMS) {
            us = rqs_scale(usum.st, umax);
            rqs_record(usum, umax, us);
        } else {
            us = rec_sc(us_rec);
        }
        par[2] = sc_mul(cs, us);
    }
    __syncthreads();
    const Sc mi = par[0], idf = par[1], hsc = par[2];
    auto act = [&](int k) -> int64_t {
        const int32_t gk = g[k];
        const int64_t idx = lut_index32(mi, gk, L.lo_index);
        const int64_t code = idx < 0 ? 0 : (idx >= L.n ? sc_apply32(idf, gk) : lut_code(codes, L.n, idx));
        return wmul(code, u[k]);
    };
    int64_t hv[RD_VPT];
    int64_t m = 0;
    if (held) {
#pragma unroll
        for (int i = 0; i < RD_VPT; i++) {  // values past n stay 0 (whole waves skip them)
            hv[i] = 0;
            if ((int)threadIdx.x + RD_THREADS * i < n) {
                const int64_t idx = lut_index32(mi, gd[i], L.lo_index);
                const int64_t code = idx < 0 ? 0 : (idx >= L.n ? sc_apply32(idf, gd[i]) : lut_code(codes, L.n, idx));
                hv[i] = wmul(code, ud[i]);
            }
            m = iabs(hv[i]) > m ? iabs(hv[i]) : m;
        }
    } else {
        for (int k = threadIdx.x; k < n; k += RD_THREADS) {
            const int64_t a = iabs(act(k));
            m = a > m ? a : m;
        }
    }
    const int64_t hmax = block_max_i64(m, red);
    const RqDen rd_hmax = rq_den(hmax);
    if (held) {
#pragma unroll
        for (int i = 0; i < RD_VPT; i++) {
            const int k = threadIdx.x + RD_THREADS * i;
            if (k < n) h[k] = hmax == 0 ? 0 : rq_apply(rd_hmax, hv[i]);
        }
    } else {
        for (int k = threadIdx.x; k < n; k += RD_THREADS) h[k] = hmax == 0 ? 0 : rq_apply(rd_hmax, act(k));
    }
    if (threadIdx.x == 0)
        put_rec(hs, hmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)hmax, (u128)ACT_LEVELS), hsc));
}

// apply_gelu (kt-model-vision/src/nonlin.rs:30-45): each code through the GELU CodeLut at x's scale (0 below the
// table, the identity factor xs / code_scale above it), cast to i32, the output at the table's code scale with no
// requantization. Grid-stride over n; each CTA forms the two factors from the record.
__global__ __launch_bounds__(RD_THREADS) void rd_gelu_kernel(const int32_t* __restrict__ x,
                                                             const kt_hip_qscale* __restrict__ xs_rec, int64_t n,
                                                             const int64_t* __restrict__ codes, kt_hip_codelut L,
                                                             int32_t* __restrict__ y,
                                                             kt_hip_qscale* __restrict__ ys) {
    __shared__ Sc par[2];  // index factor, identity factor
    const Sc cs{L.code_mant, L.code_shift};
    if (threadIdx.x == 0) {
        const Sc xs = rec_sc(xs_rec);
        par[0] = sc_mul(xs, Sc{L.inv_mant, L.inv_shift});
        par[1] = sc_mul(xs, sc_recip(cs));
    }
    __syncthreads();
    const Sc mi = par[0], idf = par[1];
    const int64_t step = (int64_t)gridDim.x * RD_THREADS;
    for (int64_t i = (int64_t)blockIdx.x * RD_THREADS + threadIdx.x; i < n; i += step) {
        const int32_t d = x[i];
        const int64_t idx = lut_index32(mi, d, L.lo_index);
        const int64_t code = idx < 0 ? 0 : (idx >= L.n ? sc_apply32(idf, d) : lut_code(codes, L.n, idx));
        y[i] = (int32_t)code;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) put_rec(ys, cs);
}

// Attention::decode_step between its projections (attention.rs:358-458), at the position *pos:
//  1. RoPE (rope_int, attention.rs:222-246) of every q head into LDS and every k head into the cache row pos; v
//     into its cache row; this step's k and v scales into the per-step scale arrays;
//  2. v_ref = the largest v scale over the steps 0..pos, vf_j = vs_j / v_ref; the score scales
//     s_j = qs * ks_j * inv_sqrt, s_ref = the largest, f_j = s_j / s_ref;
//  3. per head: score_j = f_j.apply(q . k_j), ec_j = exp_code(score_j - max score) at s_ref (0 below the table),
//     sumc = sum ec_j, out_d = sum_j ec_j * vf_j.apply(v_jd), scale_h = v_ref / sumc;
//  4. the heads brought to the largest scale_h and requantized: o and its record.
// LDS: the per-step arrays (score and v factors, 32 B per cached position; hb heads' scores, 8 B per position each)
// for max_seq positions, then the head outputs and the rotated q (12 B per q value).
struct RdAttnShared {
    int64_t red[RD_WAVES];
    ScIdx redsc[RD_THREADS];
    Sc par[4];  // v_ref, s_ref, lut factor, common
    Sc hsc[64];
    Sc inv2[2];
    int64_t hsum[KT_REF_MAX_HEADS];
};

__device__ __forceinline__ void rd_attention_core(const RdAttn& a, unsigned char* lds, RdAttnShared& sh_,
                                                  int pos, int hb) {
    int64_t* red = sh_.red;
    ScIdx* redsc = sh_.redsc;
    Sc* par = sh_.par;
    Sc* hsc = sh_.hsc;
    const int tid = threadIdx.x, hd = a.hd, half = hd / 2, nh = a.nh, nkv = a.nkv, group = nh / nkv;
    const int kstride = nkv * hd, qstride = nh * hd;
    const int steps = pos + 1, rows = a.max_seq;  // rows: the per-step arrays' length
    Sc* F = reinterpret_cast<Sc*>(lds);  // score factors, per step
    Sc* VF = F + rows;                   // v factors, per step
    int64_t* S = reinterpret_cast<int64_t*>(VF + rows);   // scores, then exp codes: [hb][rows]
    int64_t* HO = S + (size_t)hb * rows;                  // head outputs, qstride
    int32_t* QD = reinterpret_cast<int32_t*>(HO + qstride);  // rotated q, qstride

    // 1. RoPE and the cache append
    auto rot = [&](const int32_t* src, int32_t* dst, int heads) {
        for (int i = tid; i < heads * half; i += RD_THREADS) {
            const int hh = i / half, j = i - hh * half;
            const kt_hip_sscale c = a.cos[(size_t)pos * half + j], s = a.sin[(size_t)pos * half + j];
            const int32_t av = src[hh * hd + j], bv = src[hh * hd + j + half];
            const Sc cm{c.mant, c.shift}, sm{s.mant, s.shift};
            dst[hh * hd + j] = (int32_t)(c.sign * sc_apply32(cm, av) - s.sign * sc_apply32(sm, bv));
            dst[hh * hd + j + half] = (int32_t)(c.sign * sc_apply32(cm, bv) + s.sign * sc_apply32(sm, av));
        }
    };
    rot(a.q, QD, nh);
    rot(a.k, a.kc + (size_t)pos * kstride, nkv);
    for (int i = tid; i < kstride; i += RD_THREADS) a.vc[(size_t)pos * kstride + i] = a.v[i];
    const Sc qs = rec_sc(a.qs), isq{a.isq_mant, a.isq_shift};
    if (tid == 0) {
        a.kscale[pos] = kt_hip_sscale{a.ks->mant, a.ks->shift, 1};
        a.vscale[pos] = kt_hip_sscale{a.vs->mant, a.vs->shift, 1};
    }
    __syncthreads();  // the cache row and both scales of this step are visible to the whole CTA past here

    // 2. v_ref and s_ref
    ScIdx bv{Sc{0, 0}, -1}, bs{Sc{0, 0}, -1};
    for (int j = tid; j < steps; j += RD_THREADS) {
        const Sc vj{a.vscale[j].mant, a.vscale[j].shift}, kj{a.kscale[j].mant, a.kscale[j].shift};
        const Sc sj = sc_mul(sc_mul(qs, kj), isq);
        F[j] = sj;
        bv = sc_pick(bv, ScIdx{vj, j});
        bs = sc_pick(bs, ScIdx{sj, j});
    }
    {
        ScIdx two[2] = {bv, bs};
        block_fold_max_k<2>(two, redsc);
        bv = two[0], bs = two[1];
    }
    if (tid == 0) {
        par[0] = bv.s, par[1] = bs.s;
        par[2] = bs.s.mant ? sc_mul(bs.s, Sc{a.exp.inv_mant, a.exp.inv_shift}) : Sc{0, 0};
    }
    __syncthreads();
    const Sc v_ref = par[0], s_ref = par[1], lm = par[2];
    if (v_ref.mant != 0 || s_ref.mant != 0) {
        Sc* inv2 = sh_.inv2;
        if (tid == 0) inv2[0] = v_ref.mant ? sc_recip(v_ref) : Sc{0, 0};  // the two reciprocals in two waves
        if (tid == 64) inv2[1] = s_ref.mant ? sc_recip(s_ref) : Sc{0, 0};
        __syncthreads();
        for (int j = tid; j < steps; j += RD_THREADS) {
            VF[j] = v_ref.mant ? sc_mul(Sc{a.vscale[j].mant, a.vscale[j].shift}, inv2[0]) : Sc{0, 0};
            if (s_ref.mant) F[j] = sc_mul(F[j], inv2[1]);
        }
    } else {
        for (int j = tid; j < steps; j += RD_THREADS) VF[j] = Sc{0, 0};
    }
    __syncthreads();

    // 3. the heads, hb at a time: the scores by one wave per (head, cached row) with the lanes across head_dim, the
    //    integer softmax by one wave per head, P.V by one thread per (head, dim). Sums wrap as i64 (any order gives
    //    the reference's integers).
    const int lane = tid & 63, wave = tid >> 6;
    int64_t* hsum = sh_.hsum;
    for (int h0 = 0; h0 < nh; h0 += hb) {
        const int hn = nh - h0 < hb ? nh - h0 : hb;
        if (s_ref.mant == 0) {  // every head skipped (the reference's `continue`)
            for (int i = tid; i < hn * hd; i += RD_THREADS) HO[h0 * hd + i] = 0;
            if (tid < hn) hsc[h0 + tid] = Sc{0, 0};
            continue;
        }
        const int items = hn * steps;
        // (16-byte loads: rows of a multiple of 32 values, q and the cache at 16-byte aligned addresses)
        const bool vec = hd % 32 == 0 && (((size_t)((const char*)QD - (const char*)lds)) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(a.kc) & 15) == 0;
        if (vec) {
            // one thread per (head, cached row): the whole dot from 16-byte loads, 32 values of k in flight at a time
            for (int it = tid; it < items; it += RD_THREADS) {
                const int h = it / steps, j = it - h * steps, kv = (h0 + h) / group;
                const int4* kr = reinterpret_cast<const int4*>(a.kc + (size_t)j * kstride + kv * hd);
                const int4* qh = reinterpret_cast<const int4*>(QD + (h0 + h) * hd);
                int64_t dot = 0;
                for (int e4 = 0; e4 < hd / 4; e4 += 8) {
                    int4 kk[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) kk[u] = kr[e4 + u];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const int4 qq = qh[e4 + u];
                        dot = wadd(dot, (int64_t)qq.x * kk[u].x + (int64_t)qq.y * kk[u].y);  // each below 2^63
                        dot = wadd(dot, (int64_t)qq.z * kk[u].z + (int64_t)qq.w * kk[u].w);
                    }
                }
                S[(size_t)h * rows + j] = sc_apply(F[j], dot);
            }
        } else {
        // RD_SU items per wave at a time, every cached k row of them loaded before the first product (an item past
        // the end re-reads the last one and is dropped)
        constexpr int RD_SU = 8;
        for (int it0 = wave; it0 < items; it0 += RD_WAVES * RD_SU) {
            int64_t dot[RD_SU];
            int hh[RD_SU], jj[RD_SU];
#pragma unroll
            for (int u = 0; u < RD_SU; u++) {
                const int it = it0 + u * RD_WAVES, itc = it < items ? it : items - 1;
                hh[u] = itc / steps, jj[u] = itc - hh[u] * steps, dot[u] = 0;
            }
            for (int e = lane; e < hd; e += 64) {
                int32_t kk[RD_SU];
#pragma unroll
                for (int u = 0; u < RD_SU; u++)
                    kk[u] = a.kc[(size_t)jj[u] * kstride + ((h0 + hh[u]) / group) * hd + e];
#pragma unroll
                for (int u = 0; u < RD_SU; u++) dot[u] = wadd(dot[u], wmul(QD[(h0 + hh[u]) * hd + e], kk[u]));
            }
#pragma unroll
            for (int u = 0; u < RD_SU; u++) {
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) dot[u] = wadd(dot[u], __shfl_xor(dot[u], o, 64));
            }
            if (lane < RD_SU) {  // lane u stores item u (every lane holds every item's full sum)
                int64_t d = dot[0];
#pragma unroll
                for (int u = 1; u < RD_SU; u++) d = lane == u ? dot[u] : d;
                const int it = it0 + lane * RD_WAVES;
                const int h = it / steps, j = it - h * steps;
                if (it < items) S[(size_t)h * rows + j] = sc_apply(F[j], d);
            }
        }
        }
        __syncthreads();
        for (int h = wave; h < hn; h += RD_WAVES) {
            int64_t* sh = S + (size_t)h * rows;
            int64_t m = INT64_MIN;
            for (int j = lane; j < steps; j += 64) m = sh[j] > m ? sh[j] : m;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const int64_t u = __shfl_xor(m, o, 64);
                m = u > m ? u : m;
            }
            int64_t sum = 0;
            for (int j = lane; j < steps; j += 64) {
                const int64_t idx = lut_index(lm, (int64_t)((uint64_t)sh[j] - (uint64_t)m), a.exp.lo_index);
                sh[j] = idx < 0 ? 0 : lut_code(a.exp_codes, a.exp.n, idx);
                sum += sh[j];
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) sum = wadd(sum, __shfl_xor(sum, o, 64));
            if (lane == 0) {
                hsum[h] = sum;
                hsc[h0 + h] = sum <= 0 ? Sc{0, 0} : sc_mul(v_ref, from_ratio(1, (u128)(uint64_t)sum));
            }
        }
        __syncthreads();
        if (group <= RD_PV_GROUP) {
            // P.V by kv head: v_jd scaled once for the heads that share it (vf_j.apply(v_jd) is the same for every
            // head of a group), each wave one (kv head, slice of the steps) with its lanes across head_dim, the
            // heads' products summed into HO by LDS atomics (wrapping i64 sums: any order gives the same integers)
            for (int i = tid; i < hn * hd; i += RD_THREADS) HO[h0 * hd + i] = 0;
            __syncthreads();
            const int kv0 = h0 / group, nkvb = (h0 + hn - 1) / group - kv0 + 1;
            const int jp = RD_WAVES / nkvb > 1 ? RD_WAVES / nkvb : 1, tasks = nkvb * jp;
            for (int t = wave; t < tasks; t += RD_WAVES) {
                const int kv = kv0 + t / jp, js = t - (t / jp) * jp;
                const int hs = kv * group > h0 ? kv * group : h0;
                const int he = (kv + 1) * group < h0 + hn ? (kv + 1) * group : h0 + hn;  // heads [hs, he)
                for (int dd = lane; dd < hd; dd += 64) {
                    int64_t acc[RD_PV_GROUP];
#pragma unroll
                    for (int g = 0; g < RD_PV_GROUP; g++) acc[g] = 0;
                    const int32_t* vcol = a.vc + kv * hd + dd;
                    constexpr int RD_PU = 4;  // cached v values loaded before their products
                    for (int j0 = js; j0 < steps; j0 += RD_PU * jp) {
                        int32_t vv[RD_PU];
#pragma unroll
                        for (int u = 0; u < RD_PU; u++) {
                            const int j = j0 + u * jp < steps ? j0 + u * jp : steps - 1;
                            vv[u] = vcol[(size_t)j * kstride];
                        }
#pragma unroll
                        for (int u = 0; u < RD_PU; u++) {
                            const int j = j0 + u * jp;
                            if (j >= steps) break;
                            const int64_t sv = sc_apply32(VF[j], vv[u]);
#pragma unroll
                            for (int g = 0; g < RD_PV_GROUP; g++)
                                if (hs + g < he) acc[g] = wadd(acc[g], wmul(S[(size_t)(hs + g - h0) * rows + j], sv));
                        }
                    }
#pragma unroll
                    for (int g = 0; g < RD_PV_GROUP; g++)
                        if (hs + g < he && acc[g] != 0)
                            atomicAdd(reinterpret_cast<unsigned long long*>(&HO[(hs + g) * hd + dd]),
                                      (unsigned long long)acc[g]);
                }
            }
            __syncthreads();
            for (int i = tid; i < hn * hd; i += RD_THREADS)  // a head with no numerators: zeros
                if (hsum[i / hd] <= 0) HO[h0 * hd + i] = 0;
        } else {
            for (int it = tid; it < hn * hd; it += RD_THREADS) {
                const int h = it / hd, dd = it - h * hd, kv = (h0 + h) / group;
                int64_t acc = 0;
                if (hsum[h] > 0) {
                    const int64_t* sh = S + (size_t)h * rows;
                    const int32_t* vcol = a.vc + kv * hd + dd;
                    // RD_PU cached v values loaded before their products (a step past the end re-reads the last one
                    // and is dropped)
                    constexpr int RD_PU = 8;
                    for (int j0 = 0; j0 < steps; j0 += RD_PU) {
                        int32_t vv[RD_PU];
#pragma unroll
                        for (int u = 0; u < RD_PU; u++) {
                            const int j = j0 + u < steps ? j0 + u : steps - 1;
                            vv[u] = vcol[(size_t)j * kstride];
                        }
#pragma unroll
                        for (int u = 0; u < RD_PU; u++)
                            if (j0 + u < steps) acc = wadd(acc, wmul(sh[j0 + u], sc_apply32(VF[j0 + u], vv[u])));
                    }
                }
                HO[(h0 + h) * hd + dd] = acc;
            }
        }
        __syncthreads();  // S and hsum are reused by the next batch
    }

    // 4. one scale for the concatenated heads: the heads' largest by the engine's fold, then every thread its own
    //    reciprocal and its elements' head factors (no serial step)
    const Sc common = block_fold_max(tid < nh ? ScIdx{hsc[tid], tid} : ScIdx{Sc{0, 0}, -1}, redsc, nh).s;
    int64_t m = 0;
    if (common.mant != 0) {
        const Sc cinv = sc_recip(common);
        for (int i = tid; i < qstride; i += RD_THREADS) {
            HO[i] = sc_apply(sc_mul(hsc[i / hd], cinv), HO[i]);
            m = iabs(HO[i]) > m ? iabs(HO[i]) : m;
        }
    }
    const int64_t gmax = block_max_i64(m, red);
    const RqDen rd_gmax = rq_den(gmax);
    for (int i = tid; i < qstride; i += RD_THREADS) a.o[i] = gmax == 0 ? 0 : rq_apply(rd_gmax, HO[i]);
    if (tid == 0)
        put_rec(a.os, gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), common));
}

// One CTA for every head: hb heads' scores at a time in LDS (a.hb >= 1).
__global__ __launch_bounds__(RD_THREADS) void rd_attention_step_kernel(RdAttn a) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ RdAttnShared sh_;
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) {  // outside the tables: zeros (the reference asserts here)
        for (int i = threadIdx.x; i < a.nh * a.hd; i += RD_THREADS) a.o[i] = 0;
        if (threadIdx.x == 0) put_rec(a.os, Sc{0, 0});
        return;
    }
    rd_attention_core(a, lds, sh_, pos, a.hb);
}

// Attention::decode_step between its projections with L.parts CTAs per q head, for caches of any length up to
// max_seq (kt_hip_ref_attention_step_ws): the cache reads, the per-step Scale work and P.V spread over nh * parts CUs
// instead of one. rd_attention_heads_kernel (CTA h * parts + part): RoPE of q_h and of this step's k (part 0 of the
// first head of each kv group appends the step's k and v rows to the cache, part 0 of head 0 the step's scales; row
// pos is taken from the inputs by every CTA, so no CTA reads what another writes in the same launch); every step's
// score factor f_j = s_j / s_ref and v factor vf_j = vs_j / v_ref, its head's scores, maximum and integer softmax
// numerators (the same integers in every CTA of the head); P.V over its share of the steps (P.V's 64-bit products
// are the step's largest cost, so they are what the parts divide); its part of the head's sums, and (part 0) the
// head's scale v_ref / sumc, into the workspace. rd_attention_combine_kernel (one CTA, the next launch): each head's
// parts added (wrapping, exact in any order), the heads at their largest scale, requantized -- step 4 of the one-CTA
// kernel.
struct RdHeadsLayout {
    size_t ho, hsc, arr, arr_stride;  // byte offsets: head output parts, head scales, per-CTA step arrays (and stride)
    int parts;                        // CTAs per head: each sums P.V over its share of the steps
};
__host__ __device__ inline size_t rd_round256(size_t v) { return (v + 255) / 256 * 256; }
__host__ __device__ inline RdHeadsLayout rd_heads_layout(int max_seq, int nh, int hd) {
    RdHeadsLayout L;
    L.parts = 128 / nh < 1 ? 1 : (128 / nh > 8 ? 8 : 128 / nh);  // 8 CTAs per head at the Qwen shape (112 CTAs)
    L.ho = 0;
    L.hsc = rd_round256((size_t)nh * L.parts * hd * sizeof(int64_t));
    L.arr = L.hsc + rd_round256((size_t)nh * sizeof(Sc));
    L.arr_stride = rd_round256((size_t)max_seq * (2 * sizeof(Sc) + sizeof(int64_t)));
    return L;
}

// cached v values (and their steps' numerators and factors) loaded before the products; RD_PV_W: the v values a lane
// of the wave-uniform P.V path has in flight
constexpr int RD_PV_U = 8, RD_PV_W = 16;
// The heads kernel's dynamic LDS when its per-step arrays stay in LDS (max_seq up to about 2,400 at head_dim 64; the
// static part is about 33 KB).
constexpr size_t RD_HEADS_LDS = 96 * 1024;

// GA: the per-step arrays in the workspace (caches longer than LDS holds), else in LDS after q and k. SUMS: q, k and v
// are the q / k / v product's sums (a.qsum, a.ksum, a.vsum): every CTA takes their maxima over the whole outputs,
// forms their Scales and the codes it reads as ql_requant_kernel would (CTA 0 writes the records).
template <bool GA, bool SUMS>
__global__ __launch_bounds__(RD_THREADS) void rd_attention_heads_kernel(RdAttn a, RdHeadsLayout L) {
    __shared__ int64_t red[3 * RD_WAVES];
    __shared__ Sc qkv_s[3];
    __shared__ ScIdx redsc[RD_THREADS];
    __shared__ Sc par[4];  // v_ref, s_ref, lut factor, 1 / v_ref
    __shared__ Sc sinv_s;
    __shared__ int64_t PV[RD_THREADS];
    extern __shared__ __align__(16) int32_t qk[];  // the rotated q_h (hd), then this step's rotated k (hd)
    const int P = L.parts, h = (int)blockIdx.x / P, part = (int)blockIdx.x % P;
    const int tid = threadIdx.x, hd = a.hd, half = hd / 2, nh = a.nh, nkv = a.nkv;
    const int group = nh / nkv, kv = h / group, kstride = nkv * hd;
    const int pos = *a.pos;
    // q, k and v: codes and Scales from the inputs, or requant_dyn of the sums
    int64_t ymax[3] = {0, 0, 0};
    if constexpr (SUMS) {
        for (int i = tid; i < nh * hd; i += RD_THREADS) ymax[0] = iabs(a.qsum.acc[i]) > ymax[0] ? iabs(a.qsum.acc[i]) : ymax[0];
        for (int i = tid; i < nkv * hd; i += RD_THREADS) {
            ymax[1] = iabs(a.ksum.acc[i]) > ymax[1] ? iabs(a.ksum.acc[i]) : ymax[1];
            ymax[2] = iabs(a.vsum.acc[i]) > ymax[2] ? iabs(a.vsum.acc[i]) : ymax[2];
        }
        block_max_k<3>(ymax, red);
        if ((tid & 63) == 0 && tid < 192) {  // the three Scale chains in three waves
            const RqSums& r = tid == 0 ? a.qsum : (tid == 64 ? a.ksum : a.vsum);
            const int64_t ym = ymax[tid >> 6];
            const Sc sc = rqs_scale(r.st, ym);
            qkv_s[tid >> 6] = sc;
            if (blockIdx.x == 0) rqs_record(r, ym, sc);
        }
        __syncthreads();
    }
    const bool lq = SUMS && rqs_live(a.qsum.st, ymax[0]), lk = SUMS && rqs_live(a.ksum.st, ymax[1]),
               lv = SUMS && rqs_live(a.vsum.st, ymax[2]);
    const RqDen dq = rq_den(ymax[0]), dk = rq_den(ymax[1]), dv = rq_den(ymax[2]);
    auto qcode = [&](int i) -> int32_t {
        if constexpr (SUMS) return lq ? rq_apply(dq, a.qsum.acc[i]) : 0;
        else return a.q[i];
    };
    auto kcode = [&](int i) -> int32_t {
        if constexpr (SUMS) return lk ? rq_apply(dk, a.ksum.acc[i]) : 0;
        else return a.k[i];
    };
    auto vcode = [&](int i) -> int32_t {
        if constexpr (SUMS) return lv ? rq_apply(dv, a.vsum.acc[i]) : 0;
        else return a.v[i];
    };
    const Sc qs = SUMS ? qkv_s[0] : rec_sc(a.qs), ksp = SUMS ? qkv_s[1] : rec_sc(a.ks),
             vsp = SUMS ? qkv_s[2] : rec_sc(a.vs);
    unsigned char* ws = a.ws;
    int64_t* HO = reinterpret_cast<int64_t*>(ws + L.ho);
    Sc* HSC = reinterpret_cast<Sc*>(ws + L.hsc);
    if (pos < 0 || pos >= a.max_seq) {  // outside the tables: the combine writes zeros
        for (int d = tid; d < hd; d += RD_THREADS) HO[((size_t)h * P + part) * hd + d] = 0;
        if (tid == 0 && part == 0) HSC[h] = Sc{0, 0};
        return;
    }
    const int steps = pos + 1;
    int32_t* QD = qk;
    int32_t* KP = qk + hd;
    unsigned char* arr = GA ? ws + L.arr + ((size_t)h * P + part) * L.arr_stride
                            : reinterpret_cast<unsigned char*>(qk) + (size_t)rd_round256(2 * (size_t)hd * 4);
    Sc* F = reinterpret_cast<Sc*>(arr);                        // score factors, per step
    Sc* VF = F + a.max_seq;                                    // v factors, per step
    int64_t* S = reinterpret_cast<int64_t*>(VF + a.max_seq);   // scores, then exp codes

    // 1. RoPE (attention.rs:222-246) of q_h and of this step's k of kv head `kv`; the cache append
    for (int j = tid; j < half; j += RD_THREADS) {
        const kt_hip_sscale c = a.cos[(size_t)pos * half + j], sn = a.sin[(size_t)pos * half + j];
        const Sc cm{c.mant, c.shift}, sm{sn.mant, sn.shift};
        const int32_t qa = qcode(h * hd + j), qb = qcode(h * hd + j + half);
        QD[j] = (int32_t)(c.sign * sc_apply32(cm, qa) - sn.sign * sc_apply32(sm, qb));
        QD[j + half] = (int32_t)(c.sign * sc_apply32(cm, qb) + sn.sign * sc_apply32(sm, qa));
        const int32_t ka = kcode(kv * hd + j), kb = kcode(kv * hd + j + half);
        KP[j] = (int32_t)(c.sign * sc_apply32(cm, ka) - sn.sign * sc_apply32(sm, kb));
        KP[j + half] = (int32_t)(c.sign * sc_apply32(cm, kb) + sn.sign * sc_apply32(sm, ka));
    }
    __syncthreads();
    if (h == kv * group && part == 0)
        for (int i = tid; i < hd; i += RD_THREADS) {
            a.kc[(size_t)pos * kstride + kv * hd + i] = KP[i];
            a.vc[(size_t)pos * kstride + kv * hd + i] = vcode(kv * hd + i);
        }
    if (h == 0 && part == 0 && tid == 0) {
        a.kscale[pos] = kt_hip_sscale{ksp.mant, ksp.shift, 1};
        a.vscale[pos] = kt_hip_sscale{vsp.mant, vsp.shift, 1};
    }

    // 2. every step's score scale s_j = qs * ks_j * inv_sqrt and v scale; their largest (the engine's fold)
    const Sc isq{a.isq_mant, a.isq_shift};
    ScIdx bv{Sc{0, 0}, -1}, bs{Sc{0, 0}, -1};
    for (int j = tid; j < steps; j += RD_THREADS) {
        const Sc kj = j == pos ? ksp : Sc{a.kscale[j].mant, a.kscale[j].shift};
        const Sc vj = j == pos ? vsp : Sc{a.vscale[j].mant, a.vscale[j].shift};
        const Sc sj = sc_mul(sc_mul(qs, kj), isq);
        F[j] = sj;
        VF[j] = vj;
        bv = sc_pick(bv, ScIdx{vj, j});
        bs = sc_pick(bs, ScIdx{sj, j});
    }
    {
        ScIdx two[2] = {bv, bs};
        block_fold_max_k<2>(two, redsc);
        bv = two[0], bs = two[1];
    }
    if (tid == 0) {
        par[0] = bv.s, par[1] = bs.s;
        par[2] = bs.s.mant ? sc_mul(bs.s, Sc{a.exp.inv_mant, a.exp.inv_shift}) : Sc{0, 0};
        par[3] = bv.s.mant ? sc_recip(bv.s) : Sc{0, 0};  // the two reciprocals in two waves
    }
    if (tid == 64) sinv_s = bs.s.mant ? sc_recip(bs.s) : Sc{0, 0};
    __syncthreads();
    const Sc v_ref = par[0], s_ref = par[1], lm = par[2], vinv = par[3], sinv = sinv_s;
    if (s_ref.mant == 0) {  // the head is skipped (the reference's `continue`): zeros at Scale::ZERO
        for (int d = tid; d < hd; d += RD_THREADS) HO[((size_t)h * P + part) * hd + d] = 0;
        if (tid == 0 && part == 0) HSC[h] = Sc{0, 0};
        return;
    }

    // 3. scores: one thread per cached step, the whole dot (16-byte loads of the cache row where it allows)
    const bool vec = hd % 4 == 0 && (reinterpret_cast<uintptr_t>(a.kc) & 15) == 0 && ((size_t)kstride * 4) % 16 == 0;
    int64_t m = INT64_MIN;
    for (int j = tid; j < steps; j += RD_THREADS) {
        VF[j] = v_ref.mant ? sc_mul(VF[j], vinv) : Sc{0, 0};
        int64_t dot = 0;
        if (j == pos) {
            for (int d = 0; d < hd; d++) dot = wadd(dot, (int64_t)QD[d] * KP[d]);
        } else if (vec) {
            // 8 x 16 bytes of the cache row in flight at a time (16 spill registers)
            const int4* kr = reinterpret_cast<const int4*>(a.kc + (size_t)j * kstride + kv * hd);
            for (int e4 = 0; e4 < hd / 4; e4 += 8) {
                int4 kk[8];
#pragma unroll
                for (int u = 0; u < 8; u++) kk[u] = e4 + u < hd / 4 ? kr[e4 + u] : int4{0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (e4 + u >= hd / 4) break;
                    const int d = 4 * (e4 + u);
                    dot = wadd(dot, (int64_t)QD[d] * kk[u].x + (int64_t)QD[d + 1] * kk[u].y);  // each below 2^63
                    dot = wadd(dot, (int64_t)QD[d + 2] * kk[u].z + (int64_t)QD[d + 3] * kk[u].w);
                }
            }
        } else {
            const int32_t* kr = a.kc + (size_t)j * kstride + kv * hd;
            for (int d = 0; d < hd; d++) dot = wadd(dot, (int64_t)QD[d] * kr[d]);
        }
        const int64_t sc = sc_apply(sc_mul(F[j], sinv), dot);
        S[j] = sc;
        m = sc > m ? sc : m;
    }
    const int64_t dmax = block_max_i64(m, red);

    // 4. the integer-code softmax numerators and their sum
    int64_t sum = 0;
    for (int j = tid; j < steps; j += RD_THREADS) {
        const int64_t idx = lut_index(lm, (int64_t)((uint64_t)S[j] - (uint64_t)dmax), a.exp.lo_index);
        const int64_t ec = idx < 0 ? 0 : lut_code(a.exp_codes, a.exp.n, idx);
        S[j] = ec;
        sum += ec;
    }
    sum = (int64_t)wave_sum_u64((uint64_t)sum);
    if ((tid & 63) == 0) red[tid >> 6] = sum;
    __syncthreads();
    const int64_t sumc = (int64_t)lane64(row_sum_u64((tid & 63) < RD_WAVES ? (uint64_t)red[tid & 63] : 0), 0);
    if (sumc <= 0) {
        for (int d = tid; d < hd; d += RD_THREADS) HO[((size_t)h * P + part) * hd + d] = 0;
        if (tid == 0 && part == 0) HSC[h] = Sc{0, 0};
        return;
    }

    // 5. P.V: thread js * hd + d (hd <= RD_THREADS) sums the steps j = js (mod slices) of column d (wrapping i64:
    //    any order gives the reference's integers); the slices then add up in LDS
    const int slices = RD_THREADS / hd, d = tid % hd, js = tid / hd;
    const int32_t vpos = vcode(kv * hd + d);  // this step's v (its cache row is written in this same launch)
    int64_t acc = 0;
    if (hd % 64 == 0) {
        // a wave is one slice: its step, numerator and v factor are the same on every lane, so they are read once
        // into scalar registers and Scale::apply's branches and shift amounts are scalar
        // The cached v rows come from HBM (the weight streams evicted them since the previous token): RD_PV_W of
        // them in flight per lane at a time, so that a few dependent round trips, not one per RD_PV_U steps, pay
        // for the whole column.
        // slice jw of this CTA's share: the steps j = part * slices + jw (mod P * slices)
        const int jw = __builtin_amdgcn_readfirstlane(js), ST = P * slices;
        if (jw < slices) {
            const int32_t* vcol = a.vc + kv * hd + d;
            for (int j0 = part * slices + jw; j0 < steps; j0 += RD_PV_W * ST) {
                int32_t vv[RD_PV_W];
#pragma unroll
                for (int u = 0; u < RD_PV_W; u++) {  // a step past the end reads the last one and adds nothing
                    const int j = j0 + u * ST < steps ? j0 + u * ST : steps - 1;
                    vv[u] = j == pos ? vpos : vcol[(size_t)j * kstride];
                }
#pragma unroll
                for (int u = 0; u < RD_PV_W; u++) {
                    const int j = j0 + u * ST;
                    if (j < steps) {  // uniform
                        const int64_t e = S[j];
                        const Sc f = VF[j];
                        const int64_t ec = ((int64_t)__builtin_amdgcn_readfirstlane((int)((uint64_t)e >> 32)) << 32) |
                                           (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)e);
                        Sc vf;
                        vf.mant = ((int64_t)__builtin_amdgcn_readfirstlane((int)((uint64_t)f.mant >> 32)) << 32) |
                                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)f.mant);
                        vf.shift = __builtin_amdgcn_readfirstlane(f.shift);
                        acc = wadd(acc, wmul(ec, sc_apply32(vf, vv[u])));
                    }
                }
            }
        }
    } else if (js < slices) {
        const int ST = P * slices;
        const int32_t* vcol = a.vc + kv * hd + d;
        for (int j0 = part * slices + js; j0 < steps; j0 += RD_PV_U * ST) {
            int32_t vv[RD_PV_U];
            int64_t ec[RD_PV_U];
            Sc vf[RD_PV_U];
#pragma unroll
            for (int u = 0; u < RD_PV_U; u++) {  // a step past the end reads the last one and adds nothing
                const int j = j0 + u * ST < steps ? j0 + u * ST : steps - 1;
                vv[u] = j == pos ? vpos : vcol[(size_t)j * kstride];
                ec[u] = S[j];
                vf[u] = VF[j];
            }
#pragma unroll
            for (int u = 0; u < RD_PV_U; u++)
                if (j0 + u * ST < steps) acc = wadd(acc, wmul(ec[u], sc_apply32(vf[u], vv[u])));
        }
    }
    PV[tid] = acc;
    __syncthreads();
    for (int dd = tid; dd < hd; dd += RD_THREADS) {  // this CTA's part of the head's sums (the combine adds the parts)
        int64_t t = 0;
        for (int q = 0; q < slices; q++) t = wadd(t, PV[q * hd + dd]);
        HO[((size_t)h * P + part) * hd + dd] = t;
    }
    if (tid == 0 && part == 0) HSC[h] = sc_mul(v_ref, from_ratio(1, (u128)(uint64_t)sumc));
}

// Step 4 of Attention::decode_step over the heads kernel's outputs: the heads' largest scale by the engine's fold,
// each head brought to it, requant_dyn of the concatenation, the record.
constexpr int RD_CB = 2;  // head-output values a combine thread holds (nh * hd up to 2048); longer rows recompute
__global__ __launch_bounds__(RD_THREADS) void rd_attention_combine_kernel(RdAttn a, RdHeadsLayout L) {
    __shared__ int64_t red[RD_WAVES];
    __shared__ ScIdx redsc[RD_THREADS];
    const int tid = threadIdx.x, hd = a.hd, nh = a.nh, qstride = nh * hd, P = L.parts;
    const int64_t* HOP = reinterpret_cast<const int64_t*>(a.ws + L.ho);
    const Sc* HSC = reinterpret_cast<const Sc*>(a.ws + L.hsc);
    // each head's sums: its CTAs' parts (at most 8) added, wrapping, in any order (the reference's integers); the
    // parts' loads all issued before the adds
    auto ho = [&](int i) {
        const int hh = i / hd, dd = i - hh * hd;
        const int64_t* p = HOP + (size_t)hh * P * hd + dd;
        int64_t t[8];
#pragma unroll
        for (int q = 0; q < 8; q++) t[q] = q < P ? p[(size_t)q * hd] : 0;
        int64_t s = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) s = wadd(s, t[q]);
        return s;
    };
    // the sums of the values a thread holds are read before the heads' fold, so the two overlap
    const bool held = qstride <= RD_THREADS * RD_CB;
    int64_t hv[RD_CB];
#pragma unroll
    for (int k = 0; k < RD_CB; k++) {
        const int i = tid + RD_THREADS * k;
        hv[k] = held && i < qstride ? ho(i) : 0;
    }
    const Sc common = block_fold_max(tid < nh ? ScIdx{HSC[tid], tid} : ScIdx{Sc{0, 0}, -1}, redsc, nh).s;
    int64_t m = 0;
    if (common.mant != 0) {
        const Sc cinv = sc_recip(common);
        if (held) {
#pragma unroll
            for (int k = 0; k < RD_CB; k++) {  // each value at the common scale, kept for the requant
                const int i = tid + RD_THREADS * k;
                if (i < qstride) hv[k] = sc_apply(sc_mul(HSC[i / hd], cinv), hv[k]);
                m = iabs(hv[k]) > m ? iabs(hv[k]) : m;
            }
        } else {
            for (int i = tid; i < qstride; i += RD_THREADS) {
                const int64_t v = sc_apply(sc_mul(HSC[i / hd], cinv), ho(i));
                m = iabs(v) > m ? iabs(v) : m;
            }
        }
    }
    const int64_t gmax = block_max_i64(m, red);
    const RqDen rd_gmax = rq_den(gmax);
    if (gmax == 0) {
        for (int i = tid; i < qstride; i += RD_THREADS) a.o[i] = 0;
    } else if (held) {
#pragma unroll
        for (int k = 0; k < RD_CB; k++) {
            const int i = tid + RD_THREADS * k;
            if (i < qstride) a.o[i] = rq_apply(rd_gmax, hv[k]);
        }
    } else {
        const Sc cinv = sc_recip(common);
        for (int i = tid; i < qstride; i += RD_THREADS) a.o[i] = rq_apply(rd_gmax, sc_apply(sc_mul(HSC[i / hd], cinv), ho(i)));
    }
    if (tid == 0)
        put_rec(a.os, gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), common));
}

// The same ops over whole-sequence tensors on many CTAs (the batched forward's T-row tensors): one CTA forms the
// tensor's Scales (and an RMSNorm's row factors) into the workspace and zeroes its max slot, a grid pass takes the
// largest magnitude, a grid pass requantizes and writes the record. Integers identical to the one-CTA kernels.
struct RdSeqWs {
    Sc par[4];      // add: common, fa, fb; SwiGLU: index factor, identity factor, h scale; RMSNorm: cc
    uint64_t gmax;  // the largest magnitude
    Sc frow[1];     // RMSNorm: each row's factor over cc (rows of them)
};
enum { RS_ADD = 0, RS_SWIGLU = 1, RS_NORM = 2 };
struct RdSeq {
    int op;
    const int32_t *a, *b;  // add: a, b; SwiGLU: g, u; RMSNorm: x, gamma
    const kt_hip_qscale *as, *bs;
    int64_t n;             // values (rows * dim for RMSNorm)
    int rows, dim;
    int64_t g_mant, e_mant;
    int32_t g_shift, e_shift;
    const int64_t* codes;
    kt_hip_codelut lut;
    RdSeqWs* ws;
    int32_t* y;
    kt_hip_qscale* ys;
};

__device__ inline int64_t rs_value(const RdSeq& q, const RdSeqWs* w, int64_t i) {
    if (q.op == RS_ADD) return wadd(sc_apply32(w->par[1], q.a[i]), sc_apply32(w->par[2], q.b[i]));
    if (q.op == RS_SWIGLU) {
        const int32_t gd = q.a[i];
        const int64_t idx = lut_index32(w->par[0], gd, q.lut.lo_index);
        const int64_t code = idx < 0 ? 0 : (idx >= q.lut.n ? sc_apply32(w->par[1], gd) : lut_code(q.codes, q.lut.n, idx));
        return wmul(code, q.b[i]);
    }
    return sc_apply(w->frow[i / q.dim], (int64_t)q.a[i] * (int64_t)q.b[i % q.dim]);
}
// whether the values are live (a zero common scale gives zeros)
__device__ inline bool rs_live(const RdSeq& q, const RdSeqWs* w) { return q.op == RS_SWIGLU || w->par[0].mant != 0; }

__global__ __launch_bounds__(RD_THREADS) void rs_prep_kernel(RdSeq q) {
    __shared__ ScIdx redsc[RD_THREADS];
    RdSeqWs* w = q.ws;
    if (q.op == RS_NORM) {  // as rd_rmsnorm_kernel, the row factors in the workspace
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const Sc xs = rec_sc(q.as), gs{q.g_mant, q.g_shift}, eps{q.e_mant, q.e_shift};
        for (int r = wave; r < q.rows; r += RD_WAVES) {
            uint64_t hi = 0, lo = 0;
            for (int i = lane; i < q.dim; i += 64) {
                const int64_t v = q.a[(size_t)r * q.dim + i];
                const uint64_t sq = (uint64_t)(v * v), t = lo + sq;
                hi += t < lo, lo = t;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const uint64_t ohi = __shfl_xor(hi, o, 64), olo = __shfl_xor(lo, o, 64), t = lo + olo;
                hi += ohi + (t < lo), lo = t;
            }
            if (lane == 0) {
                const Sc mean_sq = sc_mul(sc_mul(from_ratio(((u128)hi << 64) | lo, (u128)q.dim), xs), xs);
                const Sc denom = sc_add(mean_sq, eps);
                w->frow[r] = sc_mul(sc_mul(xs, denom.mant == 0 ? Sc{0, 0} : sc_rsqrt(denom)), gs);
            }
        }
        __syncthreads();  // the CTA's own global writes are visible to it past the barrier
        ScIdx best{Sc{0, 0}, -1};
        for (int r = threadIdx.x; r < q.rows; r += RD_THREADS) best = sc_pick(best, ScIdx{w->frow[r], r});
        const Sc cc = block_fold_max(best, redsc, q.rows).s;
        if (cc.mant != 0) {
            const Sc cinv = sc_recip(cc);
            for (int r = threadIdx.x; r < q.rows; r += RD_THREADS) w->frow[r] = sc_mul(w->frow[r], cinv);
        }
        if (threadIdx.x == 0) w->par[0] = cc, w->gmax = 0;
        return;
    }
    if (threadIdx.x == 0) {
        const Sc as = rec_sc(q.as), bs = rec_sc(q.bs);
        if (q.op == RS_ADD) {
            const Sc common = sc_ge(as, bs) ? as : bs;
            w->par[0] = common, w->par[1] = w->par[2] = Sc{0, 0};
            if (common.mant != 0) {
                const Sc cinv = sc_recip(common);
                w->par[1] = sc_mul(as, cinv), w->par[2] = sc_mul(bs, cinv);
            }
        } else {  // SwiGLU: as is g's record, bs u's
            const Sc cs{q.lut.code_mant, q.lut.code_shift};
            w->par[0] = sc_mul(as, Sc{q.lut.inv_mant, q.lut.inv_shift});
            w->par[1] = sc_mul(as, sc_recip(cs));
            w->par[2] = sc_mul(cs, bs);
        }
        w->gmax = 0;
    }
}

__global__ __launch_bounds__(256) void rs_max_kernel(RdSeq q) {
    __shared__ int64_t red[4];
    const RdSeqWs* w = q.ws;
    int64_t m = 0;
    if (rs_live(q, w))
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < q.n; i += (int64_t)gridDim.x * 256) {
            const int64_t v = iabs(rs_value(q, w, i));
            m = v > m ? v : m;
        }
    m = block_max_4w(m, red);
    if (threadIdx.x == 0 && m > 0) atomicMax(reinterpret_cast<unsigned long long*>(&q.ws->gmax), (unsigned long long)m);
}

__global__ __launch_bounds__(256) void rs_out_kernel(RdSeq q) {
    const RdSeqWs* w = q.ws;
    const int64_t gmax = (int64_t)w->gmax;
    const RqDen rd_gmax = rq_den(gmax);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < q.n; i += (int64_t)gridDim.x * 256)
        q.y[i] = gmax == 0 ? 0 : rq_apply(rd_gmax, rs_value(q, w, i));
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const Sc sc = q.op == RS_SWIGLU ? w->par[2] : w->par[0];  // the tensor's scale before the requant
        put_rec(q.ys, gmax == 0 ? Sc{0, 0} : sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), sc));
    }
}

// Embedding::lookup_seq (layers.rs:1138-1145): the code rows of T tokens at the table's scale (a token outside the
// vocabulary gives a zero row; the reference panics there).
__global__ __launch_bounds__(256) void rd_embed_seq_kernel(const int32_t* __restrict__ emb, int64_t e_mant,
                                                           int32_t e_shift, const int32_t* __restrict__ tokens,
                                                           int T, int vocab, int dim, int32_t* __restrict__ y,
                                                           kt_hip_qscale* __restrict__ ys) {
    const int64_t n = (int64_t)T * dim;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int t = tokens[i / dim];
        y[i] = t >= 0 && t < vocab ? emb[(int64_t)t * dim + i % dim] : 0;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) put_rec(ys, Sc{e_mant, e_shift});
}

// Attention::forward_int (attention.rs:467-598) in five launches:
//  rp_rope    q and k of row i rotated at position i (rope_int, attention.rs:208-229)
//  rp_head    one CTA per (head, row i): the causal dots j <= i (exact, wrapping i64) at the one score scale
//             q.scale * k.scale * inv_sqrt, the exp-CodeLut numerators of (dot - max), their sum, the sums of
//             numerator * v over the rows
//  rp_common  one CTA: each (row, head)'s scale v.scale / sumc, the largest by the engine's fold over the
//             [row][head] order, every scale over it
//  rp_apply   the outputs brought to the common scale, their largest magnitude
//  rp_out     requant_dyn, and the output's scale
__global__ __launch_bounds__(256) void rp_rope_kernel(RdPrefill a) {
    const int i = blockIdx.x, half = a.hd / 2, qw = a.nh * a.hd, kw = a.nkv * a.hd;
    for (int e = threadIdx.x; e < (a.nh + a.nkv) * half; e += 256) {
        const bool isk = e >= a.nh * half;
        const int hh = (isk ? e - a.nh * half : e) / half, j = (isk ? e - a.nh * half : e) % half;
        const int32_t* src = isk ? a.k + (size_t)i * kw : a.q + (size_t)i * qw;
        int32_t* dst = isk ? a.kd + (size_t)i * kw : a.qd + (size_t)i * qw;
        const kt_hip_sscale c = a.cos[(size_t)i * half + j], sn = a.sin[(size_t)i * half + j];
        const int32_t av = src[hh * a.hd + j], bv = src[hh * a.hd + j + half];
        const Sc cm{c.mant, c.shift}, sm{sn.mant, sn.shift};
        dst[hh * a.hd + j] = (int32_t)(c.sign * sc_apply32(cm, av) - sn.sign * sc_apply32(sm, bv));
        dst[hh * a.hd + j + half] = (int32_t)(c.sign * sc_apply32(cm, bv) + sn.sign * sc_apply32(sm, av));
    }
}

__global__ __launch_bounds__(256) void rp_head_kernel(RdPrefill a) {
    extern __shared__ int64_t S[];  // T: the dots, then the numerators
    __shared__ int64_t red[4];
    __shared__ int64_t part[256];
    __shared__ int32_t qrow[256];
    __shared__ Sc lm_s;
    const int h = blockIdx.x / a.T, i = blockIdx.x % a.T, hd = a.hd, kv = h / (a.nh / a.nkv);
    const int kw = a.nkv * a.hd, tid = threadIdx.x;
    for (int d = tid; d < hd; d += 256) qrow[d] = a.qd[(size_t)i * a.nh * hd + h * hd + d];
    if (tid == 0) {
        const Sc s_score = sc_mul(sc_mul(rec_sc(a.qs), rec_sc(a.ks)), Sc{a.isq_mant, a.isq_shift});
        lm_s = sc_mul(s_score, Sc{a.exp.inv_mant, a.exp.inv_shift});
    }
    __syncthreads();
    int64_t m = INT64_MIN;
    for (int j = tid; j <= i; j += 256) {
        const int32_t* kr = a.kd + (size_t)j * kw + kv * hd;
        int64_t dot = 0;
        for (int d = 0; d < hd; d++) dot = wadd(dot, wmul(qrow[d], kr[d]));
        S[j] = dot;
        m = dot > m ? dot : m;
    }
    const int64_t dmax = block_max_4w(m, red);
    const Sc lm = lm_s;
    int64_t sum = 0;
    for (int j = tid; j <= i; j += 256) {
        const int64_t idx = lut_index(lm, (int64_t)((uint64_t)S[j] - (uint64_t)dmax), a.exp.lo_index);
        S[j] = idx < 0 ? 0 : lut_code(a.exp_codes, a.exp.n, idx);
        sum += S[j];
    }
    const int64_t sumc = block_sum_4w(sum, red);  // also orders the numerator writes before the reads below
    const int groups = 256 / hd, gq = tid / hd, d = tid - gq * hd;
    int64_t acc = 0;
    if (sumc > 0 && gq < groups)
        for (int j = gq; j <= i; j += groups) acc = wadd(acc, wmul(S[j], a.v[(size_t)j * kw + kv * hd + d]));
    part[tid] = acc;
    __syncthreads();
    if (tid < hd) {
        int64_t t = 0;
        for (int q = 0; q < groups; q++) t = wadd(t, part[q * hd + tid]);
        a.hout[((size_t)h * a.T + i) * hd + tid] = sumc > 0 ? t : 0;
    }
    if (tid == 0) a.hsum[(size_t)h * a.T + i] = sumc > 0 ? sumc : 0;
}

__global__ __launch_bounds__(RD_THREADS) void rp_common_kernel(RdPrefill a) {
    __shared__ ScIdx redsc[RD_THREADS];
    const int n = a.T * a.nh;
    const Sc vs = rec_sc(a.vs);
    ScIdx best{Sc{0, 0}, -1};
    for (int e = threadIdx.x; e < n; e += RD_THREADS) {
        const int i = e / a.nh, h = e - i * a.nh;
        const int64_t sumc = a.hsum[(size_t)h * a.T + i];
        const Sc sc = sumc > 0 ? sc_mul(vs, from_ratio(1, (u128)(uint64_t)sumc)) : Sc{0, 0};
        a.fac[e] = sc;
        best = sc_pick(best, ScIdx{sc, e});
    }
    const Sc common = block_fold_max(best, redsc, n).s;  // its barriers order the fac writes before the reads
    if (common.mant != 0) {
        const Sc cinv = sc_recip(common);
        for (int e = threadIdx.x; e < n; e += RD_THREADS) a.fac[e] = sc_mul(a.fac[e], cinv);
    }
    if (threadIdx.x == 0) *a.common = common, *a.gmax = 0;
}

__global__ __launch_bounds__(256) void rp_apply_kernel(RdPrefill a) {
    __shared__ int64_t red[4];
    const int64_t n = (int64_t)a.T * a.nh * a.hd;
    const bool live = a.common->mant != 0;
    int64_t m = 0;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; live && e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t hi = e / a.hd, h = hi / a.T, i = hi - h * a.T;  // e indexes hout[h][i][d]
        const int64_t v = sc_apply(a.fac[i * a.nh + h], a.hout[e]);
        a.hout[e] = v;
        m = iabs(v) > m ? iabs(v) : m;
    }
    m = block_max_4w(m, red);
    if (threadIdx.x == 0 && m > 0) atomicMax(reinterpret_cast<unsigned long long*>(a.gmax), (unsigned long long)m);
}

__global__ __launch_bounds__(256) void rp_out_kernel(RdPrefill a) {
    const int64_t gmax = (int64_t)*a.gmax;
    const RqDen rd_gmax = rq_den(gmax);
    const Sc common = *a.common;
    const bool live = common.mant != 0 && gmax > 0;
    const int qw = a.nh * a.hd;
    const int64_t n = (int64_t)a.T * qw;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const int64_t i = e / qw, r = e - i * qw, h = r / a.hd, d = r - h * a.hd;  // e indexes o[i][h][d]
        a.o[e] = live ? rq_apply(rd_gmax, a.hout[((size_t)h * a.T + i) * a.hd + d]) : 0;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0)
        put_rec(a.os, live ? sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), common) : Sc{0, 0});
}

// argmax_codes (generate.rs:48-56): *token = the first index of the largest of n codes. With record non-null the
// codes go to record + step * n and the scale to rscale[step], and *step advances (the per-step logits the
// generation hash covers) -- only while step lies in [0, cap), the rows record and rscale hold; any other step
// records nothing and stays where it is (the token is still chosen).
__global__ __launch_bounds__(RD_THREADS) void rd_argmax_kernel(const int32_t* __restrict__ logits, int n,
                                                               const kt_hip_qscale* __restrict__ ls,
                                                               int32_t* __restrict__ token, int32_t* record,
                                                               kt_hip_sscale* rscale, int32_t* step, int cap) {
    __shared__ int64_t red[RD_WAVES];
    // key: the value in the high word, the inverted index in the low word (the lower index wins a tie)
    auto key = [](int32_t v, int i) { return (int64_t)v * 4294967296LL + (int64_t)(0x7FFFFFFF - i); };
    int64_t best = INT64_MIN;
    const int s = record ? *step : 0;
    const bool keep = record && s >= 0 && s < cap;
    int32_t* rec = keep ? record + (size_t)s * n : nullptr;
    // one pass over the codes, 16-byte loads (and stores into the record) where n and the addresses allow, several in
    // flight per thread
    const bool vec = n % 4 == 0 && ((uintptr_t)logits & 15) == 0 && (!rec || ((uintptr_t)rec & 15) == 0);
    if (vec) {
        const int n4 = n / 4;
        const int4* l4 = reinterpret_cast<const int4*>(logits);
        constexpr int U = 4;
        for (int i0 = threadIdx.x; i0 < n4; i0 += U * RD_THREADS) {
            int4 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) v[u] = i0 + u * RD_THREADS < n4 ? l4[i0 + u * RD_THREADS] : int4{0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + u * RD_THREADS;
                if (i >= n4) break;
                if (rec) reinterpret_cast<int4*>(rec)[i] = v[u];
                const int64_t k0 = key(v[u].x, 4 * i), k1 = key(v[u].y, 4 * i + 1);
                const int64_t k2 = key(v[u].z, 4 * i + 2), k3 = key(v[u].w, 4 * i + 3);
                const int64_t a = k0 > k1 ? k0 : k1, b = k2 > k3 ? k2 : k3, c = a > b ? a : b;
                best = c > best ? c : best;
            }
        }
    } else {
        for (int i = threadIdx.x; i < n; i += RD_THREADS) {
            const int32_t v = logits[i];
            if (rec) rec[i] = v;
            const int64_t k = key(v, i);
            best = k > best ? k : best;
        }
    }
    best = block_max_i64(best, red);  // every thread has read *step past here
    if (threadIdx.x == 0) {
        if (keep) {
            rscale[s] = kt_hip_sscale{ls->mant, ls->shift, 1};
            *step = s + 1;
        }
        *token = 0x7FFFFFFF - (int32_t)(uint32_t)(best & 0xFFFFFFFF);
    }
}

// The attention step's LDS with hb heads' scores held at once: the per-step factors, hb score rows, the head
// outputs and the rotated q. hb = 1 is the least it runs with.
size_t rd_attention_lds(int max_seq, int nh, int hd, int hb) {
    return (size_t)max_seq * (2 * sizeof(Sc) + 8 * (size_t)hb) + (size_t)nh * hd * (8 + 4);
}
// The dynamic LDS the attention step may take on the current device: KT_REF_ATTN_LDS, less what the device's
// per-block limit leaves after the kernel's static LDS.
static size_t rd_attention_budget() {
    int dev = 0, mx = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 0;
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(&rd_attention_step_kernel)) != hipSuccess ||
        fa.sharedSizeBytes >= (size_t)mx)
        return 0;
    const size_t room = (size_t)mx - fa.sharedSizeBytes;
    return room < KT_REF_ATTN_LDS ? room : KT_REF_ATTN_LDS;
}
static int rd_attention_hb(int max_seq, int nh, int hd, size_t budget) {
    const size_t base = rd_attention_lds(max_seq, nh, hd, 0);
    if (base >= budget) return 0;
    const size_t hb = (budget - base) / (8 * (size_t)max_seq);
    return (int)(hb < (size_t)nh ? hb : (size_t)nh);
}

hipError_t launch_rd_embed(const int32_t* emb, int64_t e_mant, int32_t e_shift, const int32_t* token, int vocab,
                           int dim, int32_t* y, kt_hip_qscale* ys, hipStream_t s) {
    rd_embed_kernel<<<1, RD_THREADS, 0, s>>>(emb, e_mant, e_shift, token, vocab, dim, y, ys);
    return hipGetLastError();
}
hipError_t launch_rd_rmsnorm(const int32_t* x, int rows, int dim, const kt_hip_qscale* xs, const int32_t* g,
                             int64_t g_mant, int32_t g_shift, int64_t e_mant, int32_t e_shift, int32_t* y,
                             kt_hip_qscale* ys, hipStream_t s) {
    if (rows < 1 || rows > RD_MAX_ROWS) return hipErrorInvalidValue;
    rd_rmsnorm_kernel<<<1, RD_THREADS, 0, s>>>(x, rows, dim, xs, g, g_mant, g_shift, e_mant, e_shift, y, ys);
    return hipGetLastError();
}
hipError_t launch_rd_add(const int32_t* a, const kt_hip_qscale* as, const int32_t* b, const kt_hip_qscale* bs, int n,
                         int32_t* y, kt_hip_qscale* ys, hipStream_t s) {
    rd_add_kernel<<<1, RD_THREADS, 0, s>>>(a, as, b, bs, n, y, ys);
    return hipGetLastError();
}
hipError_t launch_rd_add_norm(const int32_t* a, const kt_hip_qscale* as, const int32_t* b, const kt_hip_qscale* bs,
                              int n, int32_t* y, kt_hip_qscale* ys, const int32_t* g, int64_t g_mant, int32_t g_shift,
                              int64_t e_mant, int32_t e_shift, int32_t* h, kt_hip_qscale* hs, hipStream_t s) {
    rd_add_norm_kernel<false><<<1, RD_THREADS, 0, s>>>(a, as, b, bs, RqSums{}, n, y, ys, g, g_mant, g_shift, e_mant,
                                                       e_shift, h, hs);
    return hipGetLastError();
}
hipError_t launch_rd_swiglu(const int32_t* g, const kt_hip_qscale* gs, const int32_t* u, const kt_hip_qscale* us,
                            int rows, int n, const int64_t* codes, const kt_hip_codelut* lut, int32_t* h,
                            kt_hip_qscale* hs, hipStream_t s) {
    rd_swiglu_kernel<false><<<(unsigned)rows, RD_THREADS, 0, s>>>(g, gs, u, us, RqSums{}, RqSums{}, n, codes, *lut, h,
                                                                  hs);
    return hipGetLastError();
}
hipError_t launch_rd_gelu(const int32_t* x, const kt_hip_qscale* xs, int64_t n, const int64_t* codes,
                          const kt_hip_codelut* lut, int32_t* y, kt_hip_qscale* ys, hipStream_t s) {
    const int64_t per = (int64_t)RD_THREADS * 4;
    const int64_t g = (n + per - 1) / per;
    rd_gelu_kernel<<<(unsigned)(g < 1 ? 1 : (g > 4096 ? 4096 : g)), RD_THREADS, 0, s>>>(x, xs, n, codes, *lut, y, ys);
    return hipGetLastError();
}
// With a workspace: the heads kernel (L.parts CTAs per q head) and the combine. Without: the one-CTA kernel, its LDS
// holding at least one head's scores at max_seq positions (the entry point checks which applies).
hipError_t launch_rd_attention_step(const RdAttn& a_in, hipStream_t s) {
    RdAttn a = a_in;
    if (a.ws) {
        const RdHeadsLayout L = rd_heads_layout(a.max_seq, a.nh, a.hd);
        const size_t qk = rd_round256((size_t)2 * a.hd * sizeof(int32_t)), lds = qk + L.arr_stride;
        if (lds <= RD_HEADS_LDS)
            a.sums ? rd_attention_heads_kernel<false, true><<<(unsigned)(a.nh * L.parts), RD_THREADS, lds, s>>>(a, L)
                   : rd_attention_heads_kernel<false, false><<<(unsigned)(a.nh * L.parts), RD_THREADS, lds, s>>>(a, L);
        else
            a.sums ? rd_attention_heads_kernel<true, true><<<(unsigned)(a.nh * L.parts), RD_THREADS, qk, s>>>(a, L)
                   : rd_attention_heads_kernel<true, false><<<(unsigned)(a.nh * L.parts), RD_THREADS, qk, s>>>(a, L);
        rd_attention_combine_kernel<<<1, RD_THREADS, 0, s>>>(a, L);
        return hipGetLastError();
    }
    const size_t budget = rd_attention_budget();
    a.hb = rd_attention_hb(a.max_seq, a.nh, a.hd, budget);
    if (a.hb < 1) return hipErrorInvalidValue;
    rd_attention_step_kernel<<<1, RD_THREADS, rd_attention_lds(a.max_seq, a.nh, a.hd, a.hb), s>>>(a);
    return hipGetLastError();
}
size_t rd_seq_workspace(int64_t rows) { return (sizeof(RdSeqWs) + (size_t)(rows > 1 ? rows - 1 : 0) * sizeof(Sc) + 255) / 256 * 256; }

hipError_t launch_rd_seq(const RdSeq& q, hipStream_t s) {
    rs_prep_kernel<<<1, RD_THREADS, 0, s>>>(q);
    const int64_t g = (q.n + 255) / 256;
    const unsigned grid = (unsigned)(g < 1 ? 1 : (g > 2048 ? 2048 : g));
    rs_max_kernel<<<grid, 256, 0, s>>>(q);
    rs_out_kernel<<<grid, 256, 0, s>>>(q);
    return hipGetLastError();
}

hipError_t launch_rd_embed_seq(const int32_t* emb, int64_t e_mant, int32_t e_shift, const int32_t* tokens, int T,
                               int vocab, int dim, int32_t* y, kt_hip_qscale* ys, hipStream_t s) {
    const int64_t g = ((int64_t)T * dim + 255) / 256;
    rd_embed_seq_kernel<<<(unsigned)(g < 1 ? 1 : (g > 4096 ? 4096 : g)), 256, 0, s>>>(emb, e_mant, e_shift, tokens,
                                                                                     T, vocab, dim, y, ys);
    return hipGetLastError();
}

// The prefill attention's workspace: rotated q and k, the head sums, the numerators' sums, the factors, gmax and
// the common scale, each part 256-byte aligned.
size_t rd_prefill_workspace(int64_t T, int64_t nh, int64_t nkv, int64_t hd, size_t off[7]) {
    const size_t sizes[7] = {(size_t)(T * nh * hd * 4), (size_t)(T * nkv * hd * 4), (size_t)(nh * T * hd * 8),
                             (size_t)(nh * T * 8), (size_t)(T * nh) * sizeof(Sc), 8, sizeof(Sc)};
    size_t at = 0;
    for (int i = 0; i < 7; i++) {
        off[i] = at;
        at += (sizes[i] + 255) / 256 * 256;
    }
    return at;
}

hipError_t launch_rd_attention_prefill(RdPrefill a, void* ws, hipStream_t s) {
    size_t off[7];
    rd_prefill_workspace(a.T, a.nh, a.nkv, a.hd, off);
    char* b = (char*)ws;
    a.qd = (int32_t*)(b + off[0]), a.kd = (int32_t*)(b + off[1]), a.hout = (int64_t*)(b + off[2]);
    a.hsum = (int64_t*)(b + off[3]), a.fac = (Sc*)(b + off[4]), a.gmax = (uint64_t*)(b + off[5]);
    a.common = (Sc*)(b + off[6]);
    rp_rope_kernel<<<(unsigned)a.T, 256, 0, s>>>(a);
    rp_head_kernel<<<(unsigned)(a.T * a.nh), 256, (size_t)a.T * 8, s>>>(a);
    rp_common_kernel<<<1, RD_THREADS, 0, s>>>(a);
    const int64_t n = (int64_t)a.T * a.nh * a.hd, g = (n + 255) / 256;
    const unsigned grid = (unsigned)(g < 1 ? 1 : (g > 2048 ? 2048 : g));
    rp_apply_kernel<<<grid, 256, 0, s>>>(a);
    rp_out_kernel<<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_rd_argmax(const int32_t* logits, int n, const kt_hip_qscale* ls, int32_t* token, int32_t* record,
                            kt_hip_sscale* rscale, int32_t* step, int cap, hipStream_t s) {
    rd_argmax_kernel<<<1, RD_THREADS, 0, s>>>(logits, n, ls, token, record, rscale, step, cap);
    return hipGetLastError();
}

}  // namespace kt


// ---------------------------------------------------------------------------------------------------------------
// C ABI (include/kt_hip.h): argument checks on the host, then one launch on `stream`.
// ---------------------------------------------------------------------------------------------------------------
#define RD_TRY(x)                               \
    do {                                        \
        const hipError_t e_ = (x);              \
        if (e_ != hipSuccess) return (int)e_;   \
    } while (0)

static const int64_t RD_MAX_N = (int64_t)1 << 30;

extern "C" int kt_hip_ref_embed(int dev, const int32_t* emb_dev, int64_t e_mant, int32_t e_shift,
                                const int32_t* token_dev, int64_t vocab, int64_t dim, int32_t* y_dev,
                                kt_hip_qscale* ys_dev, void* stream) {
    if (!emb_dev || !token_dev || !y_dev || !ys_dev || vocab < 1 || dim < 1 || vocab > INT32_MAX ||
        vocab * dim > ((int64_t)1 << 40) || dim > RD_MAX_N || e_mant < 0)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_embed(emb_dev, e_mant, e_shift, token_dev, (int)vocab, (int)dim, y_dev, ys_dev,
                                    (hipStream_t)stream);
}

extern "C" int kt_hip_ref_embed_seq(int dev, const int32_t* emb_dev, int64_t e_mant, int32_t e_shift,
                                    const int32_t* tokens_dev, int64_t T, int64_t vocab, int64_t dim, int32_t* y_dev,
                                    kt_hip_qscale* ys_dev, void* stream) {
    if (!emb_dev || !tokens_dev || !y_dev || !ys_dev || T < 1 || vocab < 1 || dim < 1 || vocab > INT32_MAX ||
        T > INT32_MAX || dim > INT32_MAX || T * dim > RD_MAX_N || e_mant < 0)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_embed_seq(emb_dev, e_mant, e_shift, tokens_dev, (int)T, (int)vocab, (int)dim, y_dev,
                                        ys_dev, (hipStream_t)stream);
}

extern "C" size_t kt_hip_ref_seq_workspace(int64_t rows) {
    return rows < 1 || rows > INT32_MAX ? 0 : kt::rd_seq_workspace(rows);
}

static int rd_seq_call(int dev, const kt::RdSeq& q, size_t ws_bytes, void* stream) {
    if (!q.a || !q.b || !q.as || !q.y || !q.ys || !q.ws || q.n < 1 || q.n > RD_MAX_N ||
        ws_bytes < kt::rd_seq_workspace(q.rows))
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_seq(q, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_add_seq(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev, const int32_t* b_dev,
                                  const kt_hip_qscale* bs_dev, int64_t n, void* ws_dev, size_t ws_bytes,
                                  int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream) {
    kt::RdSeq q{};
    q.op = kt::RS_ADD, q.a = a_dev, q.b = b_dev, q.as = as_dev, q.bs = bs_dev, q.n = n, q.rows = 1, q.dim = 1;
    q.ws = (kt::RdSeqWs*)ws_dev, q.y = y_dev, q.ys = ys_dev;
    if (!bs_dev) return (int)hipErrorInvalidValue;
    return rd_seq_call(dev, q, ws_bytes, stream);
}

extern "C" int kt_hip_ref_swiglu_seq(int dev, const int32_t* g_dev, const kt_hip_qscale* gs_dev, const int32_t* u_dev,
                                     const kt_hip_qscale* us_dev, int64_t n, const int64_t* silu_codes_dev,
                                     const kt_hip_codelut* silu, void* ws_dev, size_t ws_bytes, int32_t* h_dev,
                                     kt_hip_qscale* hs_dev, void* stream) {
    if (!silu || !silu_codes_dev || !us_dev || silu->n < 1 || !silu->right_identity) return (int)hipErrorInvalidValue;
    kt::RdSeq q{};
    q.op = kt::RS_SWIGLU, q.a = g_dev, q.b = u_dev, q.as = gs_dev, q.bs = us_dev, q.n = n, q.rows = 1, q.dim = 1;
    q.codes = silu_codes_dev, q.lut = *silu, q.ws = (kt::RdSeqWs*)ws_dev, q.y = h_dev, q.ys = hs_dev;
    return rd_seq_call(dev, q, ws_bytes, stream);
}

extern "C" int kt_hip_ref_rmsnorm_seq(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t rows,
                                      int64_t dim, const int32_t* g_dev, int64_t g_mant, int32_t g_shift,
                                      int64_t eps_mant, int32_t eps_shift, void* ws_dev, size_t ws_bytes,
                                      int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream) {
    if (rows < 1 || dim < 1 || rows > INT32_MAX || dim > INT32_MAX || rows * dim > RD_MAX_N || g_mant < 0 ||
        eps_mant < 0)
        return (int)hipErrorInvalidValue;
    kt::RdSeq q{};
    q.op = kt::RS_NORM, q.a = x_dev, q.b = g_dev, q.as = xs_dev, q.n = rows * dim, q.rows = (int)rows;
    q.dim = (int)dim, q.g_mant = g_mant, q.g_shift = g_shift, q.e_mant = eps_mant, q.e_shift = eps_shift;
    q.ws = (kt::RdSeqWs*)ws_dev, q.y = y_dev, q.ys = ys_dev;
    return rd_seq_call(dev, q, ws_bytes, stream);
}

extern "C" size_t kt_hip_ref_attention_prefill_workspace(int64_t T, int64_t nh, int64_t nkv, int64_t hd) {
    if (T < 1 || nh < 1 || nkv < 1 || hd < 2 || T > 8192 || nh > KT_REF_MAX_HEADS || hd > 256) return 0;
    size_t off[7];
    return kt::rd_prefill_workspace(T, nh, nkv, hd, off);
}

extern "C" int kt_hip_ref_attention_prefill(int dev, const int32_t* q_dev, const kt_hip_qscale* qs_dev,
                                            const int32_t* k_dev, const kt_hip_qscale* ks_dev, const int32_t* v_dev,
                                            const kt_hip_qscale* vs_dev, int64_t T, int64_t nh, int64_t nkv,
                                            int64_t hd, int64_t max_seq, const kt_hip_sscale* cos_dev,
                                            const kt_hip_sscale* sin_dev, int64_t isq_mant, int32_t isq_shift,
                                            const int64_t* exp_codes_dev, const kt_hip_codelut* exp_lut,
                                            void* ws_dev, size_t ws_bytes, int32_t* o_dev, kt_hip_qscale* os_dev,
                                            void* stream) {
    const size_t need = kt_hip_ref_attention_prefill_workspace(T, nh, nkv, hd);
    if (!q_dev || !qs_dev || !k_dev || !ks_dev || !v_dev || !vs_dev || !cos_dev || !sin_dev || !exp_codes_dev ||
        !exp_lut || !ws_dev || !o_dev || !os_dev || need == 0 || ws_bytes < need || T > max_seq || nh % nkv ||
        (hd & 1) || exp_lut->n < 1 || isq_mant < 0)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    kt::RdPrefill a{};
    a.q = q_dev, a.k = k_dev, a.v = v_dev, a.qs = qs_dev, a.ks = ks_dev, a.vs = vs_dev;
    a.T = (int)T, a.nh = (int)nh, a.nkv = (int)nkv, a.hd = (int)hd, a.cos = cos_dev, a.sin = sin_dev;
    a.isq_mant = isq_mant, a.isq_shift = isq_shift, a.exp_codes = exp_codes_dev, a.exp = *exp_lut;
    a.o = o_dev, a.os = os_dev;
    return (int)kt::launch_rd_attention_prefill(a, ws_dev, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_rmsnorm(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t rows,
                                  int64_t dim, const int32_t* g_dev, int64_t g_mant, int32_t g_shift,
                                  int64_t eps_mant, int32_t eps_shift, int32_t* y_dev, kt_hip_qscale* ys_dev,
                                  void* stream) {
    if (!x_dev || !xs_dev || !g_dev || !y_dev || !ys_dev || rows < 1 || dim < 1 || rows * dim > RD_MAX_N ||
        g_mant < 0 || eps_mant < 0)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_rmsnorm(x_dev, (int)rows, (int)dim, xs_dev, g_dev, g_mant, g_shift, eps_mant, eps_shift,
                                      y_dev, ys_dev, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_add(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev, const int32_t* b_dev,
                              const kt_hip_qscale* bs_dev, int64_t n, int32_t* y_dev, kt_hip_qscale* ys_dev,
                              void* stream) {
    if (!a_dev || !as_dev || !b_dev || !bs_dev || !y_dev || !ys_dev || n < 1 || n > RD_MAX_N)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_add(a_dev, as_dev, b_dev, bs_dev, (int)n, y_dev, ys_dev, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_add_rmsnorm(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev,
                                      const int32_t* b_dev, const kt_hip_qscale* bs_dev, int64_t n, int32_t* y_dev,
                                      kt_hip_qscale* ys_dev, const int32_t* g_dev, int64_t g_mant, int32_t g_shift,
                                      int64_t eps_mant, int32_t eps_shift, int32_t* h_dev, kt_hip_qscale* hs_dev,
                                      void* stream) {
    if (!a_dev || !as_dev || !b_dev || !bs_dev || !y_dev || !ys_dev || !g_dev || !h_dev || !hs_dev || n < 1 ||
        n > (int64_t)kt::RD_THREADS * kt::RD_AN || g_mant < 0 || eps_mant < 0 || h_dev == y_dev || h_dev == a_dev ||
        h_dev == b_dev || (void*)hs_dev == (void*)ys_dev)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_add_norm(a_dev, as_dev, b_dev, bs_dev, (int)n, y_dev, ys_dev, g_dev, g_mant, g_shift,
                                       eps_mant, eps_shift, h_dev, hs_dev, (hipStream_t)stream);
}

// The device view of one call's output of kt_hip_quant_linear_multi_sums (its workspace parts as ql_workspace_bytes
// lays them out at one row); false for a malformed description or one of other than n values.
static bool rq_sums_of(const kt_hip_ql_sums* d, int64_t n, kt::RqSums* r) {
    if (!d || !d->ws || d->seg < 0 || d->seg >= KT_QL_MAX_SEGMENTS || d->in_f < 1 || d->out_f < 1 || d->col0 < 0 ||
        d->n != n || d->col0 + d->n > d->out_f || (reinterpret_cast<uintptr_t>(d->ws) & 15))
        return false;
    size_t off[KT_QL_WS_PARTS];
    kt::ql_workspace_bytes(1, d->in_f, d->out_f, off);
    const char* base = static_cast<const char*>(d->ws);
    r->acc = reinterpret_cast<const int64_t*>(base + off[1]) + d->col0;
    r->st = reinterpret_cast<const kt::QlState*>(base + off[4]) + d->seg;
    r->rec = d->rec;
    return true;
}

extern "C" int kt_hip_ref_add_rmsnorm_sums(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev,
                                           const kt_hip_ql_sums* b, int64_t n, int32_t* y_dev, kt_hip_qscale* ys_dev,
                                           const int32_t* g_dev, int64_t g_mant, int32_t g_shift, int64_t eps_mant,
                                           int32_t eps_shift, int32_t* h_dev, kt_hip_qscale* hs_dev, void* stream) {
    kt::RqSums bs{};
    if (!a_dev || !as_dev || !y_dev || !ys_dev || !g_dev || !h_dev || !hs_dev || n < 1 ||
        n > (int64_t)kt::RD_THREADS * kt::RD_AN || g_mant < 0 || eps_mant < 0 || h_dev == y_dev || h_dev == a_dev ||
        (void*)hs_dev == (void*)ys_dev || !rq_sums_of(b, n, &bs) || bs.rec == as_dev || bs.rec == ys_dev ||
        bs.rec == hs_dev)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    kt::rd_add_norm_kernel<true><<<1, kt::RD_THREADS, 0, (hipStream_t)stream>>>(
        a_dev, as_dev, nullptr, nullptr, bs, (int)n, y_dev, ys_dev, g_dev, g_mant, g_shift, eps_mant, eps_shift, h_dev,
        hs_dev);
    return (int)hipGetLastError();
}

extern "C" int kt_hip_ref_swiglu_sums(int dev, const kt_hip_ql_sums* g, const kt_hip_ql_sums* u, int64_t n,
                                      const int64_t* silu_codes_dev, const kt_hip_codelut* silu, int32_t* h_dev,
                                      kt_hip_qscale* hs_dev, void* stream) {
    kt::RqSums gs{}, us{};
    if (!silu_codes_dev || !silu || !h_dev || !hs_dev || n < 1 || n > (int64_t)kt::RD_THREADS * 8 || silu->n < 1 ||
        !silu->right_identity || !rq_sums_of(g, n, &gs) || !rq_sums_of(u, n, &us) || gs.rec == hs_dev ||
        us.rec == hs_dev || (gs.rec && gs.rec == us.rec))
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    kt::rd_swiglu_kernel<true><<<1, kt::RD_THREADS, 0, (hipStream_t)stream>>>(
        nullptr, nullptr, nullptr, nullptr, gs, us, (int)n, silu_codes_dev, *silu, h_dev, hs_dev);
    return (int)hipGetLastError();
}

extern "C" int kt_hip_ref_swiglu(int dev, const int32_t* g_dev, const kt_hip_qscale* gs_dev, const int32_t* u_dev,
                                 const kt_hip_qscale* us_dev, int64_t rows, int64_t n, const int64_t* silu_codes_dev,
                                 const kt_hip_codelut* silu, int32_t* h_dev, kt_hip_qscale* hs_dev, void* stream) {
    if (!g_dev || !gs_dev || !u_dev || !us_dev || !silu_codes_dev || !silu || !h_dev || !hs_dev || rows < 1 ||
        rows > INT32_MAX || n < 1 || n > RD_MAX_N || silu->n < 1 || !silu->right_identity)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_swiglu(g_dev, gs_dev, u_dev, us_dev, (int)rows, (int)n, silu_codes_dev, silu, h_dev,
                                     hs_dev, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_gelu(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t n,
                               const int64_t* gelu_codes_dev, const kt_hip_codelut* gelu, int32_t* y_dev,
                               kt_hip_qscale* ys_dev, void* stream) {
    if (!x_dev || !xs_dev || !gelu_codes_dev || !gelu || !y_dev || !ys_dev || n < 1 || gelu->n < 1 ||
        !gelu->right_identity || (const void*)ys_dev == (const void*)xs_dev)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_gelu(x_dev, xs_dev, n, gelu_codes_dev, gelu, y_dev, ys_dev, (hipStream_t)stream);
}

extern "C" size_t kt_hip_ref_conv2d_workspace(int64_t ci, int64_t h, int64_t w, int64_t co, int64_t kh, int64_t kw,
                                              int64_t stride, int64_t pad) {
    if (ci < 1 || h < 1 || w < 1 || co < 1 || kh < 1 || kw < 1 || stride < 1 || pad < 0 || h + 2 * pad < kh ||
        w + 2 * pad < kw)
        return 0;
    const int64_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1;
    size_t off[KT_QL_WS_PARTS];
    return kt::ql_workspace_bytes(oh * ow, ci * kh * kw, co, off);
}

extern "C" int kt_hip_ref_conv2d(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t ci, int64_t h,
                                 int64_t w, const int8_t* w_planes_dev, int pw, int64_t co, int64_t kh, int64_t kw,
                                 int64_t stride, int64_t pad, int64_t w_mant, int32_t w_shift,
                                 const int64_t* bias_dev, int64_t b_mant, int32_t b_shift, void* ws_dev,
                                 size_t ws_bytes, int32_t* y_dev, kt_hip_qscale* os_dev, void* stream) {
    if (!x_dev || !xs_dev || !w_planes_dev || !ws_dev || !y_dev || !os_dev || (pw != 1 && pw != 3 && pw != 5) ||
        w_mant < 0 || b_mant < 0)
        return (int)hipErrorInvalidValue;
    const size_t need = kt_hip_ref_conv2d_workspace(ci, h, w, co, kh, kw, stride, pad);
    if (need == 0 || ws_bytes < need || ci * h * w >= ((int64_t)1 << 31) || kh >= 65536 || kw >= 65536 ||
        stride >= 65536 || pad >= 65536)  // the gather's pixel arithmetic stays within int32
        return (int)hipErrorInvalidValue;
    const int64_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1;
    const int64_t rows = oh * ow, kp = (ci * kh * kw + 63) / 64 * 64;
    if (rows * kp >= ((int64_t)1 << 31) || rows * co >= ((int64_t)1 << 31)) return (int)hipErrorInvalidValue;
    const kt::ConvGeom g{(int32_t)ci, (int32_t)h, (int32_t)w, (int32_t)kh, (int32_t)kw, (int32_t)stride,
                         (int32_t)pad, (int32_t)oh, (int32_t)ow};
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_ref_conv2d(x_dev, g, xs_dev, w_planes_dev, pw, co, w_mant, w_shift, bias_dev, b_mant,
                                      b_shift, kt_hip_flush_k(3, pw), ws_dev, y_dev, os_dev, (hipStream_t)stream);
}

extern "C" size_t kt_hip_ref_attention_step_workspace(int64_t max_seq, int64_t nh, int64_t hd) {
    if (nh < 1 || nh > KT_REF_MAX_HEADS || hd < 2 || hd > 1024 || max_seq < 1 || max_seq > KT_REF_ATTN_MAX_SEQ)
        return 0;
    const kt::RdHeadsLayout L = kt::rd_heads_layout((int)max_seq, (int)nh, (int)hd);
    return L.arr + (size_t)nh * L.parts * L.arr_stride;
}

extern "C" int kt_hip_ref_attention_step_ws(int dev, const int32_t* q_dev, const kt_hip_qscale* qs_dev,
                                            const int32_t* k_dev, const kt_hip_qscale* ks_dev, const int32_t* v_dev,
                                            const kt_hip_qscale* vs_dev, const int32_t* pos_dev, int64_t nh,
                                            int64_t nkv, int64_t hd, int64_t max_seq, int32_t* kc_dev,
                                            int32_t* vc_dev, kt_hip_sscale* kscale_dev, kt_hip_sscale* vscale_dev,
                                            const kt_hip_sscale* cos_dev, const kt_hip_sscale* sin_dev,
                                            int64_t isq_mant, int32_t isq_shift, const int64_t* exp_codes_dev,
                                            const kt_hip_codelut* exp_lut, int32_t* o_dev, kt_hip_qscale* os_dev,
                                            void* ws_dev, size_t ws_bytes, void* stream) {
    if (!q_dev || !qs_dev || !k_dev || !ks_dev || !v_dev || !vs_dev || !pos_dev || !kc_dev || !vc_dev ||
        !kscale_dev || !vscale_dev || !cos_dev || !sin_dev || !exp_codes_dev || !exp_lut || !o_dev || !os_dev)
        return (int)hipErrorInvalidValue;
    if (nh < 1 || nkv < 1 || nh % nkv || nh > KT_REF_MAX_HEADS || hd < 2 || (hd & 1) || hd > 1024 || max_seq < 1 ||
        max_seq > KT_REF_ATTN_MAX_SEQ || exp_lut->n < 1 || isq_mant < 0)
        return (int)hipErrorInvalidValue;
    if (ws_dev ? ((reinterpret_cast<uintptr_t>(ws_dev) & 15) ||
                  ws_bytes < kt_hip_ref_attention_step_workspace(max_seq, nh, hd))
               : kt::rd_attention_lds((int)max_seq, (int)nh, (int)hd, 1) > KT_REF_ATTN_LDS)
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    kt::RdAttn a{};
    a.q = q_dev, a.k = k_dev, a.v = v_dev, a.qs = qs_dev, a.ks = ks_dev, a.vs = vs_dev, a.pos = pos_dev;
    a.nh = (int)nh, a.nkv = (int)nkv, a.hd = (int)hd, a.max_seq = (int)max_seq;
    a.kc = kc_dev, a.vc = vc_dev, a.kscale = kscale_dev, a.vscale = vscale_dev, a.cos = cos_dev, a.sin = sin_dev;
    a.isq_mant = isq_mant, a.isq_shift = isq_shift, a.exp_codes = exp_codes_dev, a.exp = *exp_lut;
    a.o = o_dev, a.os = os_dev, a.ws = (unsigned char*)ws_dev;
    return (int)kt::launch_rd_attention_step(a, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_attention_step_sums(int dev, const kt_hip_ql_sums* q, const kt_hip_ql_sums* k,
                                              const kt_hip_ql_sums* v, const int32_t* pos_dev, int64_t nh,
                                              int64_t nkv, int64_t hd, int64_t max_seq, int32_t* kc_dev,
                                              int32_t* vc_dev, kt_hip_sscale* kscale_dev, kt_hip_sscale* vscale_dev,
                                              const kt_hip_sscale* cos_dev, const kt_hip_sscale* sin_dev,
                                              int64_t isq_mant, int32_t isq_shift, const int64_t* exp_codes_dev,
                                              const kt_hip_codelut* exp_lut, int32_t* o_dev, kt_hip_qscale* os_dev,
                                              void* ws_dev, size_t ws_bytes, void* stream) {
    if (!pos_dev || !kc_dev || !vc_dev || !kscale_dev || !vscale_dev || !cos_dev || !sin_dev || !exp_codes_dev ||
        !exp_lut || !o_dev || !os_dev || !ws_dev)
        return (int)hipErrorInvalidValue;
    if (nh < 1 || nkv < 1 || nh % nkv || nh > KT_REF_MAX_HEADS || hd < 2 || (hd & 1) || hd > 1024 || max_seq < 1 ||
        max_seq > KT_REF_ATTN_MAX_SEQ || exp_lut->n < 1 || isq_mant < 0 ||
        (reinterpret_cast<uintptr_t>(ws_dev) & 15) || ws_bytes < kt_hip_ref_attention_step_workspace(max_seq, nh, hd))
        return (int)hipErrorInvalidValue;
    kt::RdAttn a{};
    if (!rq_sums_of(q, nh * hd, &a.qsum) || !rq_sums_of(k, nkv * hd, &a.ksum) || !rq_sums_of(v, nkv * hd, &a.vsum))
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    a.sums = 1, a.pos = pos_dev;
    a.nh = (int)nh, a.nkv = (int)nkv, a.hd = (int)hd, a.max_seq = (int)max_seq;
    a.kc = kc_dev, a.vc = vc_dev, a.kscale = kscale_dev, a.vscale = vscale_dev, a.cos = cos_dev, a.sin = sin_dev;
    a.isq_mant = isq_mant, a.isq_shift = isq_shift, a.exp_codes = exp_codes_dev, a.exp = *exp_lut;
    a.o = o_dev, a.os = os_dev, a.ws = (unsigned char*)ws_dev;
    return (int)kt::launch_rd_attention_step(a, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_attention_step(int dev, const int32_t* q_dev, const kt_hip_qscale* qs_dev,
                                         const int32_t* k_dev, const kt_hip_qscale* ks_dev, const int32_t* v_dev,
                                         const kt_hip_qscale* vs_dev, const int32_t* pos_dev, int64_t nh,
                                         int64_t nkv, int64_t hd, int64_t max_seq, int32_t* kc_dev, int32_t* vc_dev,
                                         kt_hip_sscale* kscale_dev, kt_hip_sscale* vscale_dev,
                                         const kt_hip_sscale* cos_dev, const kt_hip_sscale* sin_dev,
                                         int64_t isq_mant, int32_t isq_shift, const int64_t* exp_codes_dev,
                                         const kt_hip_codelut* exp_lut, int32_t* o_dev, kt_hip_qscale* os_dev,
                                         void* stream) {
    return kt_hip_ref_attention_step_ws(dev, q_dev, qs_dev, k_dev, ks_dev, v_dev, vs_dev, pos_dev, nh, nkv, hd,
                                        max_seq, kc_dev, vc_dev, kscale_dev, vscale_dev, cos_dev, sin_dev, isq_mant,
                                        isq_shift, exp_codes_dev, exp_lut, o_dev, os_dev, nullptr, 0, stream);
}

extern "C" int kt_hip_ref_argmax(int dev, const int32_t* logits_dev, int64_t n, const kt_hip_qscale* ls_dev,
                                 int32_t* token_dev, int32_t* record_dev, kt_hip_sscale* rscale_dev,
                                 int32_t* step_dev, int64_t record_rows, void* stream) {
    if (!logits_dev || !ls_dev || !token_dev || n < 1 || n > INT32_MAX ||
        (record_dev && (!rscale_dev || !step_dev || record_rows < 1 || record_rows > INT32_MAX)))
        return (int)hipErrorInvalidValue;
    RD_TRY(hipSetDevice(dev));
    return (int)kt::launch_rd_argmax(logits_dev, (int)n, ls_dev, token_dev, record_dev, rscale_dev, step_dev,
                                     record_dev ? (int)record_rows : 0, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// Offline tables (host, f64): Scale::from_f64, CodeLut::build, Attention::new's RoPE Scales. No float expression
// here is contracted into a fused multiply-add, so each value is the one the reference's f64 arithmetic gives.
// ---------------------------------------------------------------------------------------------------------------
#pragma clang fp contract(off)

// frexp (kt-int/src/lib.rs:46-60) by bit surgery; x > 0 finite.
static double rd_frexp(double x, int* e) {
    uint64_t bits;
    memcpy(&bits, &x, 8);
    const int ef = (int)((bits >> 52) & 0x7ff);
    if (ef == 0) {
        int e2;
        const double m = rd_frexp(x * 9007199254740992.0, &e2);
        *e = e2 - 53;
        return m;
    }
    *e = ef - 1022;
    const uint64_t mb = (bits & ~(0x7ffULL << 52)) | (1022ULL << 52);
    double m;
    memcpy(&m, &mb, 8);
    return m;
}

extern "C" void kt_hip_ref_scale_from_f64(double x, int64_t* mant, int32_t* shift) {
    *mant = 0, *shift = 0;
    if (!(x > 0.0 && isfinite(x))) return;
    int e;
    const double m = rd_frexp(x, &e);
    *mant = (int64_t)round(m * 2147483648.0);
    *shift = 31 - e;
}

extern "C" int kt_hip_ref_from_reals(const double* real, int64_t n, int64_t levels, int32_t* codes, int64_t* mant,
                                     int32_t* shift) {
    if (!real || !codes || !mant || !shift || n < 0 || levels < 1 || levels > ((int64_t)1 << 30))
        return (int)hipErrorInvalidValue;
    double mx = 0.0;
    for (int64_t i = 0; i < n; i++) {
        if (!isfinite(real[i])) return (int)hipErrorInvalidValue;
        const double a = fabs(real[i]);
        mx = a > mx ? a : mx;
    }
    *mant = 0, *shift = 0;
    if (mx == 0.0) {
        memset(codes, 0, (size_t)n * sizeof(int32_t));
        return 0;
    }
    const double step = mx / (double)levels, inv = (double)levels / mx;
    for (int64_t i = 0; i < n; i++) codes[i] = (int32_t)round(real[i] * inv);  // |value| <= levels
    kt_hip_ref_scale_from_f64(step, mant, shift);
    return 0;
}

// erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7) and the exact GELU 0.5 x (1 + erf(x / sqrt 2)), in the
// reference's operation order (kt-model-vision/src/nonlin.rs:7-21).
static double rd_erf_as(double x) {
    const double sign = x < 0.0 ? -1.0 : 1.0;
    x = fabs(x);
    const double t = 1.0 / (1.0 + 0.3275911 * x);
    const double p = (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t + 0.254829592);
    return sign * (1.0 - p * t * exp(-x * x));
}
static double rd_gelu_f64(double x) { return 0.5 * x * (1.0 + rd_erf_as(x / 1.4142135623730951)); }

static double rd_lut_fn(int kind, double x) {
    switch (kind) {
        case KT_LUT_EXP:
            return exp(x);
        case KT_LUT_SILU:
            return x / (1.0 + exp(-x));
        case KT_LUT_SIGMOID:
            return 1.0 / (1.0 + exp(-x));
        case KT_LUT_GELU:
            return rd_gelu_f64(x);
        default:
            return 0.0;
    }
}

extern "C" int kt_hip_ref_codelut(int kind, double lo, double hi, int idx_bits, int code_bits, int right_identity,
                                  int64_t* codes, kt_hip_codelut* lut) {
    if (kind < KT_LUT_EXP || kind > KT_LUT_GELU || idx_bits < 1 || idx_bits > 24 || code_bits < 0 ||
        code_bits > 52 || !(hi > lo) || !lut)
        return (int)hipErrorInvalidValue;
    const int64_t n = (int64_t)1 << idx_bits;
    const double k = (double)(1ULL << code_bits);
    if (codes)
        for (int64_t i = 0; i < n; i++) {
            const double x = lo + (hi - lo) * ((double)i / (double)(n - 1));
            codes[i] = (int64_t)round(rd_lut_fn(kind, x) * k);
        }
    const double inv_step = (double)(n - 1) / (hi - lo);
    kt_hip_codelut L{};
    kt_hip_ref_scale_from_f64(inv_step, &L.inv_mant, &L.inv_shift);
    L.n = (int32_t)n;
    L.lo_index = (int64_t)round(lo * inv_step);
    kt_hip_ref_scale_from_f64(1.0 / k, &L.code_mant, &L.code_shift);
    L.right_identity = right_identity;
    *lut = L;
    return 0;
}

extern "C" int kt_hip_ref_rope_tables(int64_t max_seq, int64_t rot_dim, double theta, kt_hip_sscale* cos_tab,
                                      kt_hip_sscale* sin_tab) {
    if (max_seq < 1 || rot_dim < 2 || (rot_dim & 1) || !cos_tab || !sin_tab) return (int)hipErrorInvalidValue;
    const int64_t half = rot_dim / 2;
    for (int64_t p = 0; p < max_seq; p++)
        for (int64_t j = 0; j < half; j++) {
            const double inv_freq = pow(theta, -(2.0 * (double)j) / (double)rot_dim);
            const double ang = (double)p * inv_freq;
            const double c = cos(ang), s = sin(ang);
            kt_hip_sscale& C = cos_tab[p * half + j];
            kt_hip_sscale& S = sin_tab[p * half + j];
            kt_hip_ref_scale_from_f64(fabs(c), &C.mant, &C.shift);
            kt_hip_ref_scale_from_f64(fabs(s), &S.mant, &S.shift);
            C.sign = c < 0.0 ? -1 : 1;
            S.sign = s < 0.0 ? -1 : 1;
        }
    return 0;
}
#pragma clang fp contract(on)
