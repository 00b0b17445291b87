// The reference's MoeMlp on the device at its own integer semantics (crates/01-engine/kt-core/src/layers.rs:652-1020,
// router.rs:29-79). The reference runs its MoE token by token: every router and expert call is a QuantLinear of one
// row, quantized by that row's own maximum and requantized by its own output maximum. Grouping is exact only at the
// accumulate, so the device keeps every per-row step and groups just the products:
//
//   rq_quant / plane GEMM / rq_requant  QuantLinear::forward_int applied to each row on its own (layers.rs:275-328),
//                                       rows grouped by their weights (one digit-plane GEMM per group)
//   rm_route                            MoeMlp::route / route_sigmoid (layers.rs:826-870, router.rs:61-71)
//   rm_combine                          MoeMlp::combine, one token per CTA (layers.rs:893-923)
//   rm_merge_*                          merge_rows, the sequence's per-token outputs at one scale (layers.rs:873-891)
//
// The SwiGLU between the products is rd_swiglu_kernel (kt_refdec.hip) run one row per CTA, and the shared expert is a
// whole-tensor SwiGluMlp added with rd_add (layers.rs:757-780, 121-136).
#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "kt_kernels.h"
#include "kt_scale_dev.h"

namespace kt {

namespace {

constexpr int64_t WLEVELS = 265720;
constexpr int64_t ACT_LEVELS = 1LL << 28;
constexpr int RQ_THREADS = 256;

struct RqState {  // one output row's record between the passes
    int64_t xmax, c_mant;
    int32_t c_shift, mode;  // mode 0 normal, 1 xmax == 0, 2 c == 0
};

template <typename T>
__device__ T block_max_t(T v, T* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const T u = __shfl_xor(v, o, 64);
        v = u > v ? u : v;
    }
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) v = red[w] > v ? red[w] : v;
    __syncthreads();
    return v;
}
__device__ int64_t block_sum_i64(int64_t v, int64_t* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = (int64_t)((uint64_t)v + (uint64_t)__shfl_xor(v, o, 64));
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) v = (int64_t)((uint64_t)v + (uint64_t)red[w]);
    __syncthreads();
    return v;
}
__device__ inline Sc rec_sc(const kt_hip_qscale* r) { return Sc{r->mant, r->shift}; }
__device__ inline void put_rec(kt_hip_qscale* r, Sc s) {
    kt_hip_qscale o{};
    o.mant = s.mant, o.shift = s.shift;
    *r = o;
}
__device__ inline int64_t iabs(int64_t v) { return v < 0 ? (int64_t)(0 - (uint64_t)v) : v; }
__device__ inline int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
__device__ inline int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }

// The group of row r: the g with off[g] <= r < off[g + 1] (off: groups + 1 non-decreasing offsets).
__device__ inline int group_of(const int64_t* off, int groups, int64_t r) {
    int lo = 0, hi = groups - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= r) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

}  // namespace

// Row r: xmax of its input row, quant_to into 3 balanced base-256 planes laid out per group ([3][count_g][kp] at
// off[g] * 3 * kp), and its record: c = from_ratio(xmax, WLEVELS) * xs * ws_g (QuantLinear::forward_int steps 1-4).
__global__ __launch_bounds__(RQ_THREADS) void rq_quant_kernel(const int32_t* __restrict__ x,
                                                              const int32_t* __restrict__ xidx, int64_t x_rows,
                                                              int64_t in,
                                                              int64_t kp, const kt_hip_qscale* __restrict__ xs,
                                                              int xs_step, int groups, const int64_t* __restrict__ off,
                                                              const int64_t* __restrict__ wm,
                                                              const int32_t* __restrict__ wsh, RqState* __restrict__ st,
                                                              int8_t* __restrict__ xa) {
    __shared__ uint32_t red[RQ_THREADS / 64];
    const int64_t r = blockIdx.x;
    const int g = group_of(off, groups, r);
    const int64_t cnt = off[g + 1] - off[g], j = r - off[g];
    const int64_t xr = xidx ? (int64_t)xidx[r] : r;
    const bool inside = xr >= 0 && xr < x_rows;  // an index past x reads as a zero row (no access)
    const int32_t* src = x + (inside ? xr : 0) * in;
    uint32_t m = 0;
    for (int64_t i = threadIdx.x; inside && i < in; i += RQ_THREADS) {
        const int32_t v = src[i];
        const uint32_t a = v < 0 ? 0u - (uint32_t)v : (uint32_t)v;
        m = a > m ? a : m;
    }
    m = block_max_t(m, red);
    if (threadIdx.x == 0) {
        RqState s{};
        s.xmax = (int64_t)m;
        if (m == 0) {
            s.mode = 1;
        } else {
            const kt_hip_qscale* xrec = xs + (int64_t)xs_step * r;
            const Sc c = sc_mul(sc_mul(from_ratio((u128)m, (u128)WLEVELS), rec_sc(xrec)), Sc{wm[g], wsh[g]});
            s.c_mant = c.mant, s.c_shift = c.shift, s.mode = c.mant == 0 ? 2 : 0;
        }
        st[r] = s;
    }
    const int64_t xmax = (int64_t)m, half = xmax / 2;
    int8_t* base = xa + off[g] * 3 * kp;
    for (int64_t c = threadIdx.x; c < kp; c += RQ_THREADS) {
        int64_t v = 0;
        if (m != 0 && c < in) {
            const int64_t num = (int64_t)src[c] * WLEVELS;  // quant_to (layers.rs:23-31)
            const uint64_t q = ((uint64_t)(num < 0 ? -num : num) + (uint64_t)half) / (uint64_t)xmax;
            v = num >= 0 ? (int64_t)q : -(int64_t)q;
        }
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int64_t d = ((v + 128) & 255) - 128;
            base[(p * cnt + j) * kp + c] = (int8_t)d;
            v = (v - d) >> 8;
        }
    }
}

// Row r: ymax = max |acc|, y = requant_dyn(acc, ACT_LEVELS, ymax), the scale from_ratio(ymax, ACT_LEVELS) * c
// (QuantLinear::forward_int steps 8-10); zeros at Scale::ZERO for a zero input, a zero c or ymax = 0.
__global__ __launch_bounds__(RQ_THREADS) void rq_requant_kernel(const int64_t* __restrict__ acc, int64_t out,
                                                                const RqState* __restrict__ st,
                                                                int32_t* __restrict__ y,
                                                                kt_hip_qscale* __restrict__ ys) {
    __shared__ int64_t red[RQ_THREADS / 64];
    const int64_t r = blockIdx.x;
    const RqState s = st[r];
    const int64_t* a = acc + r * out;
    int64_t m = 0;
    if (s.mode == 0)
        for (int64_t i = threadIdx.x; i < out; i += RQ_THREADS) m = iabs(a[i]) > m ? iabs(a[i]) : m;
    const int64_t ymax = block_max_t(m, red);
    for (int64_t i = threadIdx.x; i < out; i += RQ_THREADS) y[r * out + i] = ymax ? requant_dyn_dev(a[i], ymax) : 0;
    if (threadIdx.x == 0) {
        kt_hip_qscale o{};
        o.xmax = s.xmax;
        if (ymax) {
            const Sc sc = sc_mul(from_ratio((u128)(uint64_t)ymax, (u128)ACT_LEVELS), Sc{s.c_mant, s.c_shift});
            o.mant = sc.mant, o.shift = sc.shift, o.ymax = ymax;
        }
        ys[r] = o;
    }
}

// MoeMlp::route / route_sigmoid for token t (one CTA): the softmax numerators exp(l - lmax) from the exp CodeLut at
// the logits' scale and top-k by logit code; or the sigmoid codes and top-k by code + coded bias. Ties go to the lower
// index (topk, layers.rs:800-805). sumc: the top-k codes' sum (norm_topk), all E codes' sum (softmax), or 2^20.
__global__ __launch_bounds__(RQ_THREADS) void rm_route_kernel(const int32_t* __restrict__ logits, int E, int top_k,
                                                              const kt_hip_qscale* __restrict__ ls, int sigmoid,
                                                              int norm_topk, const int64_t* __restrict__ codes,
                                                              kt_hip_codelut L, const int64_t* __restrict__ bias,
                                                              int32_t* __restrict__ sel, int64_t* __restrict__ ec,
                                                              int64_t* __restrict__ sumc) {
    extern __shared__ int64_t s_code[];  // E codes
    __shared__ int64_t red[RQ_THREADS / 64];
    __shared__ Sc s_mult;
    __shared__ int32_t s_pick;
    const int t = blockIdx.x;
    const int32_t* lg = logits + (int64_t)t * E;
    int32_t lmax = INT32_MIN;
    if (!sigmoid)
        for (int j = threadIdx.x; j < E; j += RQ_THREADS) lmax = lg[j] > lmax ? lg[j] : lmax;
    lmax = (int32_t)block_max_t((int64_t)lmax, red);
    if (threadIdx.x == 0) s_mult = sc_mul(rec_sc(ls + t), Sc{L.inv_mant, L.inv_shift});  // CodeLut::index's factor
    __syncthreads();
    int64_t part = 0;
    for (int j = threadIdx.x; j < E; j += RQ_THREADS) {
        const int64_t data = sigmoid ? (int64_t)lg[j] : (int64_t)lg[j] - lmax;
        const int64_t idx = sc_apply(s_mult, data) - L.lo_index;
        int64_t c;
        if (!sigmoid && idx < 0) c = 0;
        else c = codes[idx < 0 ? 0 : (idx > L.n - 1 ? L.n - 1 : idx)];
        s_code[j] = c;
        part += c;
    }
    const int64_t all = block_sum_i64(part, red);
    // top-k: k rounds of the largest key among the unpicked (ties to the lower index)
    int64_t tsum = 0;
    for (int i = 0; i < top_k; i++) {
        int64_t best = INT64_MIN;
        for (int j = threadIdx.x; j < E; j += RQ_THREADS) {
            bool used = false;
            for (int q = 0; q < i; q++) used |= sel[(int64_t)t * top_k + q] == j;
            if (used) continue;
            const int64_t key = sigmoid ? s_code[j] + bias[j] : (int64_t)lg[j];
            // key in the high bits, the inverted index below: the largest packed value is the largest key at the
            // lowest index (keys are below 2^40 in magnitude: codes, biases and logits are)
            const int64_t packed = key * 1048576 + (int64_t)(1048575 - j);
            best = packed > best ? packed : best;
        }
        best = block_max_t(best, red);
        if (threadIdx.x == 0) {
            const int j = 1048575 - (int)(((best % 1048576) + 1048576) % 1048576);
            s_pick = j;
            sel[(int64_t)t * top_k + i] = j;
            ec[(int64_t)t * top_k + i] = s_code[j];
        }
        __syncthreads();
        tsum += s_code[s_pick];
        __syncthreads();
    }
    if (threadIdx.x == 0) sumc[t] = norm_topk ? tsum : (sigmoid ? (int64_t)1 << 20 : all);
}

// MoeMlp::combine for token t (one CTA): its k expert outputs (rows pos[t, i] of y with records ys) brought to their
// largest scale, summed with the numerators ec, requantized, 1/sumc folded into the scale; zeros when sumc <= 0.
__global__ __launch_bounds__(RQ_THREADS) void rm_combine_kernel(const int32_t* __restrict__ y,
                                                                const kt_hip_qscale* __restrict__ ys, int y_rows,
                                                                int dim,
                                                                const int32_t* __restrict__ pos,
                                                                const int64_t* __restrict__ ec,
                                                                const int64_t* __restrict__ sumc, int top_k,
                                                                int32_t* __restrict__ out,
                                                                kt_hip_qscale* __restrict__ os) {
    __shared__ int64_t red[RQ_THREADS / 64];
    __shared__ Sc f[32], s_common;
    __shared__ int32_t s_row[32];
    const int t = blockIdx.x;
    const int64_t sc_ = sumc[t];
    if (threadIdx.x == 0) {
        Sc common{0, 0};
        for (int i = 0; i < top_k; i++) {
            const int32_t rw = pos[(int64_t)t * top_k + i];
            s_row[i] = rw >= 0 && rw < y_rows ? rw : -1;  // a row outside y contributes nothing (no access)
            const Sc s = s_row[i] >= 0 ? rec_sc(ys + rw) : Sc{0, 0};
            common = sc_ge(s, common) ? s : common;
        }
        s_common = common;
        if (common.mant != 0) {
            const Sc cinv = sc_recip(common);
            for (int i = 0; i < top_k; i++) f[i] = s_row[i] >= 0 ? sc_mul(rec_sc(ys + s_row[i]), cinv) : Sc{0, 0};
        }
    }
    __syncthreads();
    const Sc common = s_common;
    const bool live = sc_ > 0 && common.mant != 0;
    auto value = [&](int d) -> int64_t {
        int64_t acc = 0;
        for (int i = 0; i < top_k; i++)
            if (s_row[i] >= 0)
                acc = wadd(acc, wmul(ec[(int64_t)t * top_k + i], sc_apply(f[i], y[(int64_t)s_row[i] * dim + d])));
        return acc;
    };
    int64_t m = 0;
    if (live)
        for (int d = threadIdx.x; d < dim; d += RQ_THREADS) m = iabs(value(d)) > m ? iabs(value(d)) : m;
    const int64_t gmax = block_max_t(m, red);
    for (int d = threadIdx.x; d < dim; d += RQ_THREADS)
        out[(int64_t)t * dim + d] = gmax ? requant_dyn_dev(value(d), gmax) : 0;
    if (threadIdx.x == 0) {
        Sc s{0, 0};
        if (gmax)
            s = sc_mul(sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), common),
                       from_ratio(1, (u128)(uint64_t)sc_));
        put_rec(os + t, s);
    }
}

// merge_rows, pass 1 (one CTA): the largest of the T row scales (the engine's fold: of equal values the latest
// wins), each row's factor f_t = s_t / common into fac, and the global maximum's slot cleared.
__global__ __launch_bounds__(1024) void rm_merge_scale_kernel(const kt_hip_qscale* __restrict__ rs, int T,
                                                              Sc* __restrict__ fac, Sc* __restrict__ common_out,
                                                              unsigned long long* __restrict__ gmax_slot) {
    __shared__ Sc s_val[1024];
    __shared__ int s_idx[1024];
    Sc best{0, 0};
    int bi = -1;
    for (int t = threadIdx.x; t < T; t += 1024) {
        const Sc s = rec_sc(rs + t);
        if (bi < 0) {
            best = s, bi = t;
        } else {
            const bool ab = sc_ge(best, s), ba = sc_ge(s, best);
            if ((ab && ba) || ba) best = s, bi = t;  // t increases: on a tie the later row wins
        }
    }
    s_val[threadIdx.x] = best, s_idx[threadIdx.x] = bi;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) {
            const Sc a = s_val[threadIdx.x], b = s_val[threadIdx.x + o];
            const int ia = s_idx[threadIdx.x], ib = s_idx[threadIdx.x + o];
            bool take_b;
            if (ia < 0) take_b = true;
            else if (ib < 0) take_b = false;
            else {
                const bool ab = sc_ge(a, b), ba = sc_ge(b, a);
                take_b = (ab && ba) ? ib > ia : ba;
            }
            if (take_b) s_val[threadIdx.x] = b, s_idx[threadIdx.x] = ib;
        }
        __syncthreads();
    }
    const Sc common = s_val[0];
    __shared__ Sc s_cinv;
    if (threadIdx.x == 0) {
        *common_out = common;
        *gmax_slot = 0;
        if (common.mant != 0) s_cinv = sc_recip(common);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < T; t += 1024)
        fac[t] = common.mant != 0 ? sc_mul(rec_sc(rs + t), s_cinv) : Sc{0, 0};
}

// merge_rows, pass 2: the largest |f_t.apply(code)| over the whole tensor into the slot.
__global__ __launch_bounds__(RQ_THREADS) void rm_merge_max_kernel(const int32_t* __restrict__ rows, int64_t n,
                                                                  int dim, const Sc* __restrict__ fac,
                                                                  unsigned long long* __restrict__ gmax_slot) {
    __shared__ int64_t red[RQ_THREADS / 64];
    int64_t m = 0;
    for (int64_t i = (int64_t)blockIdx.x * RQ_THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * RQ_THREADS) {
        const int64_t v = iabs(sc_apply(fac[i / dim], rows[i]));
        m = v > m ? v : m;
    }
    m = block_max_t(m, red);
    if (threadIdx.x == 0 && m > 0) atomicMax(gmax_slot, (unsigned long long)m);
}

// merge_rows, pass 3: requant_dyn by the maximum, and the tensor's scale.
__global__ __launch_bounds__(RQ_THREADS) void rm_merge_out_kernel(const int32_t* __restrict__ rows, int64_t n,
                                                                  int dim, const Sc* __restrict__ fac,
                                                                  const Sc* __restrict__ common,
                                                                  const unsigned long long* __restrict__ gmax_slot,
                                                                  int32_t* __restrict__ out,
                                                                  kt_hip_qscale* __restrict__ os) {
    const int64_t gmax = (int64_t)*gmax_slot;
    for (int64_t i = (int64_t)blockIdx.x * RQ_THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * RQ_THREADS)
        out[i] = gmax ? requant_dyn_dev(sc_apply(fac[i / dim], rows[i]), gmax) : 0;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        put_rec(os, gmax ? sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), *common) : Sc{0, 0});
}

size_t rq_workspace_bytes(int64_t rows, int64_t in, int64_t out, size_t off[3]) {
    const size_t kp = (size_t)((in + 63) / 64 * 64);
    const size_t sizes[3] = {3 * (size_t)rows * kp, (size_t)rows * (size_t)out * 8, (size_t)rows * sizeof(RqState)};
    size_t at = 0;
    for (int i = 0; i < 3; i++) {
        off[i] = at;
        at += (sizes[i] + 255) / 256 * 256;
    }
    return at;
}

hipError_t launch_quant_linear_rows(const int32_t* x, const int32_t* xidx, int64_t x_rows, int64_t rows, int64_t in,
                                    const kt_hip_qscale* xs, int xs_step, int groups, const int64_t* off_host,
                                    const int64_t* off_dev, const int8_t* wb, size_t wgroup, int pw, int64_t out,
                                    const int64_t* wm_dev, const int32_t* wsh_dev, int64_t flush_k, void* ws,
                                    int32_t* y, kt_hip_qscale* ys, hipStream_t s) {
    size_t off[3];
    rq_workspace_bytes(rows, in, out, off);
    char* base = (char*)ws;
    int8_t* xa = (int8_t*)(base + off[0]);
    int64_t* acc = (int64_t*)(base + off[1]);
    RqState* st = (RqState*)(base + off[2]);
    const int64_t kp = (in + 63) / 64 * 64;
    rq_quant_kernel<<<(unsigned)rows, RQ_THREADS, 0, s>>>(x, xidx, x_rows, in, kp, xs, xs_step, groups, off_dev,
                                                          wm_dev, wsh_dev, st, xa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    for (int g = 0; g < groups; g++) {
        const int64_t r0 = off_host[g], cnt = off_host[g + 1] - r0;
        if (cnt <= 0) continue;
        for (int64_t k0 = 0; k0 < kp; k0 += flush_k) {
            const int64_t k1 = kp - k0 < flush_k ? kp : k0 + flush_k;
            e = launch_plane_gemm(3, pw, xa + r0 * 3 * kp, wb + (size_t)g * wgroup, acc + r0 * out, (int)cnt,
                                  (int)out, (int)kp, (int)k0, (int)k1, k0 > 0, 0, s);
            if (e != hipSuccess) return e;
        }
    }
    rq_requant_kernel<<<(unsigned)rows, RQ_THREADS, 0, s>>>(acc, out, st, y, ys);
    return hipGetLastError();
}

hipError_t launch_rm_route(const int32_t* logits, int T, int E, int top_k, const kt_hip_qscale* ls, int sigmoid,
                           int norm_topk, const int64_t* codes, const kt_hip_codelut* lut, const int64_t* bias,
                           int32_t* sel, int64_t* ec, int64_t* sumc, hipStream_t s) {
    rm_route_kernel<<<(unsigned)T, RQ_THREADS, (size_t)E * 8, s>>>(logits, E, top_k, ls, sigmoid, norm_topk, codes,
                                                                   *lut, bias, sel, ec, sumc);
    return hipGetLastError();
}

hipError_t launch_rm_combine(const int32_t* y, const kt_hip_qscale* ys, int y_rows, int dim, const int32_t* pos,
                             const int64_t* ec, const int64_t* sumc, int T, int top_k, int32_t* out,
                             kt_hip_qscale* os, hipStream_t s) {
    rm_combine_kernel<<<(unsigned)T, RQ_THREADS, 0, s>>>(y, ys, y_rows, dim, pos, ec, sumc, top_k, out, os);
    return hipGetLastError();
}

size_t rm_merge_workspace_bytes(int64_t T) { return (size_t)(T + 2) * sizeof(Sc) + 256; }

hipError_t launch_rm_merge_rows(const int32_t* rows, const kt_hip_qscale* rs, int T, int dim, void* ws, int32_t* out,
                                kt_hip_qscale* os, hipStream_t s) {
    Sc* fac = (Sc*)ws;
    Sc* common = fac + T;
    unsigned long long* slot = (unsigned long long*)(common + 1);
    rm_merge_scale_kernel<<<1, 1024, 0, s>>>(rs, T, fac, common, slot);
    const int64_t n = (int64_t)T * dim;
    int64_t g = (n + RQ_THREADS * 4 - 1) / (RQ_THREADS * 4);
    g = g < 1 ? 1 : (g > 1024 ? 1024 : g);
    rm_merge_max_kernel<<<(unsigned)g, RQ_THREADS, 0, s>>>(rows, n, dim, fac, slot);
    rm_merge_out_kernel<<<(unsigned)g, RQ_THREADS, 0, s>>>(rows, n, dim, fac, common, slot, out, os);
    return hipGetLastError();
}

}  // namespace kt

// ---------------------------------------------------------------------------------------------------------------
// C ABI (include/kt_hip.h)
// ---------------------------------------------------------------------------------------------------------------
#define RM_TRY(x)                               \
    do {                                        \
        const hipError_t e_ = (x);              \
        if (e_ != hipSuccess) return (int)e_;   \
    } while (0)

extern "C" size_t kt_hip_quant_linear_rows_workspace(int64_t rows, int64_t in_f, int64_t out_f) {
    size_t off[3];
    if (rows < 1 || in_f < 1 || out_f < 1) return 0;
    return kt::rq_workspace_bytes(rows, in_f, out_f, off);
}

extern "C" int kt_hip_quant_linear_rows(int dev, const int32_t* x_dev, const int32_t* xidx_dev, int64_t x_rows,
                                        int64_t rows, int64_t in_f, const kt_hip_qscale* xs_dev, int xs_step,
                                        int64_t groups, const int64_t* off_host, const int64_t* off_dev,
                                        const int8_t* w_planes_dev, size_t w_group_bytes, int pw, int64_t out_f,
                                        const int64_t* w_mant_dev, const int32_t* w_shift_dev, void* ws_dev,
                                        size_t ws_bytes, int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream) {
    if (!x_dev || !xs_dev || !off_host || !off_dev || !w_planes_dev || !w_mant_dev || !w_shift_dev || !ws_dev ||
        !y_dev || !ys_dev || rows < 1 || rows > INT32_MAX || in_f < 1 || out_f < 1 || x_rows < 1 || groups < 1 ||
        groups > INT32_MAX || (pw != 1 && pw != 3 && pw != 5) || (xs_step != 0 && xs_step != 1))
        return (int)hipErrorInvalidValue;
    const int64_t kp = (in_f + 63) / 64 * 64;
    if (rows * kp * 3 >= ((int64_t)1 << 40) || rows * out_f >= ((int64_t)1 << 31) || kp > INT_MAX)
        return (int)hipErrorInvalidValue;
    if (off_host[0] != 0 || off_host[groups] != rows) return (int)hipErrorInvalidValue;
    for (int64_t g = 0; g < groups; g++)
        if (off_host[g + 1] < off_host[g]) return (int)hipErrorInvalidValue;
    if (ws_bytes < kt_hip_quant_linear_rows_workspace(rows, in_f, out_f)) return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_quant_linear_rows(x_dev, xidx_dev, x_rows, rows, in_f, xs_dev, xs_step, (int)groups,
                                             off_host, off_dev, w_planes_dev, w_group_bytes, pw, out_f, w_mant_dev,
                                             w_shift_dev, kt_hip_flush_k(3, pw), ws_dev, y_dev, ys_dev,
                                             (hipStream_t)stream);
}

extern "C" int kt_hip_ref_moe_route(int dev, const int32_t* logits_dev, int64_t tokens, int64_t experts, int top_k,
                                    const kt_hip_qscale* ls_dev, int sigmoid, int norm_topk,
                                    const int64_t* codes_dev, const kt_hip_codelut* lut, const int64_t* bias_dev,
                                    int32_t* sel_dev, int64_t* ec_dev, int64_t* sumc_dev, void* stream) {
    if (!logits_dev || !ls_dev || !codes_dev || !lut || !sel_dev || !ec_dev || !sumc_dev || (sigmoid && !bias_dev) ||
        tokens < 1 || tokens > INT32_MAX || experts < 1 || experts > KT_REF_MOE_MAX_E || top_k < 1 ||
        top_k > experts || top_k > KT_REF_MOE_MAX_K || lut->n < 1)
        return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_rm_route(logits_dev, (int)tokens, (int)experts, top_k, ls_dev, sigmoid, norm_topk,
                                    codes_dev, lut, bias_dev, sel_dev, ec_dev, sumc_dev, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_moe_combine(int dev, const int32_t* y_dev, const kt_hip_qscale* ys_dev, int64_t y_rows,
                                      int64_t dim, const int32_t* pos_dev, const int64_t* ec_dev,
                                      const int64_t* sumc_dev, int64_t tokens, int top_k, int32_t* out_dev,
                                      kt_hip_qscale* os_dev, void* stream) {
    if (!y_dev || !ys_dev || !pos_dev || !ec_dev || !sumc_dev || !out_dev || !os_dev || dim < 1 || dim > INT32_MAX ||
        y_rows < 1 || y_rows > INT32_MAX || tokens < 1 || tokens > INT32_MAX || top_k < 1 || top_k > KT_REF_MOE_MAX_K)
        return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_rm_combine(y_dev, ys_dev, (int)y_rows, (int)dim, pos_dev, ec_dev, sumc_dev, (int)tokens,
                                      top_k, out_dev, os_dev, (hipStream_t)stream);
}

extern "C" size_t kt_hip_ref_merge_rows_workspace(int64_t tokens) {
    return tokens < 1 ? 0 : kt::rm_merge_workspace_bytes(tokens);
}

extern "C" int kt_hip_ref_merge_rows(int dev, const int32_t* rows_dev, const kt_hip_qscale* rs_dev, int64_t tokens,
                                     int64_t dim, void* ws_dev, size_t ws_bytes, int32_t* out_dev,
                                     kt_hip_qscale* os_dev, void* stream) {
    if (!rows_dev || !rs_dev || !ws_dev || !out_dev || !os_dev || tokens < 1 || tokens > INT32_MAX || dim < 1 ||
        dim > INT32_MAX || ws_bytes < kt::rm_merge_workspace_bytes(tokens))
        return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_rm_merge_rows(rows_dev, rs_dev, (int)tokens, (int)dim, ws_dev, out_dev, os_dev,
                                         (hipStream_t)stream);
}
