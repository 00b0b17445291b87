// The reference's MoeMlp on the device at its own integer semantics (crates/01-engine/kt-core/src/layers.rs:652-1020,
// router.rs:29-79). The reference runs its MoE token by token: every router and expert call is a QuantLinear of one
// row, quantized by that row's own maximum and requantized by its own output maximum. Grouping is exact only at the
// accumulate, so the device keeps every per-row step and groups just the products:
//
//   rq_plan                             the groups' tile tables, built on the device from the row offsets (no host
//                                       round trip: a caller may bucket the rows on the device, as rm_bucket does)
//   rq_quant / rq_skinny, rq_gemm /     QuantLinear::forward_int applied to each row on its own (layers.rs:275-328),
//   rq_requant                          rows grouped by their weights: the digit-plane products of every group in one
//                                       launch per kind (groups of 1 row, of 2-4 rows, 32-row MFMA tiles beyond)
//   rm_bucket                           the (token, expert) rows ordered by expert, on the device
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
#include "kt_w12_core.h"

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
            // (|num| + half) / xmax: |num| < 2^50 and the quotient at most WLEVELS, within udiv_small_q's range
            const uint64_t q = udiv_small_q((u128)(uint64_t)(num < 0 ? -num : num) + (u128)(uint64_t)half, xmax);
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

// ---------------------------------------------------------------------------------------------------------------
// The grouped digit-plane products. A row group g holds rows off_s[g] .. off_s[g + 1] - 1 (off_s: the caller's
// offsets made monotone and clamped to [0, rows] by rq_plan, so that no offset can reach outside the buffers); its
// 3 activation planes sit at xa + off_s[g] * 3 * kp as [3][count][kp], its pw weight planes at wb + g * wgroup as
// [pw][N][kp]. acc row r = the i64 sum over the planes, sum_{p,q} 256^(p+q) x_p . w_q, modulo 2^64 (the int32
// plane-group partials stay exact within the host's flush bound, as in the ungrouped product).
// ---------------------------------------------------------------------------------------------------------------
constexpr int RQ_SK_CPW = 2;   // skinny: output columns per wave
constexpr int RQ_SK_Y = 16;    // skinny: CTAs along the entry list (each strides it)
constexpr int RQ_BM = 32, RQ_BN = 128;

struct RqCaps {
    int64_t one, few, tiles;  // table capacities: groups of 1 row, of 2-4 rows, 32-row tiles of larger groups
};
RqCaps rq_caps(int64_t rows, int64_t groups) {
    const auto mn = [](int64_t a, int64_t b) { return a < b ? a : b; };
    // each kind's entries are bounded by the rows they cover: n1 <= rows, 2 n4 <= rows, and the tiles of the groups
    // of >= 5 rows number sum ceil(c / 32) < rows / 32 + (those groups) <= rows / 32 + rows / 5
    return RqCaps{mn(groups, rows), mn(groups, rows / 2), mn(groups, rows / 5) + rows / 32 + 1};
}

template <typename T, typename Op>
__device__ T block_incl_scan(T v, T* sh, Op op, T& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (int)(blockDim.x >> 6);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T u = __shfl_up(v, o, 64);
        if (lane >= o) v = op(v, u);
    }
    if (lane == 63) sh[wave] = v;
    __syncthreads();
    T pre{}, tot = sh[0];
    bool have = false;
    for (int w = 0; w < nw; w++) {
        if (w < wave) {
            pre = have ? op(pre, sh[w]) : sh[w];
            have = true;
        }
        if (w > 0) tot = op(tot, sh[w]);
    }
    __syncthreads();
    total = tot;
    return have ? op(pre, v) : v;
}

// The tables (one CTA of 1024 threads): off_s, then the group ids of the groups of exactly 1 row (e1) and of 2-4
// rows (e4), and (group, first row) of every 32-row tile of the larger groups (em); hdr = {n1, n4, nm}.
__global__ __launch_bounds__(1024) void rq_plan_kernel(const int64_t* __restrict__ off, int G, int64_t rows,
                                                       int64_t* __restrict__ off_s, int32_t* __restrict__ hdr,
                                                       int32_t* __restrict__ e1, int64_t cap1,
                                                       int32_t* __restrict__ e4, int64_t cap4, int2* __restrict__ em,
                                                       int64_t capm) {
    __shared__ int64_t sh[16];
    const auto mx = [](int64_t a, int64_t b) { return a > b ? a : b; };
    const auto add = [](int64_t a, int64_t b) { return a + b; };
    int64_t carry = 0;
    for (int base = 0; base <= G; base += 1024) {  // off_s[g] = clamp(max(off[0..g]), 0, rows); ends 0 and rows
        const int g = base + (int)threadIdx.x;
        int64_t v = g <= G ? off[g] : 0;
        v = v < 0 ? 0 : (v > rows ? rows : v);
        int64_t tot;
        v = mx(block_incl_scan(v, sh, mx, tot), carry);
        carry = mx(carry, tot);
        if (g == 0) v = 0;
        if (g == G) v = rows;
        if (g <= G) off_s[g] = v;
    }
    __syncthreads();  // off_s is read back by other threads of this CTA
    int64_t c1 = 0, c4 = 0, cm = 0;
    for (int base = 0; base < G; base += 1024) {
        const int g = base + (int)threadIdx.x;
        const int64_t cnt = g < G ? off_s[g + 1] - off_s[g] : 0;
        const int64_t a1 = cnt == 1, a4 = cnt >= 2 && cnt <= 4, am = cnt >= 5 ? (cnt + RQ_BM - 1) / RQ_BM : 0;
        int64_t t1, t4, tm;
        const int64_t p1 = block_incl_scan(a1, sh, add, t1) - a1 + c1;
        const int64_t p4 = block_incl_scan(a4, sh, add, t4) - a4 + c4;
        const int64_t pm = block_incl_scan(am, sh, add, tm) - am + cm;
        if (a1 && p1 < cap1) e1[p1] = g;
        if (a4 && p4 < cap4) e4[p4] = g;
        for (int64_t t = 0; t < am; t++)
            if (pm + t < capm) em[pm + t] = int2{g, (int)(t * RQ_BM)};
        c1 += t1, c4 += t4, cm += tm;
    }
    if (threadIdx.x == 0) {
        hdr[0] = (int32_t)(c1 < cap1 ? c1 : cap1);
        hdr[1] = (int32_t)(c4 < cap4 ? c4 : cap4);
        hdr[2] = (int32_t)(cm < capm ? cm : capm);
    }
}

// Groups of at most MM rows: a wave per RQ_SK_CPW output columns, its lanes striding k[k0, k1) in 16-byte chunks
// of every plane row (1 KB per load instruction), int32 plane-group sums per lane with sdot4, a butterfly across the
// wave. The CTAs along y stride the entry list (list[0 .. *count)).
template <int PW, int MM>
__global__ __launch_bounds__(256) void rq_skinny_kernel(const int8_t* __restrict__ xa, const int8_t* __restrict__ wb,
                                                        size_t wgroup, int64_t* __restrict__ acc, int N, int kp,
                                                        int k0, int k1, int accumulate,
                                                        const int64_t* __restrict__ off_s,
                                                        const int32_t* __restrict__ list,
                                                        const int32_t* __restrict__ count) {
    constexpr int PX = 3, NG = PX + PW - 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = ((int)blockIdx.x * 4 + wave) * RQ_SK_CPW;  // the wave's first column
    const int nch = (k1 - k0) / 16, n_ent = *count;
    for (int e = blockIdx.y; e < n_ent; e += gridDim.y) {
        const int g = list[e];
        const int64_t base = off_s[g];
        const int M = (int)(off_s[g + 1] - base);  // 1 .. MM by the plan
        const int8_t* xg = xa + base * 3 * kp;
        const int8_t* wg = wb + (size_t)g * wgroup;
        const size_t xplane = (size_t)M * kp, wplane = (size_t)N * kp;
        int a[RQ_SK_CPW][MM][NG];
#pragma unroll
        for (int c = 0; c < RQ_SK_CPW; c++)
#pragma unroll
            for (int m = 0; m < MM; m++)
#pragma unroll
                for (int q = 0; q < NG; q++) a[c][m][q] = 0;
        for (int qc = lane; qc < nch; qc += 64) {
            const size_t ko = (size_t)k0 + 16 * (size_t)qc;
            v4i xv[PX][MM], wv[RQ_SK_CPW][PW];
#pragma unroll
            for (int i = 0; i < PX; i++)
#pragma unroll
                for (int m = 0; m < MM; m++)
                    xv[i][m] = m < M ? gload16(xg + i * xplane + (size_t)m * kp + ko) : v4i{};
#pragma unroll
            for (int c = 0; c < RQ_SK_CPW; c++)
#pragma unroll
                for (int j = 0; j < PW; j++)
                    wv[c][j] = nb + c < N ? gload16(wg + j * wplane + (size_t)(nb + c) * kp + ko) : v4i{};
#pragma unroll
            for (int c = 0; c < RQ_SK_CPW; c++)
#pragma unroll
                for (int m = 0; m < MM; m++)
#pragma unroll
                    for (int i = 0; i < PX; i++)
#pragma unroll
                        for (int j = 0; j < PW; j++) {
                            int d = a[c][m][i + j];
#pragma unroll
                            for (int u = 0; u < 4; u++) d = __builtin_amdgcn_sdot4(xv[i][m][u], wv[c][j][u], d, false);
                            a[c][m][i + j] = d;
                        }
        }
#pragma unroll
        for (int c = 0; c < RQ_SK_CPW; c++)
#pragma unroll
            for (int m = 0; m < MM; m++)
#pragma unroll
                for (int q = 0; q < NG; q++)
#pragma unroll
                    for (int o = 32; o >= 1; o >>= 1) a[c][m][q] += __shfl_xor(a[c][m][q], o);
        if (lane == 0) {
#pragma unroll
            for (int c = 0; c < RQ_SK_CPW; c++) {
                const int n = nb + c;
                if (n >= N) continue;
#pragma unroll
                for (int m = 0; m < MM; m++) {
                    if (m >= M) continue;
                    uint64_t v = 0;
#pragma unroll
                    for (int q = 0; q < NG; q++) v += (uint64_t)(int64_t)a[c][m][q] << (8 * q);
                    int64_t* p = acc + (base + m) * N + n;
                    *p = (int64_t)(accumulate ? (uint64_t)*p + v : v);
                }
            }
        }
    }
}

// 32-row tiles of the larger groups: a CTA of 4 waves takes one tile (list[e] = (group, first row)) against RQ_BN
// output columns, each wave 32 x 32 with 32x32x32 int8 MFMAs per plane pair; k in 64-byte steps through
// double-buffered LDS (swizzled 16-byte chunks), the next step's loads in flight during the MFMAs. The CTAs are
// numbered so that each XCD (block b -> XCD b % 8) gets a contiguous run of (column tile, entry) work, the tiles of
// one group's rows next to each other, sharing the group's weight columns in that XCD's L2.
template <int PW>
__global__ __launch_bounds__(256) void rq_gemm_kernel(const int8_t* __restrict__ xa, const int8_t* __restrict__ wb,
                                                      size_t wgroup, int64_t* __restrict__ acc, int N, int kp, int k0,
                                                      int k1, int accumulate, const int64_t* __restrict__ off_s,
                                                      const int2* __restrict__ list, const int32_t* __restrict__ count,
                                                      int cap) {
    constexpr int PX = 3, BK = 64, CPR = BK / 16, NG = PX + PW - 1;
    constexpr int AC = PX * RQ_BM * CPR, BC = PW * RQ_BN * CPR;  // 16-byte chunks per k step
    constexpr int AL = (AC + 255) / 256, BL = BC / 256;
    static_assert(BC % 256 == 0, "B chunks per thread");
    __shared__ __attribute__((aligned(16))) int8_t sA[2][PX][RQ_BM * BK];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][PW][RQ_BN * BK];

    const int nbk = (int)gridDim.x, b = (int)blockIdx.x, xcd = b & 7, q8 = nbk >> 3, r8 = nbk & 7;
    const int w = xcd * q8 + (xcd < r8 ? xcd : r8) + (b >> 3);
    const int nt = w / cap, e = w - nt * cap;
    if (e >= *count) return;  // uniform: past the table
    const int2 ent = list[e];
    const int g = ent.x, m0 = ent.y;
    const int64_t base = off_s[g];
    const int M = (int)(off_s[g + 1] - base);
    const int n0 = nt * RQ_BN;
    const int8_t* xg = xa + base * 3 * kp;
    const int8_t* wg = wb + (size_t)g * wgroup;
    const size_t xplane = (size_t)M * kp, wplane = (size_t)N * kp;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    v16i c[NG];
#pragma unroll
    for (int q = 0; q < NG; q++) c[q] = v16i{};
    v4i ra[AL], rb[BL];
    auto gload_tile = [&](int k) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int idx = tid + 256 * i, p = idx / (RQ_BM * CPR), rem = idx % (RQ_BM * CPR);
            const int r = rem / CPR, ch = rem % CPR, gr = m0 + r;
            ra[i] = idx < AC && gr < M ? gload16(xg + p * xplane + (size_t)gr * kp + k + 16 * ch) : v4i{};
        }
#pragma unroll
        for (int i = 0; i < BL; i++) {
            const int idx = tid + 256 * i, p = idx / (RQ_BN * CPR), rem = idx % (RQ_BN * CPR);
            const int r = rem / CPR, ch = rem % CPR, gn = n0 + r;
            rb[i] = gn < N ? gload16(wg + p * wplane + (size_t)gn * kp + k + 16 * ch) : v4i{};
        }
    };
    auto lstore_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int idx = tid + 256 * i, p = idx / (RQ_BM * CPR), rem = idx % (RQ_BM * CPR);
            if (idx < AC) lds_write16(sA[buf][p], lds_off<CPR>(rem / CPR, rem % CPR), ra[i]);
        }
#pragma unroll
        for (int i = 0; i < BL; i++) {
            const int idx = tid + 256 * i, p = idx / (RQ_BN * CPR), rem = idx % (RQ_BN * CPR);
            lds_write16(sB[buf][p], lds_off<CPR>(rem / CPR, rem % CPR), rb[i]);
        }
    };

    const int nk = (k1 - k0) / BK;
    gload_tile(k0);
    lstore_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload_tile(k0 + (kt + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            const int chunk = 2 * ks + (lane >> 5);
            v4i av[PX], bv[PW];
#pragma unroll
            for (int p = 0; p < PX; p++) av[p] = lds_read16(sA[cur][p], lds_off<CPR>(lane & 31, chunk));
#pragma unroll
            for (int p = 0; p < PW; p++) bv[p] = lds_read16(sB[cur][p], lds_off<CPR>(32 * wave + (lane & 31), chunk));
#pragma unroll
            for (int i = 0; i < PX; i++)
#pragma unroll
                for (int j = 0; j < PW; j++) c[i + j] = mfma32(av[i], bv[j], c[i + j]);
        }
        if (kt + 1 < nk) lstore_tile(cur ^ 1);
        __syncthreads();
    }
    const int n = n0 + 32 * wave + (lane & 31);
    if (n >= N) return;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= M) continue;
        uint64_t v = 0;
#pragma unroll
        for (int q = 0; q < NG; q++) v += (uint64_t)(int64_t)c[q][r] << (8 * q);
        int64_t* p = acc + (base + m) * N + n;
        *p = (int64_t)(accumulate ? (uint64_t)*p + v : v);
    }
}

// MoeMlp's bucket on the device (one CTA of 1024 threads): the (token t, slot i) pairs of sel (T x k expert ids)
// grouped by expert: off (E + 1 offsets), xidx (row -> token), pos (pair -> row). Rows are placed by LDS atomics, so
// their order inside a group varies from call to call; every row is computed on its own, so the results do not. A
// pair whose id is outside [0, E) gets no row (pos -1) and the rows it would have used read as zero rows (xidx -1).
__global__ __launch_bounds__(1024) void rm_bucket_kernel(const int32_t* __restrict__ sel, int P, int top_k, int E,
                                                         int64_t* __restrict__ off, int32_t* __restrict__ xidx,
                                                         int32_t* __restrict__ pos) {
    extern __shared__ int32_t s_cur[];  // E cursors
    __shared__ int64_t sh[16];
    for (int e = threadIdx.x; e < E; e += 1024) s_cur[e] = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += 1024) {
        const int e = sel[p];
        if (e >= 0 && e < E) atomicAdd(&s_cur[e], 1);
    }
    __syncthreads();
    // exclusive scan of the counts, 1024 experts a pass
    int64_t carry = 0;
    const auto add = [](int64_t a, int64_t b) { return a + b; };
    for (int base = 0; base < E; base += 1024) {
        const int e = base + (int)threadIdx.x;
        const int64_t c = e < E ? s_cur[e] : 0;
        int64_t tot;
        const int64_t ex = block_incl_scan(c, sh, add, tot) - c + carry;
        if (e < E) off[e] = ex, s_cur[e] = (int32_t)ex;
        carry += tot;
    }
    if (threadIdx.x == 0) off[E] = carry;
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += 1024) {
        const int e = sel[p];
        if (e >= 0 && e < E) {
            const int r = atomicAdd(&s_cur[e], 1);
            xidx[r] = p / top_k, pos[p] = r;
        } else {
            pos[p] = -1;
        }
    }
    for (int r = (int)carry + (int)threadIdx.x; r < P; r += 1024) xidx[r] = -1;
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

// a.apply(v) of an int32 code v (sc_apply) in 64-bit arithmetic where that is exact: |mant| < 2^32 keeps |v * mant|
// below 2^63, and the rounding addend 2^(shift - 1) <= 2^62 keeps their sum below 2^64 unsigned. Same rounding
// (half away from zero) as sc_apply; other Scales go through it.
__device__ __forceinline__ int64_t sc_apply_i32(Sc a, bool fast, int32_t v) {
    if (!fast) return sc_apply(a, v);
    const uint64_t m = (uint64_t)(a.mant < 0 ? -a.mant : a.mant), x = v < 0 ? 0u - (uint64_t)(int64_t)v : (uint64_t)v;
    const uint64_t p = x * m;
    const uint64_t q = a.shift == 0 ? p : (p + ((uint64_t)1 << (a.shift - 1))) >> a.shift;
    return (v < 0) != (a.mant < 0) ? (int64_t)(0 - q) : (int64_t)q;
}

constexpr int RM_COMBINE_THREADS = 1024;

// MoeMlp::combine for token t (one CTA of 1024 threads): its k expert outputs (rows pos[t, i] of y with records ys)
// brought to their largest scale, summed with the numerators ec, requantized, 1/sumc folded into the scale; zeros
// when sumc <= 0. Each element's sum is formed twice (for the maximum, then for the output), not stored.
__global__ __launch_bounds__(RM_COMBINE_THREADS) void rm_combine_kernel(const int32_t* __restrict__ y,
                                                                       const kt_hip_qscale* __restrict__ ys,
                                                                       int y_rows, int dim,
                                                                       const int32_t* __restrict__ pos,
                                                                       const int64_t* __restrict__ ec,
                                                                       const int64_t* __restrict__ sumc, int top_k,
                                                                       int32_t* __restrict__ out,
                                                                       kt_hip_qscale* __restrict__ os) {
    __shared__ int64_t red[RM_COMBINE_THREADS / 64];
    __shared__ Sc f[KT_REF_MOE_MAX_K], s_common;
    __shared__ int32_t s_row[KT_REF_MOE_MAX_K];
    __shared__ int64_t s_ec[KT_REF_MOE_MAX_K];
    __shared__ bool s_fast[KT_REF_MOE_MAX_K];
    const int t = blockIdx.x;
    const int64_t sc_ = sumc[t];
    if (threadIdx.x == 0) {
        Sc common{0, 0};
        for (int i = 0; i < top_k; i++) {
            const int32_t rw = pos[(int64_t)t * top_k + i];
            s_row[i] = rw >= 0 && rw < y_rows ? rw : -1;  // a row outside y contributes nothing (no access)
            s_ec[i] = ec[(int64_t)t * top_k + i];
            const Sc s = s_row[i] >= 0 ? rec_sc(ys + rw) : Sc{0, 0};
            common = sc_ge(s, common) ? s : common;
        }
        s_common = common;
        for (int i = 0; i < top_k; i++) f[i] = Sc{0, 0}, s_fast[i] = true;
        if (common.mant != 0) {
            const Sc cinv = sc_recip(common);
            for (int i = 0; i < top_k; i++) {
                f[i] = s_row[i] >= 0 ? sc_mul(rec_sc(ys + s_row[i]), cinv) : Sc{0, 0};
                const int64_t m = f[i].mant;
                s_fast[i] = m > -((int64_t)1 << 32) && m < ((int64_t)1 << 32) && f[i].shift >= 0 && f[i].shift <= 63;
            }
        }
    }
    __syncthreads();
    const Sc common = s_common;
    const bool live = sc_ > 0 && common.mant != 0;
    auto value = [&](int d) -> int64_t {
        int64_t acc = 0;
        for (int i = 0; i < top_k; i++)
            if (s_row[i] >= 0 && f[i].mant != 0)
                acc = wadd(acc, wmul(s_ec[i], sc_apply_i32(f[i], s_fast[i], y[(int64_t)s_row[i] * dim + d])));
        return acc;
    };
    int64_t m = 0;
    if (live)
        for (int d = threadIdx.x; d < dim; d += RM_COMBINE_THREADS) {
            const int64_t a = iabs(value(d));
            m = a > m ? a : m;
        }
    const int64_t gmax = block_max_t(m, red);
    for (int d = threadIdx.x; d < dim; d += RM_COMBINE_THREADS)
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

// The workspace: activation planes, the i64 products, the row records, the sanitized offsets, the tables.
size_t rq_workspace_bytes(int64_t rows, int64_t in, int64_t out, int64_t groups, size_t off[5]) {
    const size_t kp = (size_t)((in + 63) / 64 * 64);
    const RqCaps c = rq_caps(rows, groups);
    const size_t sizes[5] = {3 * (size_t)rows * kp, (size_t)rows * (size_t)out * 8, (size_t)rows * sizeof(RqState),
                             (size_t)(groups + 1) * 8, 16 + 8 * (size_t)c.tiles + 4 * (size_t)(c.one + c.few)};
    size_t at = 0;
    for (int i = 0; i < 5; i++) {
        off[i] = at;
        at += (sizes[i] + 255) / 256 * 256;
    }
    return at;
}

template <int PW>
static void rq_products(const int8_t* xa, const int8_t* wb, size_t wgroup, int64_t* acc, int N, int kp, int k0, int k1,
                        int accumulate, const int64_t* off_s, const int32_t* hdr, const int32_t* e1, const int32_t* e4,
                        const int2* em, const RqCaps& c, hipStream_t s) {
    const unsigned gx = (unsigned)((N + 4 * RQ_SK_CPW - 1) / (4 * RQ_SK_CPW));
    if (c.one > 0)
        rq_skinny_kernel<PW, 1><<<dim3(gx, (unsigned)(c.one < RQ_SK_Y ? c.one : RQ_SK_Y)), 256, 0, s>>>(
            xa, wb, wgroup, acc, N, kp, k0, k1, accumulate, off_s, e1, hdr);
    if (c.few > 0)
        rq_skinny_kernel<PW, 4><<<dim3(gx, (unsigned)(c.few < RQ_SK_Y ? c.few : RQ_SK_Y)), 256, 0, s>>>(
            xa, wb, wgroup, acc, N, kp, k0, k1, accumulate, off_s, e4, hdr + 1);
    const int64_t nt = (N + RQ_BN - 1) / RQ_BN;
    rq_gemm_kernel<PW><<<(unsigned)(nt * c.tiles), 256, 0, s>>>(xa, wb, wgroup, acc, N, kp, k0, k1, accumulate,
                                                                 off_s, em, hdr + 2, (int)c.tiles);
}

hipError_t launch_quant_linear_rows(const int32_t* x, const int32_t* xidx, int64_t x_rows, int64_t rows, int64_t in,
                                    const kt_hip_qscale* xs, int xs_step, int groups, const int64_t* off_dev,
                                    const int8_t* wb, size_t wgroup, int pw, int64_t out, const int64_t* wm_dev,
                                    const int32_t* wsh_dev, int64_t flush_k, void* ws, int32_t* y, kt_hip_qscale* ys,
                                    hipStream_t s) {
    size_t off[5];
    rq_workspace_bytes(rows, in, out, groups, off);
    const RqCaps c = rq_caps(rows, groups);
    char* base = (char*)ws;
    int8_t* xa = (int8_t*)(base + off[0]);
    int64_t* acc = (int64_t*)(base + off[1]);
    RqState* st = (RqState*)(base + off[2]);
    int64_t* off_s = (int64_t*)(base + off[3]);
    int32_t* hdr = (int32_t*)(base + off[4]);
    int2* em = (int2*)(hdr + 4);
    int32_t* e1 = (int32_t*)(em + c.tiles);
    int32_t* e4 = e1 + c.one;
    const int64_t kp = (in + 63) / 64 * 64;
    rq_plan_kernel<<<1, 1024, 0, s>>>(off_dev, groups, rows, off_s, hdr, e1, c.one, e4, c.few, em, c.tiles);
    rq_quant_kernel<<<(unsigned)rows, RQ_THREADS, 0, s>>>(x, xidx, x_rows, in, kp, xs, xs_step, groups, off_s,
                                                          wm_dev, wsh_dev, st, xa);
    for (int64_t k0 = 0; k0 < kp; k0 += flush_k) {
        const int64_t k1 = kp - k0 < flush_k ? kp : k0 + flush_k;
        const int acc_in = k0 > 0;
        if (pw == 1)
            rq_products<1>(xa, wb, wgroup, acc, (int)out, (int)kp, (int)k0, (int)k1, acc_in, off_s, hdr, e1, e4, em,
                           c, s);
        else if (pw == 3)
            rq_products<3>(xa, wb, wgroup, acc, (int)out, (int)kp, (int)k0, (int)k1, acc_in, off_s, hdr, e1, e4, em,
                           c, s);
        else
            rq_products<5>(xa, wb, wgroup, acc, (int)out, (int)kp, (int)k0, (int)k1, acc_in, off_s, hdr, e1, e4, em,
                           c, s);
    }
    rq_requant_kernel<<<(unsigned)rows, RQ_THREADS, 0, s>>>(acc, out, st, y, ys);
    return hipGetLastError();
}

hipError_t launch_rm_bucket(const int32_t* sel, int P, int top_k, int E, int64_t* off, int32_t* xidx, int32_t* pos,
                            hipStream_t s) {
    rm_bucket_kernel<<<1, 1024, (size_t)E * 4, s>>>(sel, P, top_k, E, off, xidx, pos);
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
    rm_combine_kernel<<<(unsigned)T, RM_COMBINE_THREADS, 0, s>>>(y, ys, y_rows, dim, pos, ec, sumc, top_k, out,
                                                                  os);
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

extern "C" size_t kt_hip_quant_linear_rows_workspace(int64_t rows, int64_t in_f, int64_t out_f, int64_t groups) {
    size_t off[5];
    if (rows < 1 || in_f < 1 || out_f < 1 || groups < 1 || groups > INT32_MAX - 1) return 0;
    return kt::rq_workspace_bytes(rows, in_f, out_f, groups, off);
}

extern "C" int kt_hip_quant_linear_rows(int dev, const int32_t* x_dev, const int32_t* xidx_dev, int64_t x_rows,
                                        int64_t rows, int64_t in_f, const kt_hip_qscale* xs_dev, int xs_step,
                                        int64_t groups, const int64_t* off_host, const int64_t* off_dev,
                                        const int8_t* w_planes_dev, size_t w_group_bytes, int pw, int64_t out_f,
                                        const int64_t* w_mant_dev, const int32_t* w_shift_dev, void* ws_dev,
                                        size_t ws_bytes, int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream) {
    if (!x_dev || !xs_dev || !off_dev || !w_planes_dev || !w_mant_dev || !w_shift_dev || !ws_dev || !y_dev ||
        !ys_dev || rows < 1 || rows > INT32_MAX || in_f < 1 || out_f < 1 || out_f > INT32_MAX || x_rows < 1 ||
        groups < 1 || groups > INT32_MAX - 1 || (pw != 1 && pw != 3 && pw != 5) || (xs_step != 0 && xs_step != 1))
        return (int)hipErrorInvalidValue;
    const int64_t kp = (in_f + 63) / 64 * 64;
    if (rows * kp * 3 >= ((int64_t)1 << 40) || rows * out_f >= ((int64_t)1 << 31) || kp > INT_MAX)
        return (int)hipErrorInvalidValue;
    if (off_host) {  // the host's copy is checked; without one the device plan clamps the offsets
        if (off_host[0] != 0 || off_host[groups] != rows) return (int)hipErrorInvalidValue;
        for (int64_t g = 0; g < groups; g++)
            if (off_host[g + 1] < off_host[g]) return (int)hipErrorInvalidValue;
    }
    if (ws_bytes < kt_hip_quant_linear_rows_workspace(rows, in_f, out_f, groups)) return (int)hipErrorInvalidValue;
    const kt::RqCaps c = kt::rq_caps(rows, groups);
    if (((out_f + kt::RQ_BN - 1) / kt::RQ_BN) * c.tiles > INT32_MAX) return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_quant_linear_rows(x_dev, xidx_dev, x_rows, rows, in_f, xs_dev, xs_step, (int)groups,
                                             off_dev, w_planes_dev, w_group_bytes, pw, out_f, w_mant_dev, w_shift_dev,
                                             kt_hip_flush_k(3, pw), ws_dev, y_dev, ys_dev, (hipStream_t)stream);
}

extern "C" int kt_hip_ref_moe_bucket(int dev, const int32_t* sel_dev, int64_t tokens, int top_k, int64_t experts,
                                     int64_t* off_dev, int32_t* xidx_dev, int32_t* pos_dev, void* stream) {
    if (!sel_dev || !off_dev || !xidx_dev || !pos_dev || tokens < 1 || top_k < 1 || top_k > KT_REF_MOE_MAX_K ||
        experts < 1 || experts > KT_REF_MOE_MAX_E || tokens * top_k > INT32_MAX)
        return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_rm_bucket(sel_dev, (int)(tokens * top_k), top_k, (int)experts, off_dev, xidx_dev, pos_dev,
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
