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

// The per-row passes run one CTA of RQ_ROW_THREADS per row, each thread holding up to RQ_VPT of the row's values in
// registers between the row's maximum and its use (one load per value, all of a thread's loads in flight together);
// rows longer than RQ_ROW_THREADS * RQ_VPT take a second load per value.
constexpr int RQ_ROW_THREADS = 1024, RQ_VPT = 8;
// The grouped product's tiles: 32 rows x 128 output columns, k in steps of 64 bytes.
constexpr int RQ_BM = 32, RQ_BN = 128, RQ_BK = 64;

// The activation planes by tile: row j of group g sits in tile tb[g] + j / 32 at row j % 32; a tile is nkt
// k-steps of [3 planes][32 rows x 64 bytes], each 32 x 64 block in the MFMA reads' swizzled LDS layout (chunk c of row
// rr at rr * 64 + 16 (c ^ swz(rr))), so a k-step of a tile is 6 KB of contiguous bytes that DMA copies as they are.
__device__ __forceinline__ int64_t rq_a_off(int64_t ti, int64_t nkt, int p, int rr, int64_t c) {
    const int64_t kt = c >> 6, cc = (c >> 4) & 3;
    return ((ti * nkt + kt) * 3 + p) * (RQ_BM * RQ_BK) + rr * 64 + ((cc ^ ((rr >> 2) & 3)) << 4) + (c & 15);
}

// Row r: xmax of its input row, quant_to into 3 balanced base-256 planes (tiled as rq_a_off), and its record:
// c = from_ratio(xmax, WLEVELS) * xs * ws_g (QuantLinear::forward_int steps 1-4).
__global__ __launch_bounds__(RQ_ROW_THREADS) void rq_quant_kernel(const int32_t* __restrict__ x,
                                                                  const int32_t* __restrict__ xidx, int64_t x_rows,
                                                                  int64_t in, int64_t kp,
                                                                  const kt_hip_qscale* __restrict__ xs, int xs_step,
                                                                  int groups, const int64_t* __restrict__ off,
                                                                  const int32_t* __restrict__ tb, int64_t cap,
                                                                  const int64_t* __restrict__ wm,
                                                                  const int32_t* __restrict__ wsh,
                                                                  RqState* __restrict__ st, int8_t* __restrict__ xa) {
    __shared__ uint32_t red[RQ_ROW_THREADS / 64];
    const int64_t r = blockIdx.x;
    const int g = group_of(off, groups, r);
    const int64_t j = r - off[g], ti = tb[g] + j / RQ_BM, nkt = kp / RQ_BK;
    const int rr = (int)(j % RQ_BM);
    const int64_t xr = xidx ? (int64_t)xidx[r] : r;
    const bool inside = xr >= 0 && xr < x_rows;  // an index past x reads as a zero row (no access)
    const int32_t* src = x + (inside ? xr : 0) * in;
    const bool held = in <= (int64_t)RQ_ROW_THREADS * RQ_VPT;
    int32_t v[RQ_VPT];
    uint32_t m = 0;
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ_VPT; i++) {  // branch-free: a slot past the row loads its last value, then drops it
            const int64_t c = threadIdx.x + (int64_t)RQ_ROW_THREADS * i;
            const int32_t t = src[c < in ? c : in - 1];
            v[i] = inside && c < in ? t : 0;
        }
#pragma unroll
        for (int i = 0; i < RQ_VPT; i++) {
            const uint32_t a = v[i] < 0 ? 0u - (uint32_t)v[i] : (uint32_t)v[i];
            m = a > m ? a : m;
        }
    } else {
        for (int64_t i = threadIdx.x; inside && i < in; i += RQ_ROW_THREADS) {
            const int32_t t = src[i];
            const uint32_t a = t < 0 ? 0u - (uint32_t)t : (uint32_t)t;
            m = a > m ? a : m;
        }
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
    const bool tiled = ti < cap;  // always, by the table's capacity; a guard for the writes below
    auto put = [&](int64_t c, int32_t xv) {  // quant_to (layers.rs:23-31) of one value, its 3 digits
        if (!tiled) return;
        int64_t q = 0;
        if (m != 0 && c < in) {
            const int64_t num = (int64_t)xv * WLEVELS;
            // (|num| + half) / xmax: the numerator is below 2^51 and exact as a double, xmax below 2^32, so the
            // correctly rounded double quotient is within 2^-33 of the true one, which is at least 1 / xmax from
            // the next integer above it: its truncation is the floor (the check below is a guard)
            const uint64_t nn = (uint64_t)(num < 0 ? -num : num) + (uint64_t)half;
            uint64_t u = (uint64_t)((double)nn / (double)xmax);
            if (u * (uint64_t)xmax > nn) u--;
            q = num >= 0 ? (int64_t)u : -(int64_t)u;
        }
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int64_t d = ((q + 128) & 255) - 128;
            xa[rq_a_off(ti, nkt, p, rr, c)] = (int8_t)d;
            q = (q - d) >> 8;
        }
    };
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ_VPT; i++) {
            const int64_t c = threadIdx.x + (int64_t)RQ_ROW_THREADS * i;
            if (c < kp) put(c, v[i]);
        }
    } else {
        for (int64_t c = threadIdx.x; c < kp; c += RQ_ROW_THREADS) put(c, inside && c < in ? src[c] : 0);
    }
}

// Row r: ymax = max |acc|, y = requant_dyn(acc, ACT_LEVELS, ymax), the scale from_ratio(ymax, ACT_LEVELS) * c
// (QuantLinear::forward_int steps 8-10); zeros at Scale::ZERO for a zero input, a zero c or ymax = 0.
// acc holds `splits` slices of rows x out partial sums (runs of k); the row's product is their sum modulo 2^64.
__global__ __launch_bounds__(RQ_ROW_THREADS) void rq_requant_kernel(const int64_t* __restrict__ acc, int64_t rows,
                                                                    int64_t out, int splits,
                                                                    const RqState* __restrict__ st,
                                                                    int32_t* __restrict__ y,
                                                                    kt_hip_qscale* __restrict__ ys) {
    __shared__ int64_t red[RQ_ROW_THREADS / 64];
    const int64_t r = blockIdx.x;
    const RqState s = st[r];
    const int64_t* a = acc + r * out;
    const int64_t slice = rows * out;
    auto sum = [&](int64_t c) {
        uint64_t t = 0;
        for (int q = 0; q < splits; q++) t += (uint64_t)a[q * slice + c];
        return (int64_t)t;
    };
    const bool held = out <= (int64_t)RQ_ROW_THREADS * RQ_VPT;
    int64_t v[RQ_VPT];
    int64_t m = 0;
    if (held) {  // the slices 4 at a time, all of a thread's loads of them in flight together; a column block
                 // past the row (the same for the whole CTA) is skipped
#pragma unroll
        for (int i = 0; i < RQ_VPT; i++) v[i] = 0;
        int q0 = 0;
        for (; q0 + 4 <= splits; q0 += 4) {
            int64_t t[4][RQ_VPT];
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int i = 0; i < RQ_VPT; i++) {
                    const int64_t c = threadIdx.x + (int64_t)RQ_ROW_THREADS * i;
                    t[u][i] = (int64_t)RQ_ROW_THREADS * i < out ? a[(q0 + u) * slice + (c < out ? c : out - 1)] : 0;
                }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int i = 0; i < RQ_VPT; i++) v[i] = (int64_t)((uint64_t)v[i] + (uint64_t)t[u][i]);
        }
        for (; q0 < splits; q0++)
#pragma unroll
            for (int i = 0; i < RQ_VPT; i++) {
                const int64_t c = threadIdx.x + (int64_t)RQ_ROW_THREADS * i;
                if ((int64_t)RQ_ROW_THREADS * i < out)
                    v[i] = (int64_t)((uint64_t)v[i] + (uint64_t)a[q0 * slice + (c < out ? c : out - 1)]);
            }
#pragma unroll
        for (int i = 0; i < RQ_VPT; i++)
            if (threadIdx.x + (int64_t)RQ_ROW_THREADS * i >= out) v[i] = 0;
        if (s.mode == 0)
#pragma unroll
            for (int i = 0; i < RQ_VPT; i++) m = iabs(v[i]) > m ? iabs(v[i]) : m;
    } else if (s.mode == 0) {
        for (int64_t i = threadIdx.x; i < out; i += RQ_ROW_THREADS) m = iabs(sum(i)) > m ? iabs(sum(i)) : m;
    }
    const int64_t ymax = block_max_t(m, red);
    const RqDen rd_ymax = rq_den(ymax);
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ_VPT; i++) {
            const int64_t c = threadIdx.x + (int64_t)RQ_ROW_THREADS * i;
            if (c < out) y[r * out + c] = ymax ? rq_apply(rd_ymax, v[i]) : 0;
        }
    } else {
        for (int64_t i = threadIdx.x; i < out; i += RQ_ROW_THREADS)
            y[r * out + i] = ymax ? rq_apply(rd_ymax, sum(i)) : 0;
    }
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
// The tile table's capacity: the 32-row tiles of the non-empty groups number sum ceil(c / 32) < rows / 32 + (the
// non-empty groups) <= rows / 32 + min(groups, rows).
int64_t rq_tile_cap(int64_t rows, int64_t groups) { return (groups < rows ? groups : rows) + rows / 32 + 1; }

// The k split of the grouped product: S runs of k-tiles, each within the int32 flush bound of the plane-group sums
// (flush_k bytes), enough CTAs for the chip when the tiles are few (decode: a handful of one-row groups), each run at
// least 8 k-tiles long so the DMA ring fills; every run non-empty. The partial products land in S slices of acc.
int rq_splits(int64_t rows, int64_t groups, int64_t out, int64_t kp, int64_t flush_k) {
    const int64_t nkt = kp / RQ_BK, ftiles = flush_k / RQ_BK;
    const int64_t smin = (nkt + ftiles - 1) / ftiles;
    const int64_t ctas = ((out + RQ_BN - 1) / RQ_BN) * rq_tile_cap(rows, groups);
    int64_t S = (1024 + ctas - 1) / ctas;
    const int64_t smax = nkt / 8 > smin ? nkt / 8 : smin;
    S = S < smin ? smin : (S > smax ? smax : S);
    const int64_t per = (nkt + S - 1) / S;
    return (int)((nkt + per - 1) / per);
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

// The tile table (one CTA of 1024 threads): off_s, then (group, first row) of every 32-row tile of the non-empty
// groups in group order, tb[g] = the index of group g's first tile; hdr[0] = their number. 1024 groups a pass: off_s of the pass's 1024 upper ends by a
// running-maximum scan (kept in LDS with the lower end carried in), then a scan of the tile counts.
__global__ __launch_bounds__(1024) void rq_plan_kernel(const int64_t* __restrict__ off, int G, int64_t rows,
                                                       int64_t* __restrict__ off_s, int32_t* __restrict__ tb,
                                                       int32_t* __restrict__ hdr, int2* __restrict__ em,
                                                       int64_t capm) {
    __shared__ int64_t sh[16];
    __shared__ int64_t s_o[1025];
    const auto mx = [](int64_t a, int64_t b) { return a > b ? a : b; };
    const auto add = [](int64_t a, int64_t b) { return a + b; };
    const int tid = threadIdx.x;
    int64_t carry = 0, cm = 0;
    if (tid == 0) off_s[0] = 0;
    for (int base = 0; base < G; base += 1024) {  // groups base .. base + 1023: offsets base + 1 .. base + 1024
        const int idx = base + 1 + tid;
        int64_t v = idx <= G ? off[idx] : rows;
        v = v < 0 ? 0 : (v > rows ? rows : v);
        if (idx >= G) v = rows;
        int64_t tot;
        v = mx(block_incl_scan(v, sh, mx, tot), carry);
        if (idx <= G) off_s[idx] = v;
        s_o[tid + 1] = v;
        if (tid == 0) s_o[0] = carry;
        carry = mx(carry, tot);
        __syncthreads();
        const int g = base + tid;
        const int64_t cnt = g < G ? s_o[tid + 1] - s_o[tid] : 0;
        const int64_t am = (cnt + RQ_BM - 1) / RQ_BM;
        int64_t ptot;
        const int64_t pm = block_incl_scan(am, sh, add, ptot) - am + cm;
        if (g < G) tb[g] = (int32_t)(pm < capm ? pm : capm);  // the group's first tile
        for (int64_t t = 0; t < am; t++)
            if (pm + t < capm) em[pm + t] = int2{g, (int)(t * RQ_BM)};
        cm += ptot;
    }
    if (tid == 0) hdr[0] = (int32_t)(cm < capm ? cm : capm);
}

// The weight planes by tile (kt_hip_pack_planes_tiled): for each 128-row block of the outputs, nkt k-steps of
// [PW planes][128 rows x 64 bytes], each 128 x 64 block in the swizzled LDS layout; rows past the matrix are zero. A
// CTA's run of k-steps is then one contiguous stretch of memory.
__global__ void rq_pack_tiled_kernel(const int32_t* __restrict__ codes, int64_t rows, int64_t k, int64_t kp, int pw,
                                     int8_t* __restrict__ out) {
    // one thread per 16-byte chunk of the output: (n-block, k-step, plane, row, chunk position)
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nkt = kp / RQ_BK, nblk = (rows + RQ_BN - 1) / RQ_BN;
    if (idx >= nblk * nkt * pw * RQ_BN * 4) return;
    const int slot = (int)(idx & 3), r = (int)((idx >> 2) % RQ_BN);
    const int64_t rest = (idx >> 2) / RQ_BN;
    const int q = (int)(rest % pw);
    const int64_t kt = (rest / pw) % nkt, nb = (rest / pw) / nkt;
    const int c = slot ^ ((r >> 2) & 3);  // the chunk stored at this position
    const int64_t n = nb * RQ_BN + r, k0 = kt * RQ_BK + 16 * c;
    uint32_t wd[4] = {0, 0, 0, 0};
    for (int t = 0; t < 16; t++) {
        int64_t v = n < rows && k0 + t < k ? codes[n * k + k0 + t] : 0;
        int64_t d = 0;
        for (int i = 0; i <= q; i++) {  // digit q of the balanced base-256 expansion (as kt_hip_pack_planes)
            d = ((v + 128) & 255) - 128;
            v = (v - d) >> 8;
        }
        wd[t >> 2] |= ((uint32_t)d & 255u) << (8 * (t & 3));
    }
    *reinterpret_cast<v4i*>(out + idx * 16) = v4i{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
}

// The grouped product: a CTA of 4 waves takes one 32-row tile (list[e] = (group, first row)) against RQ_BN output
// columns and one run of k-steps, each wave 32 x 32 with 32x32x32 int8 MFMAs per plane pair. Every operand byte
// arrives by LDS DMA (buffer_load ... lds, 1 KB per instruction, lane l's 16 bytes at 16 l) into a ring of NS stages,
// NS - 1 k-steps in flight beyond the one being multiplied; both operands are stored tiled in the LDS image, so a
// k-step of the tile (6 KB) and of the weight block (PW x 8 KB) are contiguous and copy as they are. Each wave moves
// 2 + 2 PW pieces a step (A has 6: waves 2 and 3 send their second into a dump area), so one vmcnt target serves
// every wave. Tile rows past the group hold stale bytes: they only reach outputs that are not stored. The CTAs are
// numbered so that each XCD (block b -> XCD b % 8) gets a contiguous run of work.
// acc slice `split`: rows x N i64 partial sums of this run of k-steps.
template <int PW>
struct RqRing {
    static constexpr int NS = PW == 5 ? 3 : 4;
    static constexpr int A_BYTES = 3 * RQ_BM * RQ_BK, B_BYTES = PW * RQ_BN * RQ_BK, STAGE = A_BYTES + B_BYTES;
    static constexpr int DUMP = NS * STAGE, LDS = DUMP + 1024;
    static constexpr int DPW = 2 + 2 * PW;  // DMA instructions per wave and k-step
    static_assert(DPW * (NS - 2) <= 63, "vmcnt holds the DMAs of NS - 2 later steps");
};

template <int PW>
__global__ __launch_bounds__(256) void rq_gemm_kernel(const int8_t* __restrict__ xa, int64_t rows, int64_t kp_,
                                                      const int8_t* __restrict__ wb, size_t wgroup,
                                                      int64_t* __restrict__ acc, int N,
                                                      const int64_t* __restrict__ off_s,
                                                      const int2* __restrict__ list, const int32_t* __restrict__ count,
                                                      int cap, int ntile, int per) {
    using R = RqRing<PW>;
    constexpr int NS = R::NS;
    extern __shared__ __attribute__((aligned(16))) int8_t ring[];
    const int nkt = (int)(kp_ / RQ_BK);
    const int nbk = (int)gridDim.x, b = (int)blockIdx.x, xcd = b & 7, q8 = nbk >> 3, r8 = nbk & 7;
    const int w = xcd * q8 + (xcd < r8 ? xcd : r8) + (b >> 3);
    const int e = w % cap, rest = w / cap, nt = rest % ntile, split = rest / ntile;
    if (e >= *count) return;  // uniform: past the table
    const int2 ent = list[e];
    const int g = ent.x, m0 = ent.y;
    const int64_t base = off_s[g];
    const int M = (int)(off_s[g + 1] - base);
    const int n0 = nt * RQ_BN;
    const int kt0 = split * per;
    const int nk = nkt - kt0 < per ? nkt - kt0 : per;  // >= 1 by the host's choice of the split
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);

    // this tile's k-steps (e is its index in the tiled activations) and this block's weight k-steps
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(xa + (int64_t)e * nkt * R::A_BYTES, (uint32_t)(nkt * R::A_BYTES));
    const __amdgpu_buffer_rsrc_t rB =
        make_rsrc(wb + (size_t)g * wgroup + (size_t)nt * nkt * R::B_BYTES, (uint32_t)(nkt * R::B_BYTES));
    const uint32_t lo = 16u * (uint32_t)lane;
    const int pa1 = wv + 4;  // this wave's A pieces: wv and wv + 4 (pieces 6, 7 re-read piece 0 into the dump)
    auto issue = [&](int st, int kt) {
        const int kk = kt0 + (kt < nk ? kt : nk - 1);  // past the run: a re-read into a stage nobody reads
        const uint32_t ka = (uint32_t)kk * R::A_BYTES, kb = (uint32_t)kk * R::B_BYTES;
        int8_t* sp = ring + st * R::STAGE;
        dma16(rA, sp + 1024 * wv, lo + 1024u * (uint32_t)wv, ka);
        dma16(rA, pa1 < 6 ? sp + 1024 * pa1 : ring + R::DUMP, lo + (pa1 < 6 ? 1024u * (uint32_t)pa1 : 0u), ka);
#pragma unroll
        for (int t = 0; t < 2 * PW; t++)
            dma16(rB, sp + R::A_BYTES + 1024 * (wv + 4 * t), lo + 1024u * (uint32_t)(wv + 4 * t), kb);
    };
    auto wait_step = [&]() {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(R::DPW * (NS - 2)) : "memory");
    };

    v16i c[3 + PW - 1];
#pragma unroll
    for (int q = 0; q < 3 + PW - 1; q++) c[q] = v16i{};
#pragma unroll
    for (int t = 0; t < NS - 1; t++) issue(t, t);
    for (int kt = 0; kt < nk; kt++) {
        wait_step();  // step kt has landed for every wave; every wave is done reading step kt - 1
        issue((kt + NS - 1) % NS, kt + NS - 1);
        const int8_t* sp = ring + (kt % NS) * R::STAGE;
#pragma unroll
        for (int ks = 0; ks < RQ_BK / 32; ks++) {
            const int chunk = 2 * ks + (lane >> 5);
            v4i av[3], bv[PW];
#pragma unroll
            for (int p = 0; p < 3; p++) av[p] = lds_read16(sp + p * (RQ_BM * RQ_BK), lds_off<4>(lane & 31, chunk));
#pragma unroll
            for (int q = 0; q < PW; q++)
                bv[q] = lds_read16(sp + R::A_BYTES + q * (RQ_BN * RQ_BK), lds_off<4>(32 * wv + (lane & 31), chunk));
#pragma unroll
            for (int i = 0; i < 3; i++)
#pragma unroll
                for (int j = 0; j < PW; j++) c[i + j] = mfma32(av[i], bv[j], c[i + j]);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA may land after the CTA ends
    const int n = n0 + 32 * wv + (lane & 31);
    if (n >= N) return;
    int64_t* slice = acc + (int64_t)split * rows * N;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= M) continue;
        uint64_t v = 0;
#pragma unroll
        for (int q = 0; q < 3 + PW - 1; q++) v += (uint64_t)(int64_t)c[q][r] << (8 * q);
        slice[(base + m) * N + n] = (int64_t)v;
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
    // top-k: k rounds of the largest key among the unpicked (ties to the lower index). Each thread's keys (experts
    // tid + RQ_THREADS i) are formed once and held in registers; a picked expert's key drops to the minimum.
    // The key sits in the high bits and the inverted index below: the largest packed value is the largest key at
    // the lowest index (keys are below 2^40 in magnitude: codes, biases and logits are).
    constexpr int KPT = KT_REF_MOE_MAX_E / RQ_THREADS;
    int64_t kreg[KPT];
#pragma unroll
    for (int q = 0; q < KPT; q++) {
        const int j = threadIdx.x + RQ_THREADS * q;
        kreg[q] = INT64_MIN;
        if (j < E) kreg[q] = (sigmoid ? s_code[j] + bias[j] : (int64_t)lg[j]) * 1048576 + (int64_t)(1048575 - j);
    }
    int64_t tsum = 0;
    for (int i = 0; i < top_k; i++) {
        int64_t best = INT64_MIN;
#pragma unroll
        for (int q = 0; q < KPT; q++) best = kreg[q] > best ? kreg[q] : best;
        best = block_max_t(best, red);
        const int j = 1048575 - (int)(((best % 1048576) + 1048576) % 1048576);
        if (threadIdx.x == 0) {
            sel[(int64_t)t * top_k + i] = j;
            ec[(int64_t)t * top_k + i] = s_code[j];
        }
        if ((j % RQ_THREADS) == (int)threadIdx.x) {
#pragma unroll
            for (int q = 0; q < KPT; q++)
                if (q == j / RQ_THREADS) kreg[q] = INT64_MIN;
        }
        tsum += s_code[j];
    }
    if (threadIdx.x == 0) sumc[t] = norm_topk ? tsum : (sigmoid ? (int64_t)1 << 20 : all);
}

// a.apply(v) of an int32 code v (sc_apply) in 64-bit arithmetic where that is exact: |mant| < 2^32 keeps |v * mant|
// below 2^63, and the rounding addend 2^(shift - 1) <= 2^62 keeps their sum below 2^64 unsigned. Same rounding
// (half away from zero) as sc_apply; other Scales go through it.
__device__ __forceinline__ int64_t sc_apply_i32(Sc a, bool fast, int32_t v) {
    if (!fast) return sc_apply(a, v);
    // |mant| < 2^32 and |v| <= 2^31: one 32 x 32 -> 64-bit product (the integer multiplies run at quarter rate)
    const uint32_t m = (uint32_t)(a.mant < 0 ? -a.mant : a.mant), x = v < 0 ? 0u - (uint32_t)v : (uint32_t)v;
    const uint64_t p = (uint64_t)x * (uint64_t)m;
    const uint64_t q = a.shift == 0 ? p : (p + ((uint64_t)1 << (a.shift - 1))) >> a.shift;
    return (v < 0) != (a.mant < 0) ? (int64_t)(0 - q) : (int64_t)q;
}

constexpr int RM_COMBINE_THREADS = 1024, RM_VPT = 4, RM_KB = 4;

// MoeMlp::combine for token t (one CTA of 1024 threads): its k expert outputs (rows pos[t, i] of y with records ys)
// brought to their largest scale, summed with the numerators ec, requantized, 1/sumc folded into the scale; zeros
// when sumc <= 0. Up to RM_VPT sums per thread stay in registers between the maximum and the requant, and the
// expert rows are read RM_KB at a time (all those loads in flight together, branch-free); longer rows form each sum
// twice.
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
    __shared__ Sc s_rec[KT_REF_MOE_MAX_K];
    const int t = blockIdx.x;
    const int64_t sc_ = sumc[t];
    if (threadIdx.x < top_k) {  // the k rows, numerators and records, fetched in parallel
        const int i = threadIdx.x;
        const int32_t rw = pos[(int64_t)t * top_k + i];
        s_row[i] = rw >= 0 && rw < y_rows ? rw : -1;  // a row outside y contributes nothing (no access)
        s_ec[i] = ec[(int64_t)t * top_k + i];
        s_rec[i] = s_row[i] >= 0 ? rec_sc(ys + rw) : Sc{0, 0};
    }
    __syncthreads();
    __shared__ Sc s_cinv;
    if (threadIdx.x == 0) {
        Sc common{0, 0};
        for (int i = 0; i < top_k; i++) common = sc_ge(s_rec[i], common) ? s_rec[i] : common;
        s_common = common;
        if (common.mant != 0) s_cinv = sc_recip(common);
    }
    __syncthreads();
    if (threadIdx.x < top_k) {  // each row's factor to the common scale, k threads at once
        const int i = threadIdx.x;
        f[i] = s_common.mant != 0 && s_row[i] >= 0 ? sc_mul(s_rec[i], s_cinv) : Sc{0, 0};
        const int64_t m = f[i].mant;
        s_fast[i] = m > -((int64_t)1 << 32) && m < ((int64_t)1 << 32) && f[i].shift >= 0 && f[i].shift <= 63;
    }
    __syncthreads();
    const Sc common = s_common;
    const bool live = sc_ > 0 && common.mant != 0;
    // the sums of the RM_VPT elements d0 + RM_COMBINE_THREADS * j (j < RM_VPT, d < dim), rows read RM_KB at a time
    auto sums = [&](int d0, int64_t (&acc)[RM_VPT]) {
#pragma unroll
        for (int j = 0; j < RM_VPT; j++) acc[j] = 0;
        for (int i0 = 0; i0 < top_k; i0 += RM_KB) {
            int32_t yv[RM_KB][RM_VPT];
#pragma unroll
            for (int ii = 0; ii < RM_KB; ii++) {
                const int i = i0 + ii;
                const int64_t rw = i < top_k && s_row[i] >= 0 ? s_row[i] : 0;  // row 0 stands in; dropped below
#pragma unroll
                for (int j = 0; j < RM_VPT; j++) {
                    const int d = d0 + RM_COMBINE_THREADS * j;
                    yv[ii][j] = y[rw * dim + (d < dim ? d : dim - 1)];
                }
            }
#pragma unroll
            for (int ii = 0; ii < RM_KB; ii++) {
                const int i = i0 + ii;
                if (i >= top_k || s_row[i] < 0 || f[i].mant == 0) continue;  // uniform
#pragma unroll
                for (int j = 0; j < RM_VPT; j++)
                    acc[j] = wadd(acc[j], wmul(s_ec[i], sc_apply_i32(f[i], s_fast[i], yv[ii][j])));
            }
        }
    };
    const int span = RM_COMBINE_THREADS * RM_VPT;
    int64_t hv[RM_VPT];
    int64_t m = 0;
    if (live)
        for (int d0 = threadIdx.x; d0 < dim; d0 += span) {
            sums(d0, hv);
#pragma unroll
            for (int j = 0; j < RM_VPT; j++)
                if (d0 + RM_COMBINE_THREADS * j < dim) m = iabs(hv[j]) > m ? iabs(hv[j]) : m;
        }
    const int64_t gmax = block_max_t(m, red);
    const RqDen rd_gmax = rq_den(gmax);
    const bool held = dim <= span;  // hv still holds this thread's sums
    for (int d0 = threadIdx.x; d0 < dim; d0 += span) {
        if (gmax && !held) sums(d0, hv);
#pragma unroll
        for (int j = 0; j < RM_VPT; j++) {
            const int d = d0 + RM_COMBINE_THREADS * j;
            if (d < dim) out[(int64_t)t * dim + d] = gmax ? rq_apply(rd_gmax, hv[j]) : 0;
        }
    }
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
    const RqDen rd_gmax = rq_den(gmax);
    for (int64_t i = (int64_t)blockIdx.x * RQ_THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * RQ_THREADS)
        out[i] = gmax ? rq_apply(rd_gmax, sc_apply(fac[i / dim], rows[i])) : 0;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        put_rec(os, gmax ? sc_mul(from_ratio((u128)(uint64_t)gmax, (u128)ACT_LEVELS), *common) : Sc{0, 0});
}

// The workspace: the tiled activation planes, the i64 partial products (one slice per k run), the row records, the
// sanitized offsets with each group's first tile, the tile table.
size_t rq_workspace_bytes(int64_t rows, int64_t in, int64_t out, int64_t groups, size_t off[5]) {
    const int64_t kp = (in + 63) / 64 * 64;
    const int S = rq_splits(rows, groups, out, kp, kt_hip_flush_k(3, 3));  // the smallest flush bound: most runs
    const size_t cap = (size_t)rq_tile_cap(rows, groups);
    const size_t sizes[5] = {cap * RQ_BM * 3 * (size_t)kp, (size_t)S * (size_t)rows * (size_t)out * 8,
                             (size_t)rows * sizeof(RqState), (size_t)(groups + 1) * 8 + (size_t)groups * 4,
                             16 + 8 * cap};
    size_t at = 0;
    for (int i = 0; i < 5; i++) {
        off[i] = at;
        at += (sizes[i] + 255) / 256 * 256;
    }
    return at;
}

template <int PW>
static hipError_t rq_product(const int8_t* xa, int64_t rows, int64_t kp, const int8_t* wb, size_t wgroup,
                             int64_t* acc, int64_t N, const int64_t* off_s, const int2* em, const int32_t* hdr,
                             int64_t cap, int S, hipStream_t s) {
    using R = RqRing<PW>;
    int dev = 0, mx = 0;  // the ring must fit one CTA's LDS (160 KB on gfx950)
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || R::LDS > mx)
        return hipErrorInvalidConfiguration;
    const int64_t ntile = (N + RQ_BN - 1) / RQ_BN, nkt = kp / RQ_BK, per = (nkt + S - 1) / S;
    rq_gemm_kernel<PW><<<(unsigned)(ntile * cap * S), 256, R::LDS, s>>>(xa, rows, kp, wb, wgroup, acc, (int)N, off_s,
                                                                       em, hdr, (int)cap, (int)ntile, (int)per);
    return hipGetLastError();
}

hipError_t launch_quant_linear_rows(const int32_t* x, const int32_t* xidx, int64_t x_rows, int64_t rows, int64_t in,
                                    const kt_hip_qscale* xs, int xs_step, int groups, const int64_t* off_dev,
                                    const int8_t* wb, size_t wgroup, int pw, int64_t out, const int64_t* wm_dev,
                                    const int32_t* wsh_dev, int64_t flush_k, void* ws, int32_t* y, kt_hip_qscale* ys,
                                    hipStream_t s) {
    size_t off[5];
    rq_workspace_bytes(rows, in, out, groups, off);
    const int64_t cap = rq_tile_cap(rows, groups), kp = (in + 63) / 64 * 64;
    const int S = rq_splits(rows, groups, out, kp, flush_k);
    char* base = (char*)ws;
    int8_t* xa = (int8_t*)(base + off[0]);
    int64_t* acc = (int64_t*)(base + off[1]);
    RqState* st = (RqState*)(base + off[2]);
    int64_t* off_s = (int64_t*)(base + off[3]);
    int32_t* tb = (int32_t*)(off_s + groups + 1);
    int32_t* hdr = (int32_t*)(base + off[4]);
    int2* em = (int2*)(hdr + 4);
    rq_plan_kernel<<<1, 1024, 0, s>>>(off_dev, groups, rows, off_s, tb, hdr, em, cap);
    rq_quant_kernel<<<(unsigned)rows, RQ_ROW_THREADS, 0, s>>>(x, xidx, x_rows, in, kp, xs, xs_step, groups, off_s,
                                                              tb, cap, wm_dev, wsh_dev, st, xa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = pw == 1   ? rq_product<1>(xa, rows, kp, wb, wgroup, acc, out, off_s, em, hdr, cap, S, s)
        : pw == 3 ? rq_product<3>(xa, rows, kp, wb, wgroup, acc, out, off_s, em, hdr, cap, S, s)
                  : rq_product<5>(xa, rows, kp, wb, wgroup, acc, out, off_s, em, hdr, cap, S, s);
    if (e != hipSuccess) return e;
    rq_requant_kernel<<<(unsigned)rows, RQ_ROW_THREADS, 0, s>>>(acc, rows, out, S, st, y, ys);
    return hipGetLastError();
}

size_t rq_tiled_bytes(int64_t rows, int64_t k, int p) {
    return (size_t)((rows + RQ_BN - 1) / RQ_BN) * RQ_BN * (size_t)((k + 63) / 64 * 64) * (size_t)p;
}

hipError_t launch_rq_pack_tiled(const int32_t* codes, int64_t rows, int64_t k, int p, int8_t* out, hipStream_t s) {
    const int64_t chunks = (int64_t)(rq_tiled_bytes(rows, k, p) / 16);
    rq_pack_tiled_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, s>>>(codes, rows, k, (k + 63) / 64 * 64, p, out);
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
    // the grouped product addresses one tile's and one weight block's k-steps with 32-bit offsets
    if (w_group_bytes < kt::rq_tiled_bytes(out_f, in_f, pw) || (int64_t)pw * kt::RQ_BN * kp >= ((int64_t)1 << 32))
        return (int)hipErrorInvalidValue;
    const int64_t S = kt::rq_splits(rows, groups, out_f, kp, kt_hip_flush_k(3, pw));
    if (((out_f + kt::RQ_BN - 1) / kt::RQ_BN) * kt::rq_tile_cap(rows, groups) * S > INT32_MAX)
        return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_quant_linear_rows(x_dev, xidx_dev, x_rows, rows, in_f, xs_dev, xs_step, (int)groups,
                                             off_dev, w_planes_dev, w_group_bytes, pw, out_f, w_mant_dev, w_shift_dev,
                                             kt_hip_flush_k(3, pw), ws_dev, y_dev, ys_dev, (hipStream_t)stream);
}

extern "C" size_t kt_hip_pack_planes_tiled_bytes(int64_t rows, int64_t k, int planes) {
    if (rows < 1 || k < 1 || (planes != 1 && planes != 3 && planes != 5)) return 0;
    return kt::rq_tiled_bytes(rows, k, planes);
}

extern "C" int kt_hip_pack_planes_tiled(int dev, const int32_t* codes_dev, int64_t rows, int64_t k, int planes,
                                        int8_t* planes_dev, void* stream) {
    if (!codes_dev || !planes_dev || rows < 1 || k < 1 || (planes != 1 && planes != 3 && planes != 5) ||
        rows > INT32_MAX || k > INT32_MAX || kt::rq_tiled_bytes(rows, k, planes) / 16 > (size_t)UINT32_MAX * 256)
        return (int)hipErrorInvalidValue;
    RM_TRY(hipSetDevice(dev));
    return (int)kt::launch_rq_pack_tiled(codes_dev, rows, k, planes, planes_dev, (hipStream_t)stream);
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
