// QuantLinear::forward_int (crates/01-engine/kt-core/src/layers.rs:275-328) with every pass on the device: the
// reference's dynamic per-tensor quantization around the exact digit-plane GEMM, for i32 activation codes at any
// scale and weight codes held as base-256 digit planes. Four launches:
//
//   ql_absmax   partial maxima of |x|                                                    (xmax, layers.rs:279)
//   ql_quant    xmax from the partials, qx = quant_to(x, xmax) (layers.rs:23-31) split straight into 3 balanced
//               base-256 planes; CTA 0 also forms the Scale products c = from_ratio(xmax, WLEVELS) * xs * ws and
//               the bias factor f = bs * c^-1 in one thread (128-bit integer arithmetic, kt-int/src/lib.rs:191-280)
//   plane GEMM  acc = qx . w^T in i64 (kt_kernels.hip, plane_gemm_kernel), whose epilogue adds f.apply(bias[o])
//               and raises the call's max |acc| (layers.rs:304-321)
//   ql_requant  y = requant_dyn(acc, ACT_LEVELS, ymax) and the output scale (layers.rs:33-39, 321-327)
//
// Conv2d::forward_int (conv.rs:68-130) runs the same passes over the image's im2col rows: max |x| over the whole
// image, the patch gathered inside ql_quant (taps in the padding are zero, which the direct conv skips), the bias
// and gmax in the GEMM epilogue, and ql_requant_conv storing the output channel-major through an LDS transpose.
//
// No host synchronization: the maxima and the scales stay in the workspace, and the output scale is written to a
// device record the next layer reads as its input scale. Integer arithmetic only, except a double-precision
// quotient estimate in ql_requant and ql_quant that is corrected to the exact integer quotient before use (the
// quotients are below 2^29, where the estimate is within one of the exact value).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <vector>

#include "kt_dpp.h"
#include "kt_kernels.h"
#include "kt_scale_dev.h"
#include "kt_w12_core.h"

namespace kt {

namespace {

constexpr int64_t WLEVELS = 265720;       // (3^12 - 1) / 2, layers.rs:16
constexpr int64_t ACT_LEVELS = 1LL << 28;  // layers.rs:18
constexpr int QL_THREADS = 256;
constexpr int64_t QL_FUSED_MAX = 8192;  // x of at most this many values: max |x| inside the quant pass

template <typename T>
__device__ inline T block_max(T v, T* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const T u = __shfl_xor(v, o, 64);
        v = u > v ? u : v;
    }
    if (lane == 0) red[wave] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) v = red[w] > v ? red[w] : v;
        red[0] = v;
    }
    __syncthreads();
    v = red[0];
    __syncthreads();
    return v;
}

}  // namespace

__global__ __launch_bounds__(QL_THREADS) void ql_absmax_kernel(const int32_t* __restrict__ x, int64_t n,
                                                               uint32_t* __restrict__ part) {
    __shared__ uint32_t red[QL_THREADS / 64];
    uint32_t m = 0;
    const int64_t step = (int64_t)gridDim.x * QL_THREADS;
    for (int64_t i0 = (int64_t)blockIdx.x * QL_THREADS + threadIdx.x; i0 < n; i0 += 4 * step) {  // 4 loads in flight
        int32_t v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = i0 + u * step < n ? x[i0 + u * step] : 0;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t a = v[u] < 0 ? 0u - (uint32_t)v[u] : (uint32_t)v[u];
            m = a > m ? a : m;
        }
    }
    m = block_max(m, red);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// The column values of output row r from column c0 on, 4 of them: row r of x itself, or for a convolution the
// im2col patch of output pixel r = oy * ow + ox, column c = (ic * kh + ky) * kw + kx (the weights' [co][ci][kh][kw]
// order), zero for a tap in the padding or a column past `in`.
template <bool CONV>
__device__ inline void ql_fetch4(const int32_t* __restrict__ x, int64_t r, int64_t c0, int64_t in, const ConvGeom& g,
                                 int32_t v[4]) {
    if (!CONV) {
#pragma unroll
        for (int t = 0; t < 4; t++) v[t] = c0 + t < in ? x[r * in + c0 + t] : 0;
        return;
    }
    const int khw = g.kh * g.kw;
    const int oy = (int)(r / g.ow), ox = (int)(r - (int64_t)oy * g.ow);
    int ic = (int)(c0 / khw), rem = (int)(c0 - (int64_t)ic * khw);
    int ky = rem / g.kw, kx = rem - ky * g.kw;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        int32_t val = 0;
        if (c0 + t < in) {
            const int iy = oy * g.stride + ky - g.pad, ix = ox * g.stride + kx - g.pad;
            if (iy >= 0 && iy < g.h && ix >= 0 && ix < g.w) val = x[((int64_t)ic * g.h + iy) * g.w + ix];
        }
        v[t] = val;
        if (++kx == g.kw) {
            kx = 0;
            if (++ky == g.kh) ky = 0, ic++;
        }
    }
}

// qx = quant_to(x, xmax) for 4 consecutive columns per thread, split into planes [3][rows][kp]; padding columns and
// the xmax == 0 case give zero digits. |qx| <= WLEVELS < 127 * (1 + 256 + 65536), so 3 balanced digits hold it.
// xmax is taken over the nx values of x (the whole image for a convolution).
// The weight and bias Scales of each output segment of a call (QlSeg; one segment for a single QuantLinear).
struct QlScales {
    int64_t w_mant[KT_QL_MAX_SEG], b_mant[KT_QL_MAX_SEG];
    int32_t w_shift[KT_QL_MAX_SEG], b_shift[KT_QL_MAX_SEG];
    int has_bias[KT_QL_MAX_SEG];
};
// Each segment's output codes and record.
struct QlOut {
    int32_t* y[KT_QL_MAX_SEG];
    kt_hip_qscale* os[KT_QL_MAX_SEG];
};

// A segment's Scale products for max |x| = m (layers.rs:279-303): c = from_ratio(m, WLEVELS) * xs * ws, the bias
// factor f = bs * c^-1, and the mode (0: normal; 1: m == 0, the output is the bias codes or zeros; 2: c == 0, zeros).
struct QlHead {
    int64_t xmax;
    Sc c, f;
    int mode;
};
__device__ inline QlHead ql_head(uint32_t m, const kt_hip_qscale* xs, const QlScales& sc, int g) {
    QlHead h{(int64_t)m, Sc{0, 0}, Sc{0, 0}, 0};
    if (m == 0) {
        h.mode = 1;
        return h;
    }
    h.c = sc_mul(sc_mul(from_ratio((u128)m, (u128)WLEVELS), Sc{xs->mant, xs->shift}), Sc{sc.w_mant[g], sc.w_shift[g]});
    if (h.c.mant == 0) h.mode = 2;
    else if (sc.has_bias[g]) h.f = sc_mul(Sc{sc.b_mant[g], sc.b_shift[g]}, sc_recip(h.c));
    return h;
}

// The three balanced base-256 digits of quant_to(x, xmax) for 4 columns (layers.rs:23-31), as one byte of each
// plane word. |x| <= xmax, so the quotient (|x| * WLEVELS + xmax / 2) / xmax is below 2^19; it is estimated as a
// product with rinv = 1 / xmax in double precision (relative error below 2^-51, so off by less than 2^-30 and at
// most one step from the exact floor) and the two integer tests restore the exact quotient.
__device__ inline void ql_digits4r(const int32_t xv[4], uint32_t xmax, double rinv, uint32_t word[3]) {
    const uint64_t half = xmax / 2;
    word[0] = word[1] = word[2] = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        int64_t v = 0;
        if (xv[t] != 0) {
            const int64_t num = (int64_t)xv[t] * WLEVELS;
            const uint64_t a = (uint64_t)(num < 0 ? -num : num) + half;
            uint64_t qq = (uint64_t)((double)a * rinv);
            if (qq * xmax > a) qq--;
            else if ((qq + 1) * xmax <= a) qq++;
            v = num >= 0 ? (int64_t)qq : -(int64_t)qq;
        }
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int64_t d = ((v + 128) & 255) - 128;
            word[p] |= ((uint32_t)d & 255u) << (8 * t);
            v = (v - d) >> 8;
        }
    }
}

template <bool CONV>
__global__ __launch_bounds__(QL_THREADS) void ql_quant_kernel(const int32_t* __restrict__ x, int64_t nx,
                                                              int64_t rows, int64_t in, int64_t kp, ConvGeom geom,
                                                              const uint32_t* __restrict__ part, int nparts,
                                                              const kt_hip_qscale* __restrict__ xs, QlSeg seg,
                                                              QlScales sc, QlState* __restrict__ st,
                                                              int8_t* __restrict__ xa, uint64_t* __restrict__ zacc,
                                                              int64_t nzacc, uint32_t* __restrict__ zcnt,
                                                              int nzcnt) {
    __shared__ uint32_t red[QL_THREADS / 64];
    {  // a split-k GEMM follows: its accumulators and per-tile arrival counters start at zero
        const int64_t i0 = (int64_t)blockIdx.x * QL_THREADS + threadIdx.x, st_ = (int64_t)gridDim.x * QL_THREADS;
        for (int64_t i = i0; i < nzacc; i += st_) zacc[i] = 0;
        for (int64_t i = i0; i < nzcnt; i += st_) zcnt[i] = 0;
    }
    uint32_t m = 0;
    if (nparts > 0) {
        for (int i = threadIdx.x; i < nparts; i += QL_THREADS) m = part[i] > m ? part[i] : m;
    } else {  // a short x (QL_FUSED_MAX values at most): every CTA takes max |x| itself, no ql_absmax pass
        for (int64_t i0 = threadIdx.x; i0 < nx; i0 += 8 * QL_THREADS) {  // 8 loads in flight per thread
            int32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = i0 + u * QL_THREADS < nx ? x[i0 + u * QL_THREADS] : 0;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t a = v[u] < 0 ? 0u - (uint32_t)v[u] : (uint32_t)v[u];
                m = a > m ? a : m;
            }
        }
    }
    m = block_max(m, red);
    if (blockIdx.x == 0 && threadIdx.x < KT_QL_YSLOTS * seg.n)
        st[threadIdx.x / KT_QL_YSLOTS].ymax[threadIdx.x % KT_QL_YSLOTS].v = 0;
    if (blockIdx.x == 0 && (int)threadIdx.x < seg.n) {  // each segment's record, for the GEMM epilogue and ql_requant
        const QlHead h = ql_head(m, xs, sc, threadIdx.x);
        QlState* q = st + threadIdx.x;
        q->xmax = h.xmax, q->c_mant = h.c.mant, q->f_mant = h.f.mant;
        q->c_shift = h.c.shift, q->f_shift = h.f.shift, q->mode = h.mode;
    }
    const int64_t quads = rows * (kp / 4);
    const bool live = m != 0;
    const double rinv = live ? 1.0 / (double)m : 0.0;
    const size_t plane = (size_t)rows * (size_t)kp;
    const int64_t qpr = kp / 4, q0 = (int64_t)blockIdx.x * QL_THREADS + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * QL_THREADS, dr = step / qpr, dq = step - dr * qpr;
    int64_t r = q0 / qpr, cq = q0 - r * qpr;  // (row, quad) of q, advanced incrementally
    for (int64_t q = q0; q < quads; q += step, r += dr, cq += dq) {
        if (cq >= qpr) cq -= qpr, r++;
        const int64_t c0 = cq * 4;
        uint32_t word[3] = {0, 0, 0};
        int32_t xv[4] = {0, 0, 0, 0};
        if (live) {
            ql_fetch4<CONV>(x, r, c0, in, geom, xv);
            ql_digits4r(xv, m, rinv, word);
        }
        const size_t at = (size_t)r * (size_t)kp + (size_t)c0;
#pragma unroll
        for (int p = 0; p < 3; p++) *reinterpret_cast<uint32_t*>(xa + p * plane + at) = word[p];
    }
}


// One row (the decode step): the quant pass and the digit product in one launch. Every CTA takes max |x| over the
// row and forms the row's three digit planes in LDS itself (at most MAXKP values, read from L2 by each CTA) while
// its first weight chunks are in flight, then runs the product of plane_skinny_kernel over its 8 output columns
// (4 waves x 2 columns, the lanes striding k in 16-byte chunks, int32 plane-group sums by sdot4, a butterfly across
// the wave). The CTA's largest |result| goes to its own slot part[blockIdx.x] (overwritten on every call, so no
// pass has to clear it); ql_requant_kernel takes each segment's maximum over its CTAs' slots. CTA 0 writes each
// segment's state for ql_requant_kernel. A CTA whose segment has a bias forms the bias factor itself. Requires
// kp <= MAXKP and a single k-chunk (kp within the flush bound). launch_ql_impl takes this path for outputs of at
// most QS_FUSED_OUT columns: rows up to QS_MAX_KP values, and for 3 weight planes rows up to QS_LONG_KP values in an
// instantiation with the larger LDS image (the 4864-value down row: 13.6 us against 8.8 + 9.0 for the quant pass and
// the product; the small instantiation keeps the short rows' registers and LDS low).
constexpr int QS_MAX_KP = 1024, QS_LONG_KP = 8192;
constexpr int64_t QS_FUSED_OUT = 16384;
constexpr int QS_THREADS = 256, QS_WAVES = QS_THREADS / 64;
constexpr int QS_CPW = 2;  // output columns per wave
constexpr int QS_COLS = QS_WAVES * QS_CPW;

template <int PW, int MAXKP>
__global__ __launch_bounds__(QS_THREADS) void ql_skinny_kernel(const int32_t* __restrict__ x, int in, int kp,
                                                               const kt_hip_qscale* __restrict__ xs,
                                                               const int8_t* __restrict__ wb, int64_t* __restrict__ y,
                                                               int N, const int64_t* __restrict__ bias, QlSeg seg,
                                                               QlScales sc, QlState* __restrict__ st,
                                                               int64_t* __restrict__ part) {
    constexpr int NG = 3 + PW - 1, QPT = MAXKP / 4 / QS_THREADS;
    __shared__ __attribute__((aligned(16))) int8_t xq[3 * MAXKP];
    __shared__ uint32_t red[QS_WAVES];
    __shared__ int64_t s_max[QS_WAVES];
    __shared__ int64_t s_f[2];  // the bias factor of this CTA's segment (mant, shift), when it has a bias
    __shared__ int s_badd;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = ((int)blockIdx.x * QS_WAVES + wave) * QS_CPW;  // the wave's first column
    const int g = ql_seg_of(seg, (int)blockIdx.x * QS_COLS);
    const size_t wplane = (size_t)N * kp;
    const int nch = kp / 16;

    // the weights of the wave's next chunk; non-temporal loads (read once per call), so the stream does not push the
    // small tensors the next launches read (the sums, the records, the cache rows) out of the caches
    v4i wn[QS_CPW][PW];
    auto wload = [&](int q) {
#pragma unroll
        for (int c = 0; c < QS_CPW; c++)
#pragma unroll
            for (int j = 0; j < PW; j++)
                wn[c][j] = q < nch && nb + c < N
                               ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(
                                     wb + j * wplane + (size_t)(nb + c) * kp + 16 * (size_t)q))
                               : v4i{};
    };
    wload(lane);  // in flight while the row is quantized

    // the row, 4 columns per quad, QPT quads per thread held in registers; max |x| over the CTA
    int32_t xv[QPT][4];
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int c0 = 4 * (tid + QS_THREADS * k);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            xv[k][t] = c0 + t < in ? x[c0 + t] : 0;
            const uint32_t a = xv[k][t] < 0 ? 0u - (uint32_t)xv[k][t] : (uint32_t)xv[k][t];
            m = a > m ? a : m;
        }
    }
    {  // max |x| over the CTA: each wave's by DPP, then the QS_WAVES of them
        m = wave_max_u32(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < QS_WAVES; w++) m = red[w] > m ? red[w] : m;
    }
    const double rinv = m != 0 ? 1.0 / (double)m : 0.0;
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int c0 = 4 * (tid + QS_THREADS * k);
        if (c0 < kp) {
            uint32_t word[3] = {0, 0, 0};
            if (m != 0) ql_digits4r(xv[k], m, rinv, word);
#pragma unroll
            for (int p = 0; p < 3; p++) *reinterpret_cast<uint32_t*>(xq + p * kp + c0) = word[p];
        }
    }
    if (blockIdx.x == 0 && tid < seg.n) {  // each segment's state, for ql_requant_kernel
        const QlHead h = ql_head(m, xs, sc, tid);
        QlState* q = st + tid;
        q->xmax = h.xmax, q->c_mant = h.c.mant, q->f_mant = h.f.mant;
        q->c_shift = h.c.shift, q->f_shift = h.f.shift, q->mode = h.mode;
    }
    if (tid == 0) {
        int badd = 0;
        if (bias && sc.has_bias[g]) {
            const QlHead h = ql_head(m, xs, sc, g);
            badd = h.mode == 0;
            s_f[0] = h.f.mant, s_f[1] = h.f.shift;
        }
        s_badd = badd;
    }
    __syncthreads();

    int acc[QS_CPW][NG];
#pragma unroll
    for (int c = 0; c < QS_CPW; c++)
#pragma unroll
        for (int i = 0; i < NG; i++) acc[c][i] = 0;
    for (int q = lane; q < nch; q += 64) {
        v4i wv[QS_CPW][PW];
#pragma unroll
        for (int c = 0; c < QS_CPW; c++)
#pragma unroll
            for (int j = 0; j < PW; j++) wv[c][j] = wn[c][j];
        wload(q + 64);
        v4i xd[3];
#pragma unroll
        for (int i = 0; i < 3; i++) xd[i] = *reinterpret_cast<const v4i*>(xq + i * kp + 16 * q);
#pragma unroll
        for (int c = 0; c < QS_CPW; c++)
#pragma unroll
            for (int i = 0; i < 3; i++)
#pragma unroll
                for (int j = 0; j < PW; j++) {
                    int d = acc[c][i + j];
#pragma unroll
                    for (int e = 0; e < 4; e++) d = __builtin_amdgcn_sdot4(xd[i][e], wv[c][j][e], d, false);
                    acc[c][i + j] = d;
                }
    }
#pragma unroll
    for (int c = 0; c < QS_CPW; c++)
#pragma unroll
        for (int i = 0; i < NG; i++) acc[c][i] = wave_sum_i32(acc[c][i]);  // the wave's sums, in every lane
    int64_t lmax = 0;
    if (lane == 0) {
        const bool badd = s_badd != 0;
#pragma unroll
        for (int c = 0; c < QS_CPW; c++) {
            const int n = nb + c;
            if (n >= N) continue;
            uint64_t f = badd ? (uint64_t)scale_apply(s_f[0], (int32_t)s_f[1], bias[n]) : 0;
#pragma unroll
            for (int i = 0; i < NG; i++) f += (uint64_t)(int64_t)acc[c][i] << (8 * i);  // NG <= 7: 8 i < 64
            y[n] = (int64_t)f;
            const int64_t a = (int64_t)f < 0 ? (int64_t)(0 - f) : (int64_t)f;  // i64::abs, wrapping
            lmax = a > lmax ? a : lmax;
        }
        s_max[wave] = lmax;
    }
    __syncthreads();
    if (tid == 0) {
        int64_t b = s_max[0];
        for (int w = 1; w < QS_WAVES; w++) b = s_max[w] > b ? s_max[w] : b;
        part[blockIdx.x] = b > 0 ? b : 0;
    }
}

// y = requant_dyn(acc, ACT_LEVELS, ymax) per segment (layers.rs:33-39, 321-327). The grid's last CTA only writes
// each segment's record (its Scale products run beside the other CTAs' divisions); the others requantize. Each
// thread's first accumulator and the segments' states are read before the maximum is known. The maximum comes from
// the state's slots, or with `part` from the one-row product's maximum per CTA of QS_COLS columns.
__global__ __launch_bounds__(QL_THREADS) void ql_requant_kernel(const int64_t* __restrict__ acc, int64_t n,
                                                                int64_t out, const int64_t* __restrict__ bias,
                                                                const QlState* __restrict__ st, QlSeg seg,
                                                                QlScales sc, QlOut yo,
                                                                const int64_t* __restrict__ part, int nparts) {
    __shared__ int64_t s_ymax[KT_QL_MAX_SEG];
    __shared__ double s_rinv[KT_QL_MAX_SEG];
    __shared__ int32_t s_mode[KT_QL_MAX_SEG];
    __shared__ unsigned long long s_pmax[KT_QL_MAX_SEG];
    const bool rec_cta = blockIdx.x == gridDim.x - 1;
    const int tid = threadIdx.x;
    const int64_t i0 = (int64_t)blockIdx.x * QL_THREADS + tid, step = (int64_t)(gridDim.x - 1) * QL_THREADS;
    const int64_t a_first = !rec_cta && i0 < n ? acc[i0] : 0;
    int mode = 0;
    int64_t xmax = 0, c_mant = 0;
    int32_t c_shift = 0;
    if (tid < seg.n) {
        const QlState* q = st + tid;
        mode = q->mode, xmax = q->xmax, c_mant = q->c_mant, c_shift = q->c_shift;
    }
    int64_t ymax = 0;
    if (part) {  // each segment's maximum over its CTAs' slots
        if (tid < KT_QL_MAX_SEG) s_pmax[tid] = 0;
        __syncthreads();
        unsigned long long pm[KT_QL_MAX_SEG] = {};
        for (int c0 = tid; c0 < nparts; c0 += 4 * QL_THREADS) {  // 4 loads in flight per thread
            unsigned long long v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int c = c0 + u * QL_THREADS;
                v[u] = c < nparts ? (unsigned long long)part[c] : 0;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int g = ql_seg_of(seg, (c0 + u * QL_THREADS) * QS_COLS);
#pragma unroll
                for (int i = 0; i < KT_QL_MAX_SEG; i++)
                    if (i == g) pm[i] = v[u] > pm[i] ? v[u] : pm[i];
            }
        }
#pragma unroll
        for (int i = 0; i < KT_QL_MAX_SEG; i++) {
            if (i >= seg.n) break;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const unsigned long long u = __shfl_xor(pm[i], o);
                pm[i] = u > pm[i] ? u : pm[i];
            }
            if ((tid & 63) == 0 && pm[i] != 0) atomicMax(&s_pmax[i], pm[i]);
        }
        __syncthreads();
        if (tid < seg.n) ymax = (int64_t)s_pmax[tid];
    } else if (tid < seg.n) {
        const QlState* q = st + tid;
#pragma unroll
        for (int i = 0; i < KT_QL_YSLOTS; i++) ymax = (int64_t)q->ymax[i].v > ymax ? (int64_t)q->ymax[i].v : ymax;
    }
    if (rec_cta) {  // each segment's record
        if (tid < seg.n) {
            const int g = tid;
            kt_hip_qscale o{};
            o.xmax = xmax;
            if (mode == 1) {
                if (sc.has_bias[g]) o.mant = sc.b_mant[g], o.shift = sc.b_shift[g];
            } else if (mode == 0 && ymax > 0) {
                const Sc s2 = sc_mul(from_ratio((u128)(uint64_t)ymax, (u128)ACT_LEVELS), Sc{c_mant, c_shift});
                o.mant = s2.mant, o.shift = s2.shift, o.ymax = ymax;
            }
            *yo.os[g] = o;
        }
        return;
    }
    if (tid < seg.n) s_ymax[tid] = ymax, s_mode[tid] = mode, s_rinv[tid] = rq_den(ymax).rinv;
    __syncthreads();
    const int64_t dstep = step % out, rstep = step / out;
    int64_t o = i0 % out, r = i0 / out;  // (row, column) of i, advanced incrementally
    for (int64_t i = i0; i < n; i += step, r += rstep, o += dstep) {
        if (o >= out) o -= out, r++;
        const int g = ql_seg_of(seg, (int)o);
        const int64_t ym = s_ymax[g];
        const int md = s_mode[g];
        int32_t v32 = 0;
        if (md == 1) {
            v32 = sc.has_bias[g] && bias ? (int32_t)bias[o] : 0;
        } else if (md == 0 && ym > 0) {  // requant_dyn(v, 2^28, ymax)
            v32 = rq_apply(RqDen{ym, (uint64_t)(ym / 2), s_rinv[g]}, i == i0 ? a_first : acc[i]);
        }
        const int64_t w = seg.col0[g + 1] - seg.col0[g];
        yo.y[g][r * w + (o - seg.col0[g])] = v32;
    }
}

// Conv2d::forward_int's close (conv.rs:121-129): y = requant_dyn(acc, ACT_LEVELS, gmax) stored channel-major,
// y[o * rows + r] for acc[r * out + o], through a 64 x 64 LDS tile so that both the acc reads and the y writes are
// row-contiguous. An all-zero image (mode 1), c == 0 (mode 2) and gmax == 0 give zeros at Scale::ZERO.
__global__ __launch_bounds__(QL_THREADS) void ql_requant_conv_kernel(const int64_t* __restrict__ acc, int64_t rows,
                                                                     int64_t out, const QlState* __restrict__ st,
                                                                     int32_t* __restrict__ y,
                                                                     kt_hip_qscale* __restrict__ os) {
    __shared__ int32_t tile[64][65];
    int64_t ymax = 0;
#pragma unroll
    for (int i = 0; i < KT_QL_YSLOTS; i++) ymax = (int64_t)st->ymax[i].v > ymax ? (int64_t)st->ymax[i].v : ymax;
    const bool live = st->mode == 0 && ymax > 0;
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
        kt_hip_qscale o{};
        o.xmax = st->xmax;
        if (live) {
            const Sc sc = sc_mul(from_ratio((u128)(uint64_t)ymax, (u128)ACT_LEVELS), Sc{st->c_mant, st->c_shift});
            o.mant = sc.mant, o.shift = sc.shift, o.ymax = ymax;
        }
        *os = o;
    }
    const RqDen rd = rq_den(ymax);
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * 64, o0 = (int64_t)blockIdx.y * 64;
    for (int rr = ty; rr < 64; rr += QL_THREADS / 64) {
        const int64_t r = r0 + rr, o = o0 + tx;
        int32_t q32 = 0;
        if (live && r < rows && o < out) {
            q32 = rq_apply(rd, acc[r * out + o]);
        }
        tile[tx][rr] = q32;
    }
    __syncthreads();
    for (int oo = ty; oo < 64; oo += QL_THREADS / 64) {
        const int64_t o = o0 + oo, r = r0 + tx;
        if (o < out && r < rows) y[o * rows + r] = tile[oo][tx];
    }
}

size_t ql_workspace_bytes(int64_t rows, int64_t in, int64_t out, size_t off[KT_QL_WS_PARTS]) {
    const size_t kp = (size_t)((in + 63) / 64 * 64);
    // part 2: the partial maxima of |x|, or for one row the product's maximum per CTA of QS_COLS columns
    const size_t pmax = rows == 1 ? (size_t)((out + QS_COLS - 1) / QS_COLS) * 8 : 0;
    const size_t sizes[KT_QL_WS_PARTS] = {3 * (size_t)rows * kp, (size_t)rows * (size_t)out * 8,
                                          pmax > KT_QL_PARTS * 4 ? pmax : KT_QL_PARTS * 4, KT_QL_PARTS * 8,
                                          KT_QL_MAX_SEG * sizeof(QlState)};
    size_t at = 0;
    for (int i = 0; i < KT_QL_WS_PARTS; i++) {
        off[i] = at;
        at += (sizes[i] + 255) / 256 * 256;
    }
    return at;
}

// The workspace of kt_hip_quant_linear_noalloc: one copy per GPU, resident from the code object's load until the
// process ends. Host code never passes this name to a kernel (on the host it is a stand-in, not a device address):
// it uses the address ql_scratch looked up for the current device.
static __device__ __align__(256) uint8_t scratch[KT_QL_SCRATCH_BYTES];

// The lookup is a runtime call outside any stream; a first call whose stream is being captured into a graph is
// refused (hipErrorStreamCaptureUnsupported) rather than making it there: one eager call per device comes first.
hipError_t ql_scratch(int dev, void** ptr, hipStream_t s) {
    static std::mutex mu;
    static std::vector<void*> addr;  // per device, filled on the device's first call
    *ptr = nullptr;
    if (dev < 0) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(mu);
    if ((size_t)dev >= addr.size()) addr.resize((size_t)dev + 1, nullptr);
    if (!addr[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        const hipError_t ce = hipStreamIsCapturing(s, &cs);
        if (ce != hipSuccess) return ce;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

static int grid_for(int64_t n, int64_t per_thread) {
    const int64_t g = (n + QL_THREADS * per_thread - 1) / (QL_THREADS * per_thread);
    return (int)(g < 1 ? 1 : (g > KT_QL_PARTS ? KT_QL_PARTS : g));
}

// Whether one row of in values -> out columns takes the one-launch product (ql_skinny_kernel): the row within one
// k-chunk and the kernel's LDS image, at most QS_FUSED_OUT columns.
bool ql_sums_ok(int64_t in, int64_t out, int pw, int64_t flush_k) {
    const int64_t kp = (in + 63) / 64 * 64;
    const bool long_row = kp > QS_MAX_KP && kp <= QS_LONG_KP && pw == 3;
    return in >= 1 && out >= 1 && (kp <= QS_MAX_KP || long_row) && out <= QS_FUSED_OUT && kp <= flush_k &&
           (pw == 1 || pw == 3 || pw == 5);
}
// every CTA of QS_COLS columns within one segment
static bool ql_seg_cols_ok(const QlSeg& seg) {
    bool ok = true;
    for (int g = 1; g < seg.n; g++) ok = ok && seg.col0[g] % QS_COLS == 0;
    return ok;
}
// The one-row product (ql_sums_ok): the sums at the workspace's part 1, each segment's state at part 4, each CTA's
// largest |sum| at part 2.
static hipError_t launch_ql_skinny(const int32_t* x, int64_t in, const kt_hip_qscale* xs, const int8_t* wb, int pw,
                                   int64_t out, const QlSeg& seg, const QlScales& sc, const int64_t* bias, void* ws,
                                   hipStream_t s) {
    size_t off[KT_QL_WS_PARTS];
    ql_workspace_bytes(1, in, out, off);
    char* base = (char*)ws;
    int64_t* acc = (int64_t*)(base + off[1]);
    int64_t* pm = reinterpret_cast<int64_t*>(base + off[2]);
    QlState* st = (QlState*)(base + off[4]);
    const int64_t kp = (in + 63) / 64 * 64;
    const bool long_row = kp > QS_MAX_KP && kp <= QS_LONG_KP && pw == 3;
    const int ctas = (int)((out + QS_COLS - 1) / QS_COLS);
#define KT_QS(P, K) ql_skinny_kernel<P, K><<<ctas, QS_THREADS, 0, s>>>(x, (int)in, (int)kp, xs, wb, acc, (int)out, bias, \
                                                                      seg, sc, st, pm)
    if (long_row) KT_QS(3, QS_LONG_KP);
    else if (pw == 1) KT_QS(1, QS_MAX_KP);
    else if (pw == 3) KT_QS(3, QS_MAX_KP);
    else KT_QS(5, QS_MAX_KP);
#undef KT_QS
    return hipGetLastError();
}

// The four passes of QuantLinear::forward_int, or of Conv2d::forward_int when geom is non-null (the image x of
// geom->ci x h x w values read as its im2col rows; the output channel-major, zeros at Scale::ZERO for an all-zero
// image). seg splits the out columns into the outputs of several calls on the same x (their own weight and bias
// Scales in sc, their own maximum, requantization and record): the x pass is shared and the digit GEMM runs once
// over the side-by-side weights.
static hipError_t launch_ql_impl(const int32_t* x, int64_t rows, int64_t in, const ConvGeom* geom,
                                 const kt_hip_qscale* xs, const int8_t* wb, int pw, int64_t out, const QlSeg& seg,
                                 const QlScales& sc, const int64_t* bias, int64_t flush_k, void* ws, const QlOut& yo,
                                 hipStream_t s) {
    size_t off[KT_QL_WS_PARTS];
    ql_workspace_bytes(rows, in, out, off);
    char* base = (char*)ws;
    int8_t* xa = (int8_t*)(base + off[0]);
    int64_t* acc = (int64_t*)(base + off[1]);
    uint32_t* part_x = (uint32_t*)(base + off[2]);
    uint32_t* tile_cnt = (uint32_t*)(base + off[3]);  // the split-k GEMM's per-tile arrival counters
    QlState* st = (QlState*)(base + off[4]);
    const int64_t kp = (in + 63) / 64 * 64, n = rows * out;
    const int64_t nx = geom ? (int64_t)geom->ci * geom->h * geom->w : rows * in;
    // one k-chunk whose tiles leave CUs idle (the decode row, N = 896 at M = 512): split k across CTAs
    const int splits = kp <= flush_k ? plane_gemm_splits(3, pw, (int)rows, (int)out, 0, (int)kp) : 1;
    const int ntiles = splits > 1 ? (int)(((out + 63) / 64) * ((rows + 63) / 64)) : 0;
    if (ntiles * 4 > KT_QL_PARTS * 8) return hipErrorInvalidValue;  // cannot happen: a split grid has < 128 tiles

    // one row within one k-chunk (the decode step): the quant pass inside the product, then the requant pass
    if (!geom && rows == 1 && ql_sums_ok(in, out, pw, flush_k) && ql_seg_cols_ok(seg)) {
        const hipError_t e = launch_ql_skinny(x, in, xs, wb, pw, out, seg, sc, bias, ws, s);
        if (e != hipSuccess) return e;
        const int ctas = (int)((out + QS_COLS - 1) / QS_COLS);
        int64_t* pm = reinterpret_cast<int64_t*>(base + off[2]);
        ql_requant_kernel<<<grid_for(n, 1) + 1, QL_THREADS, 0, s>>>(acc, n, out, bias, st, seg, sc, yo, pm, ctas);
        return hipGetLastError();
    }
    // max |x| by its own pass, or inside every quant CTA when x is short (one launch fewer for a decode row)
    const int gx = nx <= QL_FUSED_MAX ? 0 : grid_for(nx, 8);
    if (gx > 0) ql_absmax_kernel<<<gx, QL_THREADS, 0, s>>>(x, nx, part_x);
    uint64_t* zacc = splits > 1 ? reinterpret_cast<uint64_t*>(acc) : nullptr;
    const int64_t nzacc = splits > 1 ? n : 0;
    const int gq = grid_for(rows * kp / 4, 1);
    if (geom)
        ql_quant_kernel<true><<<gq, QL_THREADS, 0, s>>>(x, nx, rows, in, kp, *geom, part_x, gx, xs, seg, sc, st, xa,
                                                        zacc, nzacc, tile_cnt, ntiles);
    else
        ql_quant_kernel<false><<<gq, QL_THREADS, 0, s>>>(x, nx, rows, in, kp, ConvGeom{}, part_x, gx, xs, seg, sc, st,
                                                         xa, zacc, nzacc, tile_cnt, ntiles);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    for (int64_t k0 = 0; k0 < kp; k0 += flush_k) {
        const int64_t k1 = kp - k0 < flush_k ? kp : k0 + flush_k;
        const bool last = k1 == kp;
        e = launch_plane_gemm(3, pw, xa, wb, acc, (int)rows, (int)out, (int)kp, (int)k0, (int)k1, k0 > 0, 0, s,
                              last ? bias : nullptr, last ? st : nullptr, splits, tile_cnt, &seg);
        if (e != hipSuccess) return e;
    }
    if (geom) {
        const dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((out + 63) / 64));
        ql_requant_conv_kernel<<<grid, QL_THREADS, 0, s>>>(acc, rows, out, st, yo.y[0], yo.os[0]);
        return hipGetLastError();
    }
    // one output per thread for short outputs (a decode row: its divisions then run side by side, not 8 in a row)
    ql_requant_kernel<<<grid_for(n, n <= 65536 ? 1 : 2) + 1, QL_THREADS, 0, s>>>(acc, n, out, bias, st, seg, sc, yo,
                                                                                 nullptr, 0);
    return hipGetLastError();
}

static void ql_one(int64_t out, int64_t w_mant, int32_t w_shift, const int64_t* bias, int64_t b_mant,
                   int32_t b_shift, int32_t* y, kt_hip_qscale* os, QlSeg& seg, QlScales& sc, QlOut& yo) {
    seg = QlSeg{1, {0, (int)out, (int)out, (int)out, (int)out}};
    sc = QlScales{};
    sc.w_mant[0] = w_mant, sc.w_shift[0] = w_shift, sc.has_bias[0] = bias != nullptr;
    sc.b_mant[0] = b_mant, sc.b_shift[0] = b_shift;
    yo = QlOut{};
    yo.y[0] = y, yo.os[0] = os;
}

hipError_t launch_quant_linear(const int32_t* x, int64_t rows, int64_t in, const kt_hip_qscale* xs,
                               const int8_t* wb, int pw, int64_t out, int64_t w_mant, int32_t w_shift,
                               const int64_t* bias, int64_t b_mant, int32_t b_shift, int64_t flush_k, void* ws,
                               int32_t* y, kt_hip_qscale* os, hipStream_t s) {
    QlSeg seg;
    QlScales sc;
    QlOut yo;
    ql_one(out, w_mant, w_shift, bias, b_mant, b_shift, y, os, seg, sc, yo);
    return launch_ql_impl(x, rows, in, nullptr, xs, wb, pw, out, seg, sc, bias, flush_k, ws, yo, s);
}

hipError_t launch_quant_linear_multi(const int32_t* x, int64_t rows, int64_t in, const kt_hip_qscale* xs,
                                     const int8_t* wb, int pw, int nseg, const int64_t* seg_out,
                                     const int64_t* w_mant, const int32_t* w_shift, const int64_t* bias,
                                     const int* has_bias, const int64_t* b_mant, const int32_t* b_shift,
                                     int64_t flush_k, void* ws, int32_t* const* y, kt_hip_qscale* os,
                                     hipStream_t s) {
    QlSeg seg{nseg, {0, 0, 0, 0, 0}};
    QlScales sc{};
    QlOut yo{};
    int64_t at = 0;
    for (int g = 0; g < nseg; g++) {
        seg.col0[g] = (int)at;
        at += seg_out[g];
        sc.w_mant[g] = w_mant[g], sc.w_shift[g] = w_shift[g], sc.has_bias[g] = bias && has_bias[g];
        sc.b_mant[g] = sc.has_bias[g] ? b_mant[g] : 0, sc.b_shift[g] = sc.has_bias[g] ? b_shift[g] : 0;
        yo.y[g] = y[g], yo.os[g] = os + g;
    }
    for (int g = nseg; g <= KT_QL_MAX_SEG; g++) seg.col0[g] = (int)at;
    return launch_ql_impl(x, rows, in, nullptr, xs, wb, pw, at, seg, sc, bias, flush_k, ws, yo, s);
}

hipError_t launch_quant_linear_sums(const int32_t* x, int64_t in, const kt_hip_qscale* xs, const int8_t* wb, int pw,
                                    int nseg, const int64_t* seg_out, const int64_t* w_mant, const int32_t* w_shift,
                                    int64_t flush_k, void* ws, hipStream_t s) {
    QlSeg seg{nseg, {0, 0, 0, 0, 0}};
    QlScales sc{};
    int64_t at = 0;
    for (int g = 0; g < nseg; g++) {
        seg.col0[g] = (int)at;
        at += seg_out[g];
        sc.w_mant[g] = w_mant[g], sc.w_shift[g] = w_shift[g];
    }
    for (int g = nseg; g <= KT_QL_MAX_SEG; g++) seg.col0[g] = (int)at;
    if (!ql_sums_ok(in, at, pw, flush_k) || !ql_seg_cols_ok(seg)) return hipErrorInvalidValue;
    return launch_ql_skinny(x, in, xs, wb, pw, at, seg, sc, nullptr, ws, s);
}

hipError_t launch_ref_conv2d(const int32_t* x, const ConvGeom& g, const kt_hip_qscale* xs, const int8_t* wb, int pw,
                             int64_t co, int64_t w_mant, int32_t w_shift, const int64_t* bias, int64_t b_mant,
                             int32_t b_shift, int64_t flush_k, void* ws, int32_t* y, kt_hip_qscale* os,
                             hipStream_t s) {
    QlSeg seg;
    QlScales sc;
    QlOut yo;
    ql_one(co, w_mant, w_shift, bias, b_mant, b_shift, y, os, seg, sc, yo);
    return launch_ql_impl(x, (int64_t)g.oh * g.ow, (int64_t)g.ci * g.kh * g.kw, &g, xs, wb, pw, co, seg, sc, bias,
                          flush_k, ws, yo, s);
}

}  // namespace kt
