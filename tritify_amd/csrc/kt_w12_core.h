// Device building blocks shared by the gfx950 kernels: MFMA wrappers, LDS swizzle, raw buffer loads, the exact
// requant epilogue arithmetic, and the W12 tile mainloop that the dense, grouped (MoE) and im2col GEMMs all run.
//
// W12 (int8 activations x 12-bit weight codes in [-2048, 2047]): lo = (v & 255) - 128 (int8) and
// hi = (v + 2048) >> 8 (4 bits), v = lo + 256*hi - 1920, so sum_k x*v = S_lo + 256*S_hi - 1920*sum_k x.
// The weights are stored fragment-tiled: blocks of 32 rows x 32 k, each 64 lanes x (16 lo bytes + 8 nib bytes) in
// exactly the order one MFMA B operand takes them (lane l: row l%32, k = 16*(l/32) .. +16), so a wave fetches a B
// fragment with one fully coalesced 1 KB load and one 512-byte load, no LDS round trip. A lane's 8 nib bytes as
// dwords D0, D1 unpack in k order as D0 & 0x0F0F0F0F, (D0 >> 4) & .., D1 & .., (D1 >> 4) & .. . One 32-row column
// block is kp*32 lo bytes + kp*16 nib bytes, contiguous along k.
//
// MFMA: v_mfma_i32_32x32x32_i8 and v_mfma_i32_16x16x64_i8. A lane's 16 operand bytes are 16 consecutive k of one
// row (A) / one column (B); the hardware pairs A and B bytes with the same k-slot, so any lane->k assignment that is
// the same for A and B gives the exact dot product. The C layout of the 32x32 MFMA is lane l, register r -> row
// 8*(r/4) + 4*(l/32) + (r%4), column l%32; of the 16x16 MFMA: row 4*(l/16) + r, col l%16 (the layout test in
// tests/test_gpu.py checks both).
//
// Buffer loads: the hardware range-checks a raw buffer access by its VGPR offset (plus the instruction offset);
// the SGPR offset is added to the address unchecked. Every load here keeps voffset + soffset inside the buffer, and
// uses an out-of-range voffset (never soffset) where a row must read as zero.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kt_dpp.h"
#include "kt_hip.h"

namespace kt {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// LDS tiles are rows of BK bytes in 16-byte chunks; chunk c of row r sits at chunk position c ^ swz(r) so that the
// MFMA operand reads (consecutive lanes = consecutive rows, same chunk) fall in distinct banks. For 64-byte rows
// swz = (r >> 2) & 3 measured conflict-free on gfx950 (about 195 B/clk per CU for ds_read_b128, against about
// 120 for (r >> 1) & 3 and 62 without a swizzle).
template <int CPR>
__device__ __forceinline__ int swz(int r) {
    if constexpr (CPR == 4) return (r >> 2) & 3;
    else return (r ^ (r >> 3)) & 7;
}

template <int CPR>
__device__ __forceinline__ int lds_off(int r, int c) {
    return r * (CPR * 16) + ((c ^ swz<CPR>(r)) << 4);
}

__device__ __forceinline__ v4i lds_read16(const int8_t* base, int off) {
    return *reinterpret_cast<const v4i*>(base + off);
}
__device__ __forceinline__ void lds_write16(int8_t* base, int off, v4i v) {
    *reinterpret_cast<v4i*>(base + off) = v;
}

__device__ __forceinline__ v4i gload16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

// A raw buffer over `bytes` bytes at `base`: a load whose VGPR offset is past the end returns zeros, so tile rows
// beyond the matrix need no branch. The descriptor lives in SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
__device__ __forceinline__ v2i bload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}
// The same loads non-temporal (cache policy nt): for weight streams a launch reads once, so that they do not push
// the small tensors the next launches read out of the caches.
__device__ __forceinline__ v4i bload16nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
}
__device__ __forceinline__ v2i bload8nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 2);
}
// An offset that is out of range for every buffer here (buffers are below 4 GB - 16 B).
#define KT_OOB 0xFFFFFFF0u

// 8 nib bytes of a lane -> 16 hi digits in natural k order.
__device__ __forceinline__ v4i unpack_hi(v2i d) {
    const int m4 = 0x0F0F0F0F;
    return v4i{d.x & m4, (d.x >> 4) & m4, d.y & m4, (d.y >> 4) & m4};
}

// The thread's index as a value the compiler cannot prove loop-invariant (an empty asm that may change it): the tile
// code derives its per-lane offsets from it, so that a persistent kernel recomputes them for each tile (a few VALU
// instructions) instead of hoisting them out of its tile loop and holding them, or spilling them to scratch memory,
// across every mainloop (the grouped MoE kernel went from 77-153 spilled VGPRs to none).
__device__ __forceinline__ int tid_now() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ int sum4(v4i v) {
    const int ones = 0x01010101;
    int s = __builtin_amdgcn_sdot4(v.x, ones, 0, false);
    s = __builtin_amdgcn_sdot4(v.y, ones, s, false);
    s = __builtin_amdgcn_sdot4(v.z, ones, s, false);
    return __builtin_amdgcn_sdot4(v.w, ones, s, false);
}

// round(acc * mant / 2^shift), half away from zero, from the exact 128-bit product, saturated to i64 -- for every
// int32 shift. kt-int's requant (crates/00-kernels/kt-int/src/lib.rs:78-86) computes the same value and casts it to
// i64 with wrap-around; the two agree wherever the value fits i64 (always for shift > 0 and |acc| < 2^32).
__device__ __forceinline__ int64_t requant_dev(int64_t acc, int64_t mant, int shift) {
    typedef unsigned __int128 u128;
    const __int128 prod = (__int128)acc * (__int128)mant;  // |prod| <= 2^126
    if (prod == 0) return 0;
    const bool neg = prod < 0;
    const u128 a = neg ? (u128)(-prod) : (u128)prod, top = (u128)1 << 63;
    u128 q;
    if (shift <= 0) {
        const int s = shift < -64 ? 64 : -shift;
        q = (s >= 64 || (a >> (63 - s)) != 0) ? top : a << s;
    } else if (shift >= 127) {
        q = 0;  // |prod| < 2^126 <= 2^(shift - 1)
    } else {
        q = (a + ((u128)1 << (shift - 1))) >> shift;
    }
    if (q >= top) return neg ? INT64_MIN : INT64_MAX;
    return neg ? -(int64_t)q : (int64_t)q;
}

// a + b saturated to int32 (a residual add: the stored value plus a requantized output).
__device__ __forceinline__ int32_t sat_add32(int32_t a, int64_t b) {
    const int64_t v = (int64_t)a + b;
    return (int32_t)(v > INT32_MAX ? INT32_MAX : (v < INT32_MIN ? INT32_MIN : v));
}

template <int OUT>
__device__ __forceinline__ void store_out(void* y, size_t idx, int64_t v, const int32_t* mant, const int32_t* shift,
                                          int n) {
    if constexpr (OUT == KT_OUT_I64) {
        reinterpret_cast<int64_t*>(y)[idx] = v;
    } else {
        int64_t q = requant_dev(v, mant[n], shift[n]);
        if constexpr (OUT == KT_OUT_I32 || OUT == KT_OUT_I32_ADD) {
            q = q > INT32_MAX ? INT32_MAX : (q < INT32_MIN ? INT32_MIN : q);
            if constexpr (OUT == KT_OUT_I32_ADD) q = sat_add32(reinterpret_cast<int32_t*>(y)[idx], q);
            reinterpret_cast<int32_t*>(y)[idx] = (int32_t)q;
        } else {
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            reinterpret_cast<int8_t*>(y)[idx] = (int8_t)q;
        }
    }
}

// s_lo + 256 s_hi + corr for a dot known to fit int32: formed modulo 2^32 (256 s_hi alone may not fit).
__device__ __forceinline__ int w12_value(int s_lo, int s_hi, int corr) {
    return (int)((uint32_t)s_lo + ((uint32_t)s_hi << 8) + (uint32_t)corr);
}

// The per-channel requant of a value |v| < 2^32 as one multiply-add and shift: for int32 mant and any shift,
// requant(v, mant, shift) = sign * ((|v| * mt + bias) >> shr) with mt <= 2^32 - 1 (kt-int/src/lib.rs:78-86):
//   shift > 0: mt = |mant|, shr = shift, bias = 2^(shift-1) (shift >= 63 gives 0: |v| * mt < 2^63 - 2^62);
//   shift <= 0: mt = |mant| << -shift, saturated at 2^32 - 1 -- a saturated mt only arises when any nonzero |v|
//   already exceeds every clamp bound, and zero stays zero.
struct ColQ {
    uint32_t mt, shr;
    uint64_t bias;
    bool neg;
};

__device__ __forceinline__ ColQ col_q(int32_t mant, int32_t sh) {
    ColQ q;
    q.neg = mant < 0;
    const uint64_t am = mant < 0 ? (uint64_t)(-(int64_t)mant) : (uint64_t)mant;
    if (sh >= 63) {
        q.mt = 0, q.shr = 0, q.bias = 0;
    } else if (sh > 0) {
        q.mt = (uint32_t)am, q.shr = (uint32_t)sh, q.bias = (uint64_t)1 << (sh - 1);
    } else {
        const int up = -sh;
        const uint64_t t = up >= 32 ? (am ? 0xFFFFFFFFull : 0) : am << up;
        q.mt = (uint32_t)(t > 0xFFFFFFFFull ? 0xFFFFFFFFull : t), q.shr = 0, q.bias = 0;
    }
    return q;
}

// requant(v) clamped to the output: [-127, 127] for int8, [-2^31, 2^31 - 1] for int32.
template <bool I32>
__device__ __forceinline__ int32_t col_requant(int v, const ColQ& q) {
    const uint32_t a = v < 0 ? 0u - (uint32_t)v : (uint32_t)v;
    uint64_t m = ((uint64_t)a * q.mt + q.bias) >> q.shr;
    const bool neg = (v < 0) != q.neg;
    const uint64_t lim = I32 ? (neg ? 0x80000000ull : 0x7FFFFFFFull) : 127;
    m = m > lim ? lim : m;
    return neg ? (int32_t)(0u - (uint32_t)m) : (int32_t)m;
}

// The int8 requant of one output channel with a double-precision path. requant(v) = round(v mant / 2^shift) half
// away from zero, clamped to +-127, is odd in v and in mant, so it equals sign(v) sign(mant) min(floor(|v| ms + 0.5),
// 127) with ms = |mant| 2^-shift (exact in double: a 31-bit integer scaled by a power of two in range). For
// shift <= 46, unless the value saturates, |v mant| < 127.5 2^shift < 2^53, so |v| ms + 0.5 is exact and truncation
// floors it; a saturating value rounds to 127.5 or more (rounding is monotone) and the clamp holds it at 127. Other
// shifts take col_requant.
struct ColQ8 {
    ColQ q;
    double ms;     // mant x 2^-shift (exact when fp)
    bool fp;       // the double path is exact for this channel
    uint32_t hsb;  // high dword of 0.5 with the scale's sign: 0x3FE00000, or 0xBFE00000 for a negative scale
};

__device__ __forceinline__ ColQ8 col_q8(int32_t mant, int32_t sh) {
    ColQ8 c;
    c.q = col_q(mant, sh);
    c.fp = sh >= -512 && sh <= 46;
    c.ms = c.fp ? ldexp((double)mant, -sh) : 0.0;
    c.hsb = 0x3FE00000u | (mant < 0 ? 0x80000000u : 0u);
    return c;
}

// v_cvt_i32_f64: values beyond the int32 range convert to its nearest end (a C++ conversion of them is undefined).
__device__ __forceinline__ int cvt_i32_sat(double d) {
    int r;
    asm("v_cvt_i32_f64 %0, %1" : "=v"(r) : "v"(d));
    return r;
}

// The double operand 0.5 sign(v) sign(scale), from the column's hsb: one bit operation on its high dword.
__device__ __forceinline__ double rq8_half(int v, uint32_t hsb) {
    return __longlong_as_double((long long)((uint64_t)(((uint32_t)v & 0x80000000u) ^ hsb) << 32));
}

// a * b + c in one rounding as the three-operand v_fma_f64: the compiler's two-operand v_fmac_f64 would copy the
// addend first, since the addend's zero low dword is one register shared by every value of an epilogue
__device__ __forceinline__ double fma3_f64(double a, double b, double c) {
    double r;
    asm("v_fma_f64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// col_requant<false>(v, q) for a channel with fp (ms = mant x 2^-shift, hsb its half's high dword): v ms +
// 0.5 sign(v ms) truncated toward zero is sign(v ms) floor(|v ms| + 0.5), clamped to [-127, 127]. Unless the result
// saturates, |v| |mant| < 127.5 * 2^shift < 2^53 (shift <= 46), so the fma is exact; a saturating value stays at or
// beyond 127.5 in magnitude after rounding (rounding is monotone) and the clamp holds it at 127. |v ms| < 2^574, so
// no value is infinite and the saturating conversion keeps the clamp's input ordered.
__device__ __forceinline__ int32_t rq8_fp(int v, double ms, uint32_t hsb) {
    const int y = cvt_i32_sat(fma3_f64((double)v, ms, rq8_half(v, hsb)));
    return min(max(y, -127), 127);
}
__device__ __forceinline__ int32_t rq8_fp(int v, const ColQ8& c) { return rq8_fp(v, c.ms, c.hsb); }

// -1920 x (a row's sum of x), the W12 offset term of the int8-output epilogues, as one full-rate 24-bit multiply: those
// products have kp <= KT_SMALL_KP, so |row sum| <= 128 kp < 2^23 and the product fits int32.
__device__ __forceinline__ int w12_corr(int rowsum) { return __mul24(rowsum, -1920); }

// clamp(requant(v, 1, sh), -127, 127) for 1 <= sh <= 30 and |v| < 2^31: round half away from zero.
// |v| + 2^(sh - 1) <= 2^31 + 2^29 stays below 2^32, so the sum and shift are 32-bit; the sign is applied as
// (m ^ s) - s with s = v >> 31.
__device__ __forceinline__ int32_t shift_rq8(int v, int sh) {
    const int32_t s = v >> 31;
    const uint32_t a = ((uint32_t)v ^ (uint32_t)s) - (uint32_t)s;
    uint32_t m = (a + (1u << (sh - 1))) >> sh;
    m = m > 127u ? 127u : m;
    return ((int32_t)m ^ s) - s;
}

// The longest k for which every W12 dot fits int32: 8128 * 128 * 2048 < 2^31 <= 8192 * 128 * 2048.
#define KT_SMALL_KP 8128

// floor(sqrt(n)) exactly: a double estimate, then corrected by whole steps.
__device__ __forceinline__ uint64_t isqrt_u64(uint64_t n) {
    uint64_t x = (uint64_t)sqrt((double)n);
    while (x > 0 && x * x > n) x--;
    while ((x + 1) * (x + 1) <= n) x++;
    return x;
}

// floor(S / d) of an exact sum of squares S = hi * 2^16 + lo kept as two wrapping-free parts: hi sums v^2 >> 16 and
// lo sums v^2 & 0xFFFF over at most 2^18 values of |v| <= 2^31 (hi < 2^64, lo < 2^34). The quotient is at most 2^62.
__device__ __forceinline__ uint64_t sq_mean_floor(uint64_t hi, uint64_t lo, uint64_t d) {
    const uint64_t q1 = hi / d, r1 = hi - q1 * d;
    return (q1 << 16) + ((r1 << 16) + lo) / d;
}

// The decoder's RMSNorm code of one residual value: clamp(div_round(32 x, rms), +-127), 0 when rms = 0 (div_round =
// round half away from zero). div_round(a, rms) = floor((2|a| + rms) / dd) with a's sign, dd = 2 rms. inv =
// floor((2^64 - 1) / dd) (rms_inv) makes the quotient one high multiply: below the clamp n = 2|a| + rms < 2^38, so
// mulhi(n, inv) is the exact quotient or one less, and the remainder test settles it.
__device__ __forceinline__ uint64_t rms_inv(int64_t rms) { return rms > 0 ? ~0ULL / (uint64_t)(2 * rms) : 0; }
__device__ __forceinline__ int rms_q8(int32_t x, int64_t rms, uint64_t inv) {
    if (rms == 0) return 0;
    const int64_t a = 32 * (int64_t)x, aa = a < 0 ? -a : a;
    if (aa >= 128 * rms) return a < 0 ? -127 : 127;
    const uint64_t n = (uint64_t)(2 * aa + rms), dd = (uint64_t)(2 * rms);
    uint64_t q = __umul64hi(n, inv);
    if ((q + 1) * dd <= n) q++;
    q = q > 127 ? 127 : q;
    return a < 0 ? -(int)q : (int)q;
}

// RMSNorm of rows 0 .. M-1 (M <= 16) of the int32 residual r (row stride d) into int8 rows q[m][0 .. kp) in LDS,
// zero padded from d: rms = isqrt(floor(sum r^2 / d)) over the row (the exact sum, sq_mean_floor), then rms_q8 per
// value. All NT threads share every row; row 0's values tid + j NT (j < PRE) come preloaded in pre[] (norm_preload,
// issued before anything else so their latency overlaps the caller's weight loads). s_ss (NT / 64 x 32) and s_rq
// (2 x 16) are LDS scratch. Ends with a barrier.
template <int NT, int PRE>
__device__ __forceinline__ void norm_preload(const int32_t* __restrict__ r, int d, int32_t (&pre)[PRE]) {
#pragma unroll
    for (int j = 0; j < PRE; j++) {
        const int i = (int)threadIdx.x + j * NT;
        pre[j] = i < d ? r[i] : 0;
    }
}

template <int NT, int PRE>
__device__ __forceinline__ void norm_rows_to_lds(const int32_t* __restrict__ r, int M, int d, int kp, int8_t* q,
                                                 uint64_t* s_ss, uint64_t* s_rq, const int32_t (&pre)[PRE]) {
    const int tid = tid_now(), lane = tid & 63, w = tid >> 6;
    for (int m = 0; m < M; m++) {
        uint64_t sh = 0, sl = 0;
        int i = tid;
        if (m == 0) {
#pragma unroll
            for (int j = 0; j < PRE; j++, i += NT) {  // zero past d
                const uint64_t sq = (uint64_t)((int64_t)pre[j] * pre[j]);
                sh += sq >> 16, sl += sq & 0xFFFF;
            }
        }
        for (; i < d; i += NT) {
            const int64_t v = r[(size_t)m * d + i];
            const uint64_t sq = (uint64_t)(v * v);
            sh += sq >> 16, sl += sq & 0xFFFF;
        }
        sh = wave_sum_u64(sh), sl = wave_sum_u64(sl);  // DPP, no LDS
        if (lane == 0) s_ss[w * 32 + m] = sh, s_ss[w * 32 + 16 + m] = sl;
    }
    __syncthreads();
    if (tid < M) {
        uint64_t sh = 0, sl = 0;
#pragma unroll
        for (int q2 = 0; q2 < NT / 64; q2++) sh += s_ss[q2 * 32 + tid], sl += s_ss[q2 * 32 + 16 + tid];
        const int64_t rms = (int64_t)isqrt_u64(sq_mean_floor(sh, sl, (uint64_t)d));
        s_rq[tid] = (uint64_t)rms;
        s_rq[16 + tid] = rms_inv(rms);
    }
    __syncthreads();
    for (int m = 0; m < M; m++) {
        const int64_t rms = (int64_t)s_rq[m];
        const uint64_t inv = s_rq[16 + m];
        int i = tid;
        if (m == 0) {
#pragma unroll
            for (int j = 0; j < PRE; j++, i += NT)
                if (i < kp) q[i] = (int8_t)(i < d ? rms_q8(pre[j], rms, inv) : 0);
        }
        for (; i < kp; i += NT) q[(size_t)m * kp + i] = (int8_t)(i < d ? rms_q8(r[(size_t)m * d + i], rms, inv) : 0);
    }
    __syncthreads();
}

// The device QuantLinear's per-call record (kt_quant.hip writes it; the digit GEMM's epilogue reads it). The output
// maximum is kept in KT_QL_YSLOTS words on separate 128-byte lines: CTA b of the GEMM raises slot b % KT_QL_YSLOTS
// with an atomic maximum (a few hundred CTAs on one word serialize), ql_requant takes the largest.
#define KT_QL_YSLOTS 16
struct QlYSlot {
    unsigned long long v;
    unsigned long long pad[15];
};
struct QlState {
    int64_t xmax;                // max |x|
    int64_t c_mant, f_mant;      // c = from_ratio(xmax, WLEVELS) * xs * ws; f = bias scale * c^-1
    int32_t c_shift, f_shift;
    int32_t mode;                // 0: normal; 1: xmax == 0 (bias codes or zeros); 2: c == 0 (zeros)
    int32_t pad;
    unsigned long long pad2[13];
    QlYSlot ymax[KT_QL_YSLOTS];  // max |acc + bias| over the output, in slots (above)
};

// Several QuantLinear calls on one input with their outputs side by side (the projections of one tensor): segment s
// holds the output columns col0[s] .. col0[s + 1] - 1 and has its own state at ql + s. Every CTA of the digit GEMM
// lies within one segment (the host checks that each boundary is a multiple of the CTA's columns). n = 1: one call.
#define KT_QL_MAX_SEG KT_QL_MAX_SEGMENTS
struct QlSeg {
    int n;
    int col0[KT_QL_MAX_SEG + 1];
};
__device__ __forceinline__ int ql_seg_of(const QlSeg& g, int col) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < KT_QL_MAX_SEG; i++) s += (i < g.n && col >= g.col0[i]) ? 1 : 0;
    return s;
}

// Raise the call's output maximum from CTA b (b > 0 only).
__device__ __forceinline__ void ql_raise_ymax(QlState* ql, int64_t b) {
    atomicMax(&ql->ymax[blockIdx.x % KT_QL_YSLOTS].v, (unsigned long long)b);
}

// Scale::apply / requant (crates/00-kernels/kt-int/src/lib.rs:78-86, 261-272): round(v * mant / 2^shift) half away
// from zero from the i128 product, cast to i64. Shifts of 127 or more either way give 0 (the product has at most
// 126 bits).
__device__ __forceinline__ int64_t scale_apply(int64_t mant, int32_t shift, int64_t v) {
    if (mant == 0) return 0;
    const __int128 prod = (__int128)v * (__int128)mant;
    if (shift <= 0) return shift <= -127 ? 0 : (int64_t)(prod << (-shift));
    if (shift >= 127) return 0;
    const __int128 half = (__int128)1 << (shift - 1);
    return (int64_t)(prod >= 0 ? (prod + half) >> shift : -(((-prod) + half) >> shift));
}

// Longest RMSNorm-fused skinny product: the normalized rows live in LDS (M * kp bytes).
#define KT_NORM_LDS_MAX KT_NORM_LDS_BYTES

template <int I>
using slot_t = std::integral_constant<int, I>;

// Compile-time loop: f(integral_constant<int, I>) for I = B..E-1.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// ------------------------------------------------------------------------------------------------------------------
// The W12 tile mainloop. CTA = WM x WN waves (WM along M, WN along N); each wave owns WTM x WTN tiles of 32x32 (its
// wave row's 32*WTM rows, its own 32*WTN columns), BK = 64. A goes global -> registers -> an NSLOT-slot LDS ring;
// each wave's B fragments go straight from global memory into registers. Both are issued NSLOT-1 tiles ahead of the
// tile being multiplied, and the loop is unrolled by NSLOT so every register set has a compile-time slot. Loads of
// tiles past the end re-read the last tile (staying inside the buffers) and are masked to zero when staged, so their
// MFMAs add zero instead of being branched around -- no MFMA sits under control flow, which would cost accumulator
// copies. Row sums of x (for -1920 * sum_k x) come from the A staging registers.
// ------------------------------------------------------------------------------------------------------------------
template <int WM_, int WTM_, int WTN_, int NSLOT_, int WN_ = 4>
struct W12Tile {
    static constexpr int WM = WM_, WTM = WTM_, WTN = WTN_, NSLOT = NSLOT_, WN = WN_;  // WN waves along N
    static constexpr int NT = 64 * WM * WN;  // threads
    static constexpr int BK = 64, CPR = 4;
    static constexpr int BM = 32 * WTM * WM, BN = 32 * WTN * WN;
    static constexpr int AC = BM * CPR, AL = (AC + NT - 1) / NT;  // 16-byte A chunks per k-tile / per thread
    static constexpr int RING = NSLOT * BM * BK;                   // bytes of the A ring
};

// A chunk idx = tid + NT * i of a k-tile is tile row idx >> 2, 16-byte column idx & 3; oa[i] is its byte offset in
// rA at k = 0 (KT_OOB for a row that must read as zero or a chunk index past the tile). B column block j of the
// wave starts at ob[j] in rL (1 KB per k32 block) and on[j] in rN (512 B per k32 block). nk = kp / 64 >= 1.
template <class C>
__device__ __forceinline__ void w12_mainloop(const __amdgpu_buffer_rsrc_t rA, const uint32_t (&oa)[C::AL],
                                             const __amdgpu_buffer_rsrc_t rL, const __amdgpu_buffer_rsrc_t rN,
                                             const uint32_t (&ob)[C::WTN], const uint32_t (&on)[C::WTN], int nk,
                                             int8_t* smem, v16i (&acc0)[C::WTM][C::WTN],
                                             v16i (&acc1)[C::WTM][C::WTN], int (&rsum)[C::AL]) {
    constexpr int NT = C::NT, NSLOT = C::NSLOT, AL = C::AL, AC = C::AC, WTM = C::WTM, WTN = C::WTN;
    constexpr int CPR = C::CPR, BM = C::BM, BK = C::BK;
    int8_t(*sA)[BM * BK] = reinterpret_cast<int8_t(*)[BM * BK]>(smem);
    const int tid = tid_now(), lane = tid & 63, half = lane >> 5;
    const int rw0 = ((tid >> 6) / C::WN) * 32 * WTM;  // the wave's first row in the tile

#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++) acc0[i][j] = acc1[i][j] = v16i{};
#pragma unroll
    for (int i = 0; i < AL; i++) rsum[i] = 0;

    v4i ra[NSLOT][AL];
    v4i bl[NSLOT][WTN][2];
    v2i bn[NSLOT][WTN][2];

    auto issue = [&](auto S, int kt) {  // global loads of tile kt (clamped to the last tile) into register slot S
        constexpr int sl = decltype(S)::value;
        const uint32_t kl = (uint32_t)(kt < nk ? kt : nk - 1);
#pragma unroll
        for (int j = 0; j < WTN; j++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                bl[sl][j][ks] = bload16(rL, ob[j], (2 * kl + ks) * 1024u);
                bn[sl][j][ks] = bload8(rN, on[j], (2 * kl + ks) * 512u);
            }
#pragma unroll
        for (int i = 0; i < AL; i++) ra[sl][i] = bload16(rA, oa[i], kl * BK);
        // keep the loads at the head of the step: the scheduler would otherwise sink them behind the MFMAs and
        // shorten the distance they have to land
        __builtin_amdgcn_sched_barrier(0);
    };
    // `mask` is -1, or 0 for a tile past the end in the last round: such a tile is staged as zeros (and adds
    // nothing to the row sums)
    auto stage = [&](auto S, int mask) {  // A of slot S into LDS buffer S
        constexpr int sl = decltype(S)::value;
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int idx = tid + NT * i;
            if (AC % NT != 0 && idx >= AC) continue;
            const v4i v = ra[sl][i] & mask;
            lds_write16(sA[sl], lds_off<CPR>(idx >> 2, idx & 3), v);
            rsum[i] += sum4(v);
        }
    };
    auto mma = [&](auto S, const v4i (&a)[WTM], int ks) {
        constexpr int sl = decltype(S)::value;
#pragma unroll
        for (int j = 0; j < WTN; j++) {
            const v4i b0 = bl[sl][j][ks], b1 = unpack_hi(bn[sl][j][ks]);
#pragma unroll
            for (int i = 0; i < WTM; i++) {
                acc0[i][j] = mfma32(a[i], b0, acc0[i][j]);
                acc1[i][j] = mfma32(a[i], b1, acc1[i][j]);
            }
        }
    };
    auto compute = [&](auto S) {
        constexpr int sl = decltype(S)::value;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i a[WTM];
#pragma unroll
            for (int i = 0; i < WTM; i++) a[i] = lds_read16(sA[sl], lds_off<CPR>(rw0 + i * 32 + (lane & 31), 2 * ks + half));
            mma(S, a, ks);
        }
    };

    // Rounds of NSLOT tiles kt .. kt+NSLOT-1 in slots 0 .. NSLOT-1. Before a round, tile kt is in LDS slot 0 and
    // tiles kt+1 .. kt+NSLOT-2 are in flight in register slots 1 .. NSLOT-2; step s issues tile kt+s+NSLOT-1 (NSLOT-1
    // tiles ahead), multiplies tile kt+s and stages tile kt+s+1. A do-while: the accumulators have one path out.
    static_for<0, NSLOT - 1>([&](auto S) { issue(S, decltype(S)::value); });
    stage(slot_t<0>{}, -1);
    __syncthreads();
    int kt = 0;
    do {
        static_for<0, NSLOT>([&](auto S) {
            constexpr int st = decltype(S)::value;
            issue(slot_t<(st + NSLOT - 1) % NSLOT>{}, kt + st + NSLOT - 1);
            compute(S);
            stage(slot_t<(st + 1) % NSLOT>{}, kt + st + 1 < nk ? -1 : 0);
            __syncthreads();
        });
        kt += NSLOT;
    } while (kt < nk);
}

// ------------------------------------------------------------------------------------------------------------------
// W12 mainloop for a 256 x 128 CTA tile whose operands all arrive by LDS DMA (buffer_load ... lds: each lane's bytes
// land at M0 + size * lane without passing through VGPRs). 8 waves: wave w computes rows 128 (w / 4) .. + 127 against
// column block w % 4 (4 x 1 tiles of 32x32, two planes). A stage holds one k-tile (BK = 64) of every operand:
//   A    [0, 16384):     256 rows x 64 bytes, chunk c of row r at r * 64 + 16 (c ^ swz(r)) (the register path's layout)
//   lo   [16384, 24576): the 4 column blocks' two 1 KB k32 fragments, block (cb, ks) at 1024 (2 cb + ks)
//   nib  [24576, 28672): the matching 512-byte nib fragments at 512 (2 cb + ks)
// Each wave moves 5 pieces per k-tile: A rows 32w .. 32w + 31 (two 1 KB DMAs whose lanes gather the swizzled
// chunks), fragment (w / 2, w % 2) of lo (one 16-byte DMA) and of nib (two 4-byte DMAs). Operands are re-read by
// every wave that uses them from LDS, so each byte crosses the L2 -> CU path once per CTA, against twice for A and
// four times for B with two 128 x 128 CTAs. The ring has NS stages, NS - 1 k-tiles in flight beyond the one being
// multiplied; a wave waits for its own DMAs of a tile (vmcnt, in order) and a barrier publishes everyone's. Tiles
// past the end are re-reads of the last one into stages that are never consumed. The row sums of x come from the
// A fragment of row tile w % 4, read once more by each wave. Ends with every DMA landed, sRow[256] written and a barrier: the ring is free.
// ------------------------------------------------------------------------------------------------------------------
constexpr int KT_DMA_STAGE = 28672, KT_DMA_LO = 16384, KT_DMA_NIB = 24576;
// BAL (the balanced two-plane weights, W12B): the hi plane is a full int8 fragment like lo, 1 KB per (column block,
// k32 half), at KT_DMA_HI; a stage is 32 KB.
constexpr int KT_DMA_STAGE_BAL = 32768, KT_DMA_HI = 24576;
template <bool BAL>
constexpr int dma_stage_bytes() { return BAL ? KT_DMA_STAGE_BAL : KT_DMA_STAGE; }
// XR = 32 (W12 planes only): the stage's A part holds 32 more rows (256 .. 287), so the lo and nib parts move up by
// 2 KB: A [0, 18432), lo [18432, 26624), nib [26624, 30720).
constexpr int KT_DMA_XR = 32;
template <int XR>
constexpr int dma_lo_off() { return 64 * (256 + XR); }
template <int XR>
constexpr int dma_nib_off() { return dma_lo_off<XR>() + 8192; }
template <int XR>
constexpr int dma_stage_x() { return dma_nib_off<XR>() + 4096; }
static_assert(dma_lo_off<0>() == KT_DMA_LO && dma_nib_off<0>() == KT_DMA_NIB && dma_stage_x<0>() == KT_DMA_STAGE,
              "XR = 0 is the plain stage");

// The strip of a 288-row tile (XR): rows 256 + 16 mh .. + 15 of M-half mh against the wave's 32 columns as two
// 16 x 16 blocks (j = 0, 1), both planes; vx: this lane's A piece of the strip rows at k = 0 (see w12_mainloop_dma).
struct DmaStrip {
    uint32_t vx;
    v4i acc0[2], acc1[2];
};
#ifndef KT_DMA_NS
#define KT_DMA_NS 4  // ring stages of the DMA-fed kernels
#endif

typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, int8_t* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, int8_t* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 4, voff, soff, 0, 0);
}

// The A rows a lane moves: tile rows 32w + l / 4 and 32w + 16 + l / 4 (DMA instructions 2w and 2w + 1 cover LDS rows
// 16 j .. 16 j + 15; lane l lands at row 16 j + l / 4, chunk position l % 4). Returns the chunk of x it must fetch,
// (l % 4) ^ swz(row) = (l % 4) ^ ((l / 16) % 4), as a byte offset within a k-tile row.
__device__ __forceinline__ int dma_a_row(int w, int lane, int j) { return 32 * w + 16 * j + (lane >> 2); }
__device__ __forceinline__ uint32_t dma_a_chunk(int lane) { return 16u * ((lane & 3) ^ ((lane >> 4) & 3)); }

// The strip rows' A pieces (XR): wave w moves rows 256 + 4 w .. + 3 with one 4-byte DMA (lane l: row 256 + 4 w +
// l / 16, byte 4 (l % 16) of its LDS row, i.e. chunk position (l % 16) / 4, dword l % 4); the swizzle of those rows is
// (row >> 2) & 3 = w & 3. Returns the byte offset within a k-tile row of x that the lane fetches.
__device__ __forceinline__ int dma_x_row(int w, int lane) { return 256 + 4 * w + (lane >> 4); }
__device__ __forceinline__ uint32_t dma_x_byte(int w, int lane) {
    return 16u * (((lane >> 2) & 3) ^ (w & 3)) + 4u * (lane & 3);
}

// va0 / va1: the byte offsets in rA of this lane's two A pieces at k = 0 (rows dma_a_row(w, lane, 0 / 1), chunk
// dma_a_chunk(lane)); an offset past the descriptor reads zeros (rows past the tile's rows).
// BAL: rN is the hi plane of the balanced split (v = lo + 256 hi, no offset): each wave moves its hi fragment with one
// 16-byte DMA like lo (4 DMAs per k-tile, not 5), the MFMA takes it as read, and there are no row sums (sRow is 0).
// XR (W12 planes): a 288-row tile. Each wave also moves its 4 strip rows (one more DMA per k-tile) and multiplies
// the strip of its M-half (xs: 16 rows x its 32 columns, two 16x16x64 products per plane per k-tile, the operands
// read from the stage in the 16x16x64 layout: A row 256 + 16 mh + l % 16, k chunk l / 16; B lane l' = 32 ((l / 16)
// % 2) + 16 j + l % 16 of the (column block, k32 half l / 32) fragment); the waves of column block 0 write the strip
// rows' sums to sRow[256 ..].
template <int NS, bool BAL = false, int XR = 0>
__device__ __forceinline__ void w12_mainloop_dma(const __amdgpu_buffer_rsrc_t rA, const __amdgpu_buffer_rsrc_t rL,
                                                 const __amdgpu_buffer_rsrc_t rN, uint32_t va0, uint32_t va1, int kp,
                                                 int8_t* ring, v16i (&acc0)[4][1], v16i (&acc1)[4][1], int* sRow,
                                                 DmaStrip* xs = nullptr) {
    static_assert(XR == 0 || (XR == KT_DMA_XR && !BAL), "the strip is for the W12 planes");
    constexpr int ND = (BAL ? 4 : 5) + (XR ? 1 : 0);  // DMAs per wave and k-tile
    constexpr int STAGE = XR ? dma_stage_x<XR>() : dma_stage_bytes<BAL>();
    constexpr int LO = XR ? dma_lo_off<XR>() : KT_DMA_LO, NIB = XR ? dma_nib_off<XR>() : KT_DMA_NIB;
    static_assert(NS >= 2 && ND * (NS - 2) <= 63, "vmcnt holds the DMAs of NS - 2 later tiles");
    const int tid = tid_now(), lane = tid & 63, half = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = w & 3, rw0 = 128 * (w >> 2);
    const int nk = kp / 64, KB = kp / 32;

    const int cbw = w >> 1, ksw = w & 1;  // the fragment this wave moves
    const uint32_t vl = (uint32_t)(cbw * KB) * 1024u + 16 * lane, vn = (uint32_t)(cbw * KB) * 512u + 4 * lane;

    // ND DMAs per wave and k-tile on every wave, so one vmcnt target serves all (a wave-dependent count would put
    // branches in the loop, which keep the scheduler from moving MFMAs across the barrier)
    auto issue = [&](int st, int kt) {
        const uint32_t kl = (uint32_t)(kt < nk ? kt : nk - 1);
        int8_t* s = ring + st * STAGE;
        dma16(rA, s + 2048 * w, va0, kl * 64);
        dma16(rA, s + 2048 * w + 1024, va1, kl * 64);
        dma16(rL, s + LO + 1024 * w, vl, (2 * kl + ksw) * 1024u);
        if constexpr (BAL) {
            dma16(rN, s + KT_DMA_HI + 1024 * w, vl, (2 * kl + ksw) * 1024u);
        } else {
            dma4(rN, s + NIB + 512 * w, vn, (2 * kl + ksw) * 512u);
            dma4(rN, s + NIB + 512 * w + 256, vn + 256, (2 * kl + ksw) * 512u);
        }
        if constexpr (XR != 0) dma4(rA, s + 64 * (256 + 4 * w), xs->vx, kl * 64);
    };
    // the wave's DMAs of a tile have landed once at most those of the NS - 2 later tiles are outstanding
    auto wait_tile = [&]() {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(ND * (NS - 2)) : "memory");
    };

    struct Frag {  // one k32 half of a k-tile: the wave's 4 A fragments, its row-sum fragment and its B fragments
        v4i a[4], ar, b0, b1;
        v2i bn;
    };
    // XR: the strip's operands of a whole k-tile, read with its second half
    struct XFrag {
        v4i a, b0[2];
        v2i bn[2];
    };
    const int xrow = 256 + 16 * (w >> 2) + (lane & 15), xl = 32 * ((lane >> 4) & 1) + (lane & 15), xks = lane >> 5;
    auto load = [&](const int8_t* s, int ks, Frag& f) {
#pragma unroll
        for (int i = 0; i < 4; i++) f.a[i] = lds_read16(s, lds_off<4>(rw0 + 32 * i + (lane & 31), 2 * ks + half));
        f.b0 = lds_read16(s + LO + 1024 * (2 * wn + ks), 16 * lane);
        if constexpr (BAL) {
            f.b1 = lds_read16(s + KT_DMA_HI + 1024 * (2 * wn + ks), 16 * lane);
        } else {
            // row tile wn once more: a wave-uniform select among f.a would compile to branches
            f.ar = lds_read16(s, lds_off<4>(rw0 + 32 * wn + (lane & 31), 2 * ks + half));
            f.bn = *reinterpret_cast<const v2i*>(s + NIB + 512 * (2 * wn + ks) + 8 * lane);
        }
    };
    auto xload = [&](const int8_t* s, XFrag& x) {
        x.a = lds_read16(s, lds_off<4>(xrow, lane >> 4));
#pragma unroll
        for (int j = 0; j < 2; j++) {
            x.b0[j] = lds_read16(s + LO + 1024 * (2 * wn + xks), 16 * (xl + 16 * j));
            x.bn[j] = *reinterpret_cast<const v2i*>(s + NIB + 512 * (2 * wn + xks) + 8 * (xl + 16 * j));
        }
    };
    int rsum = 0, xsum = 0;
    auto mma = [&](const Frag& f) {
        const v4i b1 = BAL ? f.b1 : unpack_hi(f.bn);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            acc0[i][0] = mfma32(f.a[i], f.b0, acc0[i][0]);
            acc1[i][0] = mfma32(f.a[i], b1, acc1[i][0]);
        }
        if constexpr (!BAL) rsum += sum4(f.ar);
    };
    auto xmma = [&](const XFrag& x) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            xs->acc0[j] = mfma16(x.a, x.b0[j], xs->acc0[j]);
            xs->acc1[j] = mfma16(x.a, unpack_hi(x.bn[j]), xs->acc1[j]);
        }
        xsum += sum4(x.a);
    };

#pragma unroll
    for (int i = 0; i < 4; i++) acc0[i][0] = acc1[i][0] = v16i{};
    if constexpr (XR != 0)
#pragma unroll
        for (int j = 0; j < 2; j++) xs->acc0[j] = xs->acc1[j] = v4i{};
#pragma unroll
    for (int t = 0; t < NS - 1; t++) issue(t, t);
    wait_tile();
    issue(NS - 1, NS - 1);
    Frag f0, f1;
    XFrag xf;
    load(ring, 0, f0);
    load(ring, 1, f1);
    if constexpr (XR != 0) xload(ring, xf);
    // Ping-pong: the first half of tile kt's MFMAs covers the barrier that publishes tile kt + 1, the second half
    // covers the LDS reads of tile kt + 1's first half and the DMAs of tile kt + NS (one DMA after every two MFMAs:
    // issued all at once after the barrier, the eight waves' DMAs queue up at the CU's memory path and hold back
    // the MFMAs behind them; 1.7% faster measured), and the reads of its second half run under the next step's
    // first MFMAs. Reads in the last step fetch a stage nobody consumes.
    for (int kt = 0; kt < nk; kt++) {
        mma(f0);
        // tile kt + 1 has landed once at most the DMAs of tiles kt + 2 .. kt + NS - 1 are outstanding; every wave's
        // reads of tile kt are done (lgkmcnt), so after the barrier its stage takes tile kt + NS
        wait_tile();
        const int8_t* sn = ring + ((kt + 1) % NS) * STAGE;
        load(sn, 0, f0);
        __builtin_amdgcn_sched_barrier(0);  // the reads go out before the MFMAs they hide under
        issue(kt % NS, kt + NS);
        mma(f1);
        if constexpr (XR != 0) xmma(xf);
#pragma unroll
        for (int q = 0; q < ND; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one vector-memory read (a DMA)
        }
        __builtin_amdgcn_sched_barrier(0);
        load(sn, 1, f1);
        if constexpr (XR != 0) xload(sn, xf);
    }
    // the re-reads past the end still target the ring
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    rsum += __shfl_xor(rsum, 32);
    if (lane < 32) sRow[rw0 + 32 * wn + lane] = BAL ? 0 : rsum;  // BAL: no offset term to correct
    if constexpr (XR != 0) {  // the strip row's sum over the four k chunks (lanes l, l ^ 16, l ^ 32, l ^ 48)
        xsum += __shfl_xor(xsum, 16);
        xsum += __shfl_xor(xsum, 32);
        if (wn == 0 && lane < 16) sRow[xrow] = xsum;
    }
    __syncthreads();
}

// The CTA's row sums of x into sRow[BM] (the 4 threads of a row are consecutive lanes). Ends with a barrier.
template <class C>
__device__ __forceinline__ void w12_row_sums(const int (&rsum)[C::AL], int* sRow) {
    const int tid = tid_now();
#pragma unroll
    for (int i = 0; i < C::AL; i++) {
        const int idx = tid + C::NT * i;
        int v = rsum[i];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        if (idx < C::AC && (idx & 3) == 0) sRow[idx >> 2] = v;
    }
    __syncthreads();
}

// Requantize the CTA tile (SMALL domain: every dot fits int32) per output channel into an int8 tile sO[BM][BN] in
// LDS. Channel n of the tile's column c is n0 + c; chan(n) maps it to the index of its (mant, shift) pair, and
// columns at or past N get a zero scale.
// LUT: sLut (LDS, 255 entries indexed by q + 127) maps each requantized code as it is written.
template <class C, bool LUT = false, class ChanFn>
__device__ __forceinline__ void w12_requant_tile8(const v16i (&acc0)[C::WTM][C::WTN],
                                                  const v16i (&acc1)[C::WTM][C::WTN], const int* sRow,
                                                  const int32_t* mant, const int32_t* shift, int n0, int N,
                                                  ChanFn chan, int8_t* sO, const int8_t* sLut = nullptr) {
    const int tid = tid_now(), lane = tid & 63, half = lane >> 5;
    const int wave = (tid >> 6) % C::WN, rw0 = ((tid >> 6) / C::WN) * 32 * C::WTM;
#pragma unroll
    for (int j = 0; j < C::WTN; j++) {
        const int c = wave * 32 * C::WTN + j * 32 + (lane & 31), n = n0 + c;
        const int ch = n < N ? chan(n) : 0;
        const ColQ8 q = col_q8(n < N ? mant[ch] : 0, n < N ? shift[ch] : 1);
        auto put = [&](int rt, int code) {
            if constexpr (LUT) sO[rt * C::BN + c] = sLut[code + 127];
            else sO[rt * C::BN + c] = (int8_t)code;
        };
        if (__all(q.fp)) {  // every channel of the wave on the double path
#pragma unroll
            for (int i = 0; i < C::WTM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int rt = rw0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    put(rt, rq8_fp(w12_value(acc0[i][j][r], acc1[i][j][r], w12_corr(sRow[rt])), q));
                }
        } else {
#pragma unroll
            for (int i = 0; i < C::WTM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int rt = rw0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    put(rt, col_requant<false>(w12_value(acc0[i][j][r], acc1[i][j][r], w12_corr(sRow[rt])), q.q));
                }
        }
    }
}

// The strip of a 288-row DMA tile (DmaStrip) requantized into rows 256 .. 287 of the int8 tile sO[.][BN] as
// w12_requant_tile8 does the rest: wave w (M-half w / 4, column block w % 4) holds rows 256 + 16 (w / 4) + 4 (l / 16)
// + r of columns 32 (w % 4) + 16 j + l % 16.
template <int BN, class ChanFn>
__device__ __forceinline__ void w12_requant_strip8(const DmaStrip& xs, const int* sRow, const int32_t* mant,
                                                   const int32_t* shift, int n0, int N, ChanFn chan, int8_t* sO) {
    const int tid = tid_now(), lane = tid & 63, w = tid >> 6;
    const int r0 = 256 + 16 * (w >> 2) + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int c = 32 * (w & 3) + 16 * j + (lane & 15), n = n0 + c;
        const int ch = n < N ? chan(n) : 0;
        const ColQ8 q = col_q8(n < N ? mant[ch] : 0, n < N ? shift[ch] : 1);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int v = w12_value(xs.acc0[j][r], xs.acc1[j][r], w12_corr(sRow[r0 + r]));
            sO[(r0 + r) * BN + c] = (int8_t)(q.fp ? rq8_fp(v, q) : col_requant<false>(v, q.q));
        }
    }
}

// Block-wide exclusive prefix sums of two ints per thread (blockDim.x = NT, a multiple of 64); `tot` receives the
// totals. Uses 2 * (NT / 64) ints of LDS at `scr` and ends with a barrier.
template <int NT>
__device__ __forceinline__ void block_scan2(int a, int b, int& ea, int& eb, int& ta, int& tb, int* scr) {
    const int tid = tid_now(), lane = tid & 63, w = tid >> 6;
    int ia = a, ib = b;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int xa = __shfl_up(ia, d), xb = __shfl_up(ib, d);
        if (lane >= d) ia += xa, ib += xb;
    }
    if (lane == 63) scr[2 * w] = ia, scr[2 * w + 1] = ib;
    __syncthreads();
    int pa = 0, pb = 0;
    ta = 0, tb = 0;
#pragma unroll
    for (int q = 0; q < NT / 64; q++) {
        if (q < w) pa += scr[2 * q], pb += scr[2 * q + 1];
        ta += scr[2 * q], tb += scr[2 * q + 1];
    }
    ea = pa + ia - a, eb = pb + ib - b;
    __syncthreads();
}

}  // namespace kt
