// The non-GEMM kernels of the config-3 decoder on gfx950: embedding rows, integer RMSNorm, table RoPE with the KV
// cache append, integer-softmax attention, greedy argmax with the logits record, and the position counter. The
// GEMMs (q/k/v, o, gate/up, down, lm_head) are the W12 kernels; this file holds what sits between them in the
// reference's decoder (DecoderModel::blocks_int / decode_step, crates/01-engine/kt-core/src/model.rs:168-188,
// 290-353; Attention, attention.rs; generate_greedy_by, generate.rs:82-111).
//
// Positions live in device memory (`pos`: the position of row 0 of the call) and advance on the device, so one
// captured decode step replays for every position with no host involvement. The integer rules are stated with
// kt_hip_dec_* in include/kt_hip.h.

#include <algorithm>
#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "kt_dpp.h"
#include "kt_kernels.h"
#include "kt_w12_core.h"

namespace kt {

// round(a / b) half away from zero, b > 0.
__device__ __forceinline__ int64_t div_round(int64_t a, int64_t b) {
    const int64_t q = (2 * (a < 0 ? -a : a) + b) / (2 * b);
    return a < 0 ? -q : q;
}

__device__ __forceinline__ int shift_round(int v, int s) {  // |v| < 2^30
    const int q = ((v < 0 ? -v : v) + (1 << (s - 1))) >> s;
    return v < 0 ? -q : q;
}

__device__ __forceinline__ int clamp127(int64_t v) { return (int)(v > 127 ? 127 : (v < -127 ? -127 : v)); }

// r[t][i] = emb[tokens[t]][i] (int16 codes -> the int32 residual).
__global__ __launch_bounds__(256) void dec_embed_kernel(const int32_t* __restrict__ tokens,
                                                        const int16_t* __restrict__ emb, int d,
                                                        int32_t* __restrict__ r) {
    const int t = blockIdx.x;
    const int16_t* e = emb + (size_t)tokens[t] * d;
    for (int i = threadIdx.x; i < d; i += 256) r[(size_t)t * d + i] = e[i];
}

// One CTA per row: rms = isqrt(floor(sum r^2 / d)), q = clamp(div_round(32 r, rms), +-127), 0 when rms = 0. q rows
// have stride qs (columns d .. qs - 1 are left alone).
__global__ __launch_bounds__(256) void dec_rmsnorm_kernel(const int32_t* __restrict__ r, int d, int8_t* __restrict__ q,
                                                          int qs) {
    __shared__ uint64_t sw[8];
    __shared__ int64_t s_rms;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int32_t* x = r + (size_t)t * d;
    uint64_t sh = 0, sl = 0;  // the exact sum of squares as sh * 2^16 + sl (sq_mean_floor)
    for (int i = tid; i < d; i += 256) {
        const uint64_t sq = (uint64_t)((int64_t)x[i] * x[i]);
        sh += sq >> 16, sl += sq & 0xFFFF;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sh += __shfl_xor(sh, o), sl += __shfl_xor(sl, o);
    if ((tid & 63) == 0) sw[tid >> 6] = sh, sw[4 + (tid >> 6)] = sl;
    __syncthreads();
    if (tid == 0)
        s_rms = (int64_t)isqrt_u64(sq_mean_floor(sw[0] + sw[1] + sw[2] + sw[3], sw[4] + sw[5] + sw[6] + sw[7], (uint64_t)d));
    __syncthreads();
    const int64_t rms = s_rms;
    const uint64_t inv = rms_inv(rms);
    for (int i = tid; i < d; i += 256) q[(size_t)t * qs + i] = (int8_t)rms_q8(x[i], rms, inv);
}

// One CTA per row t (position p = pos[0] + t): rotate-half RoPE of the nh q heads and nkv k heads in place
// (a' = sr(a C - b S, 14), b' = sr(b C + a S, 14), C/S the int16 tables at p), then k and v to the caches at p.
__global__ __launch_bounds__(256) void dec_rope_kv_kernel(int8_t* __restrict__ qkv, int nqkv,
                                                          const int32_t* __restrict__ pos, int nh, int nkv, int hd,
                                                          const int16_t* __restrict__ cosT,
                                                          const int16_t* __restrict__ sinT, int8_t* __restrict__ kc,
                                                          int8_t* __restrict__ vc) {
    const int t = blockIdx.x, p = pos[0] + t, hh = hd / 2;
    int8_t* row = qkv + (size_t)t * nqkv;
    for (int idx = threadIdx.x; idx < (nh + nkv) * hh; idx += 256) {
        const int hv = idx / hh, i = idx - hv * hh;
        int8_t* x = row + hv * hd;
        const int a = x[i], b = x[i + hh], C = cosT[(size_t)p * hh + i], S = sinT[(size_t)p * hh + i];
        const int na = clamp127(shift_round(a * C - b * S, 14)), nb = clamp127(shift_round(b * C + a * S, 14));
        x[i] = (int8_t)na;
        x[i + hh] = (int8_t)nb;
        if (hv >= nh) {
            int8_t* kr = kc + ((size_t)p * nkv + (hv - nh)) * hd;
            kr[i] = (int8_t)na;
            kr[i + hh] = (int8_t)nb;
        }
    }
    for (int i = threadIdx.x; i < nkv * hd; i += 256) vc[(size_t)p * nkv * hd + i] = row[(nh + nkv) * hd + i];
}

// One CTA (256 threads) per (row t, q head h), hd = 64: scores s_j = q . k_j over positions j <= p (kv head
// g = h / (nh / nkv)) into LDS, m = max, e_j = EXP[(m - s_j + 64) >> 7] (0 past 1024), then sum_j e_j v_j with four
// threads per v row (16 dimensions each, 16-byte loads) and 64 rows in flight, the 64 row groups summed through
// LDS, and o = div_round(sum, sum e). The partial sums fit int32: each thread adds at most max_pos / 64 <= 256
// products of |e| <= 2^15 and |v| <= 127.
__global__ __launch_bounds__(256) void dec_attention_kernel(const int8_t* __restrict__ qkv, int nqkv,
                                                            const int32_t* __restrict__ pos,
                                                            const int8_t* __restrict__ kc,
                                                            const int8_t* __restrict__ vc, int nh, int nkv,
                                                            const int32_t* __restrict__ exp_tab,
                                                            int8_t* __restrict__ o, int max_pos) {
    constexpr int HD = 64;
    extern __shared__ int s_sc[];  // max_pos scores, then weights
    __shared__ int s_red[8];
    __shared__ int s_part[64][HD + 1];
    const int t = blockIdx.x / nh, h = blockIdx.x - t * nh, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int p = pos[0] + t, g = h / (nh / nkv), L = p + 1;
    const int8_t* qr = qkv + (size_t)t * nqkv + h * HD;
    v4i q4[4];
#pragma unroll
    for (int c = 0; c < 4; c++) q4[c] = *reinterpret_cast<const v4i*>(qr + 16 * c);
    int mx = INT_MIN;
    for (int j = tid; j < L; j += 256) {
        const int8_t* kr = kc + ((size_t)j * nkv + g) * HD;
        int s = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const v4i k4 = *reinterpret_cast<const v4i*>(kr + 16 * c);
            s = __builtin_amdgcn_sdot4(q4[c].x, k4.x, s, false);
            s = __builtin_amdgcn_sdot4(q4[c].y, k4.y, s, false);
            s = __builtin_amdgcn_sdot4(q4[c].z, k4.z, s, false);
            s = __builtin_amdgcn_sdot4(q4[c].w, k4.w, s, false);
        }
        s_sc[j] = s;
        mx = s > mx ? s : mx;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const int v = __shfl_xor(mx, d);
        mx = v > mx ? v : mx;
    }
    if (lane == 0) s_red[w] = mx;
    __syncthreads();
    mx = s_red[0];
#pragma unroll
    for (int q = 1; q < 4; q++) mx = s_red[q] > mx ? s_red[q] : mx;
    int den = 0;
    for (int j = tid; j < L; j += 256) {
        const int idx = (int)(((int64_t)mx - s_sc[j] + 64) >> 7);
        const int e = idx < 1024 ? exp_tab[idx] : 0;
        s_sc[j] = e;
        den += e;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) den += __shfl_xor(den, d);
    __syncthreads();  // every wave has read s_red[0..3]; every weight is in LDS
    if (lane == 0) s_red[4 + w] = den;
    // thread (row group rg, 16-dimension chunk c): rows rg, rg + 64, ...
    const int c = tid & 3, rg = tid >> 2;
    int acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0;
    const int8_t* vb = vc + (size_t)g * HD + 16 * c;
    for (int j = rg; j < L; j += 64) {
        const v4i v = *reinterpret_cast<const v4i*>(vb + (size_t)j * nkv * HD);
        const int e = s_sc[j];
        const int8_t* b = reinterpret_cast<const int8_t*>(&v);
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] += e * b[i];
    }
#pragma unroll
    for (int i = 0; i < 16; i++) s_part[rg][16 * c + i] = acc[i];
    __syncthreads();
    if (tid < HD) {
        int64_t sum = 0;
        for (int q = 0; q < 64; q++) sum += s_part[q][tid];
        const int64_t dn = (int64_t)s_red[4] + s_red[5] + s_red[6] + s_red[7];
        o[(size_t)t * nh * HD + h * HD + tid] = (int8_t)clamp127(div_round(sum, dn));
    }
}

// Greedy argmax over n int32 logits (the first maximum, argmax_codes of generate.rs:48-56), one CTA of 1024 threads:
// token[0] = the index; the logits row is also copied to record + step[0] * n and step[0] advances (the per-step
// logits the hash covers). record may be null.
__global__ __launch_bounds__(1024) void dec_argmax_kernel(const int32_t* __restrict__ logits, int n,
                                                          int32_t* __restrict__ token, int32_t* __restrict__ record,
                                                          int32_t* __restrict__ step) {
    __shared__ int64_t s_key[16];
    const int tid = threadIdx.x;
    // key = (value, -index) ordered as one signed 64-bit integer: the max key is the first maximum
    int64_t best = INT64_MIN;
    int32_t* rec = record ? record + (size_t)step[0] * n : nullptr;
    for (int i = tid; i < n; i += 1024) {
        const int32_t v = logits[i];
        if (rec) rec[i] = v;
        const int64_t key = ((int64_t)v << 32) | (uint32_t)(0x7FFFFFFF - i);
        best = key > best ? key : best;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const int64_t o = __shfl_xor(best, d);
        best = o > best ? o : best;
    }
    if ((tid & 63) == 0) s_key[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        int64_t b = s_key[0];
        for (int q = 1; q < 16; q++) b = s_key[q] > b ? s_key[q] : b;
        token[0] = 0x7FFFFFFF - (int32_t)(b & 0xFFFFFFFF);
        if (record) step[0] += 1;
    }
}

// A single-token decode step's attention with its RoPE and cache append fused (T = 1, position p = pos[0]). One CTA
// of 512 threads per q head h; positions go in chunks of 512. Every load that does not depend on p is issued first:
// the first two chunks' k and v (all rows below max_pos; rows at or past p are masked), the EXP table and the head's
// q / k / v inputs. The head's q and its kv head's new k are rotated into LDS; the first q head of each kv group
// writes the rotated k and the v to the caches at p; rows j < p come from the caches, j = p from LDS (no CTA uses
// the cached row p, so the writers race with no reader). Layouts keep each load instruction on few cache lines:
//   scores: 4 lanes per k row (16 bytes each, summed by two shuffles), 128 rows per pass, 4 passes per chunk;
//   P.V:    lane group gq = lane / 16 of wave w takes rows 32 i + 4 w + gq (i < 16), lane c = lane % 16 dims
//           4c .. 4c + 3: one dword of v per row, so a wave reads 4 rows x 64 bytes per instruction.
// Partial sums of e v stay below 64 * 2^15 * 127 < 2^31 within a chunk and add in int64 across chunks and waves.
// The integer rules are those of dec_rope_kv_kernel + dec_attention_kernel.
constexpr int ATT_NT = 512, ATT_PRE = 2;  // threads; chunks of ATT_NT positions prefetched into registers

// The o projection's dot products inside the attention step (FUSE_O): acc[n] += sum_h W_o[n, h] . o_h over d output
// channels, W_o the d x (nh * 64) W12 planes. Each head runs on og CTAs that all compute its attention (the K / V
// rows come from L2 after the first) and split the d channels into og ranges of cw: CTA (h, part) multiplies the
// head's 64 outputs by W_o's 64 columns of head h for channels part * cw .. part * cw + cw - 1 (loaded while the
// attention runs; og CTAs per head spread the d x 64 W12 bytes over og CUs) and adds the partial dots into acc
// with atomics whose results nothing waits for. The requantization into the residual happens in the consumers: the next RMSNorm-fused
// product folds requant(acc) into the residual it normalizes, and the residual-add product after it folds it into
// the stored residual and clears acc (w12_skinny_swiglu_kernel / w12_skinny_kernel with FOLD_O).
struct AttnO {
    const int8_t* lo;
    const uint8_t* nib;
    int32_t* acc;
    int d;
    int og, cw;  // CTAs per head; channels per CTA (<= ATT_NT: one per thread)
};
#ifndef KT_ATT_OG
#define KT_ATT_OG 8  // CTAs per head in the o-projection step
#endif

template <bool FUSE_O>
__global__ __launch_bounds__(ATT_NT) void dec_attention_step_kernel(const int8_t* __restrict__ qkv,
                                                                    const int32_t* __restrict__ pos,
                                                                    int8_t* __restrict__ kc, int8_t* __restrict__ vc,
                                                                    int nh, int nkv, const int16_t* __restrict__ cosT,
                                                                    const int16_t* __restrict__ sinT,
                                                                    const int32_t* __restrict__ exp_tab,
                                                                    int8_t* __restrict__ o, int max_pos, AttnO fo) {
    constexpr int HD = 64, HH = 32, NWV = ATT_NT / 64, KP = ATT_NT / 128, VR = ATT_NT / 32;
    extern __shared__ int s_sc[];  // max_pos: the scores, then the weights
    __shared__ int s_exp[1024];
    __shared__ int s_red[2][NWV];
    __shared__ int64_t s_acc[NWV][HD];
    __shared__ __attribute__((aligned(16))) int8_t s_q[HD], s_k[HD], s_v[HD];
    const int h = FUSE_O ? (int)blockIdx.x / fo.og : (int)blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int part = FUSE_O ? (int)blockIdx.x % fo.og : 0;
    const int rep = nh / nkv, g = h / rep;
    const size_t rstride = (size_t)nkv * HD;
    const int8_t* kg = kc + (size_t)g * HD;
    const int8_t* vg = vc + (size_t)g * HD;
    const int kq = tid & 3, kr = tid >> 2;      // scores: 16-byte quarter kq of row kr + 128 i
    const int gq = lane >> 4, c16 = lane & 15;  // P.V: rows 32 i + 4 w + gq, dims 4 c16 ..

    v4i K[ATT_PRE][KP];
    int V[ATT_PRE][VR];
#pragma unroll
    for (int c = 0; c < ATT_PRE; c++) {
#pragma unroll
        for (int i = 0; i < KP; i++) {
            const int j = c * ATT_NT + 128 * i + kr;
            K[c][i] = j < max_pos ? *reinterpret_cast<const v4i*>(kg + (size_t)j * rstride + 16 * kq) : v4i{};
        }
#pragma unroll
        for (int i = 0; i < VR; i++) {
            const int j = c * ATT_NT + 32 * i + 4 * w + gq;
            V[c][i] = j < max_pos ? *reinterpret_cast<const int*>(vg + (size_t)j * rstride + 4 * c16) : 0;
        }
    }
    int ex[1024 / ATT_NT];
#pragma unroll
    for (int i = 0; i < 1024 / ATT_NT; i++) ex[i] = exp_tab[tid + i * ATT_NT];
    const int ri = tid & (HH - 1), isk = (tid >> 5) & 1;
    int ra = 0, rb = 0;
    if (tid < 2 * HH) {
        const int8_t* src = qkv + (isk ? (nh + g) * HD : h * HD);
        ra = src[ri], rb = src[ri + HH];
    } else if (tid < 2 * HH + HD) {
        ra = qkv[(nh + nkv + g) * HD + tid - 2 * HH];
    }
    const int p = pos[0], L = p + 1;
    if (p < 0 || p >= max_pos) {  // a position outside the caches and tables: no access, a zero output
        if (!FUSE_O && tid < HD) o[h * HD + tid] = 0;  // (FUSE_O: the residual is left as a zero output leaves it)
        return;
    }
#pragma unroll
    for (int i = 0; i < 1024 / ATT_NT; i++) s_exp[tid + i * ATT_NT] = ex[i];
    if (tid < 2 * HH) {  // rotate q (threads 0..31) and k (32..63) pairs i, i + 32
        const int C = cosT[(size_t)p * HH + ri], S = sinT[(size_t)p * HH + ri];
        int8_t* dst = isk ? s_k : s_q;
        dst[ri] = (int8_t)clamp127(shift_round(ra * C - rb * S, 14));
        dst[ri + HH] = (int8_t)clamp127(shift_round(rb * C + ra * S, 14));
    } else if (tid < 2 * HH + HD) {
        s_v[tid - 2 * HH] = (int8_t)ra;
    }
    __syncthreads();
    if (h % rep == 0 && part == 0 && tid < HD) {
        kc[(size_t)p * rstride + g * HD + tid] = s_k[tid];
        vc[(size_t)p * rstride + g * HD + tid] = s_v[tid];
    }
    // FUSE_O: this head's W_o fragments for channel n = part * cw + tid: k32 blocks 2h, 2h + 1 of column block n / 32,
    // lane slot n % 32 + 32 kh in each (kh: the 16-k half), 16 lo bytes and 8 nib bytes per (block, half). Issued
    // after the q / k / v, position and rotation loads (vector loads complete in order, so a wait for those would
    // wait for these too) and before the score pass, whose operands are already in registers.
    v4i wl[4];
    v2i wn[4];
    const int on = part * fo.cw + tid;
    const bool has_col = FUSE_O && tid < fo.cw && on < fo.d;
    if constexpr (FUSE_O) {
        const int KB = nh * 2;  // k32 blocks per column block (K = nh * 64)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const size_t blk = (size_t)(on / 32) * KB + 2 * h + (q >> 1);
            const int slot = on % 32 + 32 * (q & 1);
            // W_o, read once per launch: non-temporal, as the other weight streams
            wl[q] = has_col ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(fo.lo + blk * 1024 + 16 * slot))
                            : v4i{};
            wn[q] = has_col ? __builtin_nontemporal_load(reinterpret_cast<const v2i*>(fo.nib + blk * 512 + 8 * slot))
                            : v2i{};
        }
    }
    const v4i q4 = *reinterpret_cast<const v4i*>(s_q + 16 * kq);
    const v4i knew = *reinterpret_cast<const v4i*>(s_k + 16 * kq);
    const int nch = (L + ATT_NT - 1) / ATT_NT;

    // scores into LDS, and their maximum
    int mx = INT_MIN;
    auto score = [&](int j, v4i k4) {
        if (j == p) k4 = knew;
        int sc = __builtin_amdgcn_sdot4(q4.x, k4.x, 0, false);
        sc = __builtin_amdgcn_sdot4(q4.y, k4.y, sc, false);
        sc = __builtin_amdgcn_sdot4(q4.z, k4.z, sc, false);
        sc = __builtin_amdgcn_sdot4(q4.w, k4.w, sc, false);
        sc = add_xor2(add_xor1(sc));  // the quad's sum (DPP)
        if (j < L) {
            if (kq == 0) s_sc[j] = sc;
            mx = sc > mx ? sc : mx;
        }
    };
#pragma unroll
    for (int c = 0; c < ATT_PRE; c++) {
#pragma unroll
        for (int i = 0; i < KP; i++) {
            if (c * ATT_NT + 128 * i >= L) break;  // uniform: every later row is past p
            score(c * ATT_NT + 128 * i + kr, K[c][i]);
        }
    }
    for (int c = ATT_PRE; c < nch; c++) {
#pragma unroll
        for (int i = 0; i < KP; i++) {
            const int j = c * ATT_NT + 128 * i + kr;
            score(j, j < p ? *reinterpret_cast<const v4i*>(kg + (size_t)j * rstride + 16 * kq) : v4i{});
        }
    }
    mx = wave_max_i32(mx);
    if (lane == 0) s_red[0][w] = mx;
    __syncthreads();
    mx = s_red[0][0];
#pragma unroll
    for (int q = 1; q < NWV; q++) mx = s_red[0][q] > mx ? s_red[0][q] : mx;

    // weights e_j = EXP[(m - s_j + 64) >> 7] in place of the scores, and their sum
    int den = 0;
    for (int j = tid; j < L; j += ATT_NT) {
        const int64_t idx = ((int64_t)mx - s_sc[j] + 64) >> 7;
        const int e = idx < 1024 ? s_exp[idx] : 0;
        s_sc[j] = e;
        den += e;
    }
    den = wave_sum_i32(den);
    if (lane == 0) s_red[1][w] = den;
    __syncthreads();

    // P.V
    const int vnew = *reinterpret_cast<const int*>(s_v + 4 * c16);
    int64_t accd[4] = {0, 0, 0, 0};
    auto pv_chunk = [&](int c, const int (&v)[VR]) {
        int a[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < VR; i++) {
            if (c * ATT_NT + 32 * i >= L) break;  // uniform: every later row is past p
            const int j = c * ATT_NT + 32 * i + 4 * w + gq;
            const int vv = j == p ? vnew : v[i];
            const int ew = s_sc[j < L ? j : 0];  // branch-free: always an in-range read
            const int e = j < L ? ew : 0;
#pragma unroll
            for (int b = 0; b < 4; b++) a[b] += __mul24(e, (int)(int8_t)(vv >> (8 * b)));  // |e v| < 2^23
        }
#pragma unroll
        for (int b = 0; b < 4; b++) accd[b] += add_xor32(add_xor16(a[b]));
    };
#pragma unroll
    for (int c = 0; c < ATT_PRE; c++) {
        if (c < nch) pv_chunk(c, V[c]);
    }
    for (int c = ATT_PRE; c < nch; c++) {
        int v[VR];
#pragma unroll
        for (int i = 0; i < VR; i++) {
            const int j = c * ATT_NT + 32 * i + 4 * w + gq;
            v[i] = j < p ? *reinterpret_cast<const int*>(vg + (size_t)j * rstride + 4 * c16) : 0;
        }
        pv_chunk(c, v);
    }
    if (lane < 16) {
#pragma unroll
        for (int b = 0; b < 4; b++) s_acc[w][4 * c16 + b] = accd[b];
    }
    __syncthreads();
    if (tid < HD) {
        int64_t sum = 0, dn = 0;
#pragma unroll
        for (int q = 0; q < NWV; q++) sum += s_acc[q][tid], dn += s_red[1][q];
        const int8_t ov = (int8_t)clamp127(div_round(sum, dn));
        if constexpr (FUSE_O) s_q[tid] = ov;  // s_q is free again: the head's output, the A side of the o product
        else o[h * HD + tid] = ov;
    }
    if constexpr (FUSE_O) {
        __syncthreads();
        const v4i* a4 = reinterpret_cast<const v4i*>(s_q);
        int asum = 0;  // -1920 * sum(a): the W12 offset term, the same for every column
#pragma unroll
        for (int q = 0; q < 4; q++) asum += sum4(a4[q]);
        if (has_col) {
            uint32_t v = 0u - 1920u * (uint32_t)asum;
#pragma unroll
            for (int q = 0; q < 4; q++) {  // k = 16 q .. 16 q + 15 of the head
                const v4i a = a4[q], lw = wl[q], hw = unpack_hi(wn[q]);
                int dl = 0, dh = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    dl = __builtin_amdgcn_sdot4(a[e], lw[e], dl, false);
                    dh = __builtin_amdgcn_sdot4(a[e], hw[e], dh, false);
                }
                v += (uint32_t)dl + ((uint32_t)dh << 8);
            }
            atomicAdd(fo.acc + on, (int)v);
        }
    }
}

// First stage of the greedy argmax: CTA b reduces its share of the n logits to one key (logit, then the lower
// index: ((v ^ 2^31) << 32) | (2^32 - 1 - i), the largest key is the first maximum), copies its share to
// record + step[0] * n when record is set, and CTA 0 advances the position by `advance`.
__global__ __launch_bounds__(256) void dec_argmax_part_kernel(const int32_t* __restrict__ logits, int n,
                                                              uint64_t* __restrict__ part,
                                                              int32_t* __restrict__ record,
                                                              const int32_t* __restrict__ step,
                                                              int32_t* __restrict__ pos, int advance) {
    __shared__ uint64_t s_key[4];
    const int tid = threadIdx.x, per = (n + gridDim.x - 1) / gridDim.x;
    const int i0 = blockIdx.x * per, i1 = min(n, i0 + per);
    int32_t* rec = record ? record + (size_t)step[0] * n : nullptr;
    uint64_t best = 0;
    for (int i = i0 + tid; i < i1; i += 256) {
        const int32_t v = logits[i];
        if (rec) rec[i] = v;
        const uint64_t key = ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
        best = key > best ? key : best;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = __shfl_xor(best, d);
        best = o > best ? o : best;
    }
    if ((tid & 63) == 0) s_key[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = s_key[0];
        for (int q = 1; q < 4; q++) b = s_key[q] > b ? s_key[q] : b;
        part[blockIdx.x] = b;
        if (blockIdx.x == 0 && pos) pos[0] += advance;
    }
}

// Second stage, fused with the next step's embedding: token = the best of nparts keys, r = emb[token], step += 1.
__global__ __launch_bounds__(256) void dec_embed_argmax_kernel(const uint64_t* __restrict__ part, int nparts,
                                                               const int16_t* __restrict__ emb, int d,
                                                               int32_t* __restrict__ r, int32_t* __restrict__ token,
                                                               int32_t* __restrict__ step) {
    __shared__ uint64_t s_key[4];
    __shared__ int s_tok;
    const int tid = threadIdx.x;
    uint64_t best = 0;
    for (int i = tid; i < nparts; i += 256) best = part[i] > best ? part[i] : best;
#pragma unroll
    for (int dd = 32; dd >= 1; dd >>= 1) {
        const uint64_t o = __shfl_xor(best, dd);
        best = o > best ? o : best;
    }
    if ((tid & 63) == 0) s_key[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = s_key[0];
        for (int q = 1; q < 4; q++) b = s_key[q] > b ? s_key[q] : b;
        s_tok = (int)(0xFFFFFFFFu - (uint32_t)b);
        if (token) token[0] = s_tok;
        if (step) step[0] += 1;
    }
    __syncthreads();
    const int16_t* e = emb + (size_t)s_tok * d;
    for (int i = tid; i < d; i += 256) r[i] = e[i];
}

__global__ void dec_advance_kernel(int32_t* pos, int by) {
    if (threadIdx.x == 0) pos[0] += by;
}

// ------------------------------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------------------------------

hipError_t launch_dec_embed(const int32_t* tokens, int T, const int16_t* emb, int d, int32_t* r, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    dec_embed_kernel<<<dim3((unsigned)T), dim3(256), 0, s>>>(tokens, emb, d, r);
    return hipGetLastError();
}

hipError_t launch_dec_rmsnorm(const int32_t* r, int T, int d, int8_t* q, int qs, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    dec_rmsnorm_kernel<<<dim3((unsigned)T), dim3(256), 0, s>>>(r, d, q, qs);
    return hipGetLastError();
}

hipError_t launch_dec_rope_kv(int8_t* qkv, int T, int nqkv, const int32_t* pos, int nh, int nkv, int hd,
                              const int16_t* cosT, const int16_t* sinT, int8_t* kc, int8_t* vc, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    dec_rope_kv_kernel<<<dim3((unsigned)T), dim3(256), 0, s>>>(qkv, nqkv, pos, nh, nkv, hd, cosT, sinT, kc, vc);
    return hipGetLastError();
}

hipError_t launch_dec_attention(const int8_t* qkv, int T, int nqkv, const int32_t* pos, const int8_t* kc,
                                const int8_t* vc, int nh, int nkv, const int32_t* exp_tab, int8_t* o, int max_pos,
                                hipStream_t s) {
    if (T <= 0) return hipSuccess;
    const size_t lds = (size_t)max_pos * sizeof(int);
    dec_attention_kernel<<<dim3((unsigned)(T * nh)), dim3(256), lds, s>>>(qkv, nqkv, pos, kc, vc, nh, nkv, exp_tab, o,
                                                                          max_pos);
    return hipGetLastError();
}

hipError_t launch_dec_argmax(const int32_t* logits, int n, int32_t* token, int32_t* record, int32_t* step,
                             hipStream_t s) {
    dec_argmax_kernel<<<dim3(1), dim3(1024), 0, s>>>(logits, n, token, record, step);
    return hipGetLastError();
}

template <bool FUSE_O>
static hipError_t attention_step(const int8_t* qkv, const int32_t* pos, int8_t* kc, int8_t* vc, int nh, int nkv,
                                 const int16_t* cosT, const int16_t* sinT, const int32_t* exp_tab, int8_t* o,
                                 int max_pos, const AttnO& fo, hipStream_t s) {
    const size_t lds = (size_t)max_pos * sizeof(int);
    static size_t lds_static = 0, lds_max = 0;  // queried once per process
    if (lds_max == 0) {
        hipFuncAttributes fa;
        int dev = 0, mx = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (e == hipSuccess)
            e = hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(&dec_attention_step_kernel<FUSE_O>));
        if (e != hipSuccess) return e;
        lds_static = fa.sharedSizeBytes, lds_max = (size_t)mx;
    }
    if (lds_static + lds > lds_max) return hipErrorInvalidValue;  // max_pos too long for one CTA
    const unsigned ctas = (unsigned)nh * (FUSE_O ? (unsigned)fo.og : 1u);
    dec_attention_step_kernel<FUSE_O><<<dim3(ctas), dim3(ATT_NT), lds, s>>>(qkv, pos, kc, vc, nh, nkv, cosT, sinT,
                                                                            exp_tab, o, max_pos, fo);
    return hipGetLastError();
}

hipError_t launch_dec_attention_step(const int8_t* qkv, const int32_t* pos, int8_t* kc, int8_t* vc, int nh, int nkv,
                                     const int16_t* cosT, const int16_t* sinT, const int32_t* exp_tab, int8_t* o,
                                     int max_pos, hipStream_t s) {
    return attention_step<false>(qkv, pos, kc, vc, nh, nkv, cosT, sinT, exp_tab, o, max_pos, AttnO{}, s);
}

hipError_t launch_dec_attention_o_step(const int8_t* qkv, const int32_t* pos, int8_t* kc, int8_t* vc, int nh,
                                       int nkv, const int16_t* cosT, const int16_t* sinT, const int32_t* exp_tab,
                                       int max_pos, const int8_t* wo_lo, const uint8_t* wo_nib, int d, int32_t* acc,
                                       hipStream_t s) {
    if (d < 1 || d > 1024 || nh * 64 > KT_SMALL_KP) return hipErrorInvalidValue;
    const int og = std::max(KT_ATT_OG, (d + ATT_NT - 1) / ATT_NT), cw = (d + og - 1) / og;
    const AttnO fo{wo_lo, wo_nib, acc, d, og, cw};
    return attention_step<true>(qkv, pos, kc, vc, nh, nkv, cosT, sinT, exp_tab, nullptr, max_pos, fo, s);
}

hipError_t launch_dec_argmax_part(const int32_t* logits, int n, uint64_t* part, int nparts, int32_t* record,
                                  const int32_t* step, int32_t* pos, int advance, hipStream_t s) {
    dec_argmax_part_kernel<<<dim3((unsigned)nparts), dim3(256), 0, s>>>(logits, n, part, record, step, pos, advance);
    return hipGetLastError();
}

hipError_t launch_dec_embed_argmax(const uint64_t* part, int nparts, const int16_t* emb, int d, int32_t* r,
                                   int32_t* token, int32_t* step, hipStream_t s) {
    dec_embed_argmax_kernel<<<dim3(1), dim3(256), 0, s>>>(part, nparts, emb, d, r, token, step);
    return hipGetLastError();
}

hipError_t launch_dec_advance(int32_t* pos, int by, hipStream_t s) {
    dec_advance_kernel<<<dim3(1), dim3(64), 0, s>>>(pos, by);
    return hipGetLastError();
}

}  // namespace kt
