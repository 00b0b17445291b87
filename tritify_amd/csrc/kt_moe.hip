// The MoE layer of benchmark config 4 on gfx950: routing, bucketing, the ragged grouped W12 GEMM and the weighted
// combine. The reference runs a MoE layer token by token (MoeMlp::forward_routed / forward_one_int,
// crates/01-engine/kt-core/src/layers.rs:928-936, 988-1020), each selected expert called with one row; here the
// tokens are bucketed by expert and every expert's rows run as one ragged group of a single grouped GEMM launch.
// Integer sums do not depend on the order, so the bytes equal the per-token evaluation.
//
//   route   one wave per token: top-k router codes (descending, ties to the lower index, layers.rs:800-805) and
//           their sigmoid-table weights;
//   bucket  one CTA per expert: the tokens that chose it, in increasing token order (a block prefix sum, so the
//           order is deterministic), and each (token, choice)'s row within the group; group E (the shared expert)
//           lists every token;
//   grouped GEMM  persistent CTAs walk the (group row tile, column tile) space, A rows gathered through the token
//           lists (or contiguous per group), each group's own W12 weights and scales, the mainloop of kt_w12_core.h;
//           epilogues: per-channel int8 requant, or SwiGLU on an interleaved gate/up matrix;
//   combine one CTA per token: sum_i cw_i d_i + 4096 d_shared, requantized to int8.

#include <hip/hip_runtime.h>

#include <type_traits>
#include <limits.h>
#include <stdint.h>

#include "kt_kernels.h"
#include "kt_w12_core.h"

namespace kt {

// round_half_away(r / 16) clamped to [-127, 127]: the sigmoid table index of a router code.
__device__ __forceinline__ int sig_index(int r) {
    const uint32_t a = r < 0 ? 0u - (uint32_t)r : (uint32_t)r;
    uint32_t q = (a + 8) >> 4;
    q = q > 127 ? 127 : q;
    return r < 0 ? -(int)q : (int)q;
}

// One wave per token: top_k rounds of a wave-wide max over (code, -index) keys. Up to 16 codes per lane (E <= 1024).
__global__ __launch_bounds__(256) void moe_route_kernel(const int32_t* __restrict__ logits, int T, int E, int top_k,
                                                        const int16_t* __restrict__ sig, int32_t* __restrict__ sel,
                                                        int32_t* __restrict__ cw) {
    constexpr int MAXV = 16;
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // the whole wave
    const int32_t* r = logits + (size_t)t * E;
    uint64_t key[MAXV];
#pragma unroll
    for (int q = 0; q < MAXV; q++) {
        const int e = lane + 64 * q;
        // the code with its sign bit flipped orders as unsigned; the low word orders lower indices first
        key[q] = e < E ? ((uint64_t)((uint32_t)r[e] ^ 0x80000000u) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e) : 0;
    }
    for (int it = 0; it < top_k; it++) {
        uint64_t best = 0;
#pragma unroll
        for (int q = 0; q < MAXV; q++) best = key[q] > best ? key[q] : best;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const uint64_t o = __shfl_xor(best, d);
            best = o > best ? o : best;
        }
        const int e = (int)(0xFFFFFFFFu - (uint32_t)best);
        const int code = (int)((uint32_t)(best >> 32) ^ 0x80000000u);
        if (lane == (e & 63)) {
#pragma unroll
            for (int q = 0; q < MAXV; q++)
                if (q == (e >> 6)) key[q] = 0;  // taken
        }
        if (lane == 0) {
            sel[(size_t)t * top_k + it] = e;
            cw[(size_t)t * top_k + it] = sig[sig_index(code) + 127];
        }
    }
}

// One CTA per group g <= E: list[g * T + j] = the j-th token (increasing) that chose g, pos[t * top_k + i] = j for
// (t, its choice i == g), count[g] = the group size. Group E (the shared expert) is every token. A pass covers
// 1024 x BK_TPT tokens, thread tid the BK_TPT consecutive tokens from BK_TPT * tid, so one block scan of the
// threads' hit counts orders a pass's hits by token. MAXK >= top_k bounds the unrolled selection loads (0: a loop
// over top_k).
constexpr int BK_NT = 1024, BK_TPT = 4;
template <int MAXK>
__global__ __launch_bounds__(BK_NT) void moe_bucket_kernel(const int32_t* __restrict__ sel, int T, int E, int top_k,
                                                           int32_t* __restrict__ list, int32_t* __restrict__ pos,
                                                           int32_t* __restrict__ count) {
    __shared__ int scr[2 * (BK_NT / 64)];
    const int g = blockIdx.x, tid = threadIdx.x;
    int32_t* lg = list + (size_t)g * T;
    if (g == E) {
        for (int t = tid; t < T; t += BK_NT) lg[t] = t;
        if (tid == 0) count[E] = T;
        return;
    }
    int base = 0;
    for (int t0 = 0; t0 < T; t0 += BK_NT * BK_TPT) {
        const int tb = t0 + BK_TPT * tid;
        int hit[BK_TPT], n = 0;
#pragma unroll
        for (int j = 0; j < BK_TPT; j++) {
            const int t = tb + j;
            hit[j] = -1;
            if constexpr (MAXK > 0) {  // every load of the token's selections in flight before the first compare
                int32_t v[MAXK];
#pragma unroll
                for (int i = 0; i < MAXK; i++) v[i] = t < T && i < top_k ? sel[(size_t)t * top_k + i] : -1;
#pragma unroll
                for (int i = 0; i < MAXK; i++)
                    if (v[i] == g) hit[j] = i;
            } else if (t < T) {
                for (int i = 0; i < top_k; i++)
                    if (sel[(size_t)t * top_k + i] == g) hit[j] = i;
            }
            n += hit[j] >= 0 ? 1 : 0;
        }
        int ex, ez, tot, tz;
        block_scan2<BK_NT>(n, 0, ex, ez, tot, tz, scr);
        int p = base + ex;
#pragma unroll
        for (int j = 0; j < BK_TPT; j++)
            if (hit[j] >= 0) {
                lg[p] = tb + j;
                pos[(size_t)(tb + j) * top_k + hit[j]] = p;
                p++;
            }
        base += tot;
    }
    if (tid == 0) count[g] = base;
}

// The grouped GEMM's CTA tiles: the dense GEMM's 128 x 128 (4 waves along N, 4 x 1 tiles of 32x32 each), and a
// 64 x 128 tile (2 x 1 tiles per wave) for a group's last row tile when it holds at most 64 rows, so ragged group
// tails run half the MFMA work of a full tile.
typedef W12Tile<1, 4, 1, 4> GTile;
typedef W12Tile<1, 2, 1, 4> GTileH;

// The epilogue of one grouped output tile (rows row0 .. row0 + rows - 1 of group g, columns n0 .. n0 + BN - 1): the
// int8 requant (EPI_I8) or the SwiGLU of the tile's gate/up block pairs (EPI_SWIGLU), staged through `smem`
// (BM x BN bytes, free once the mainloop is done).
// XR (the 288-row DMA tile): xs holds the strip of rows 256 .. 287, requantized into the same staged tile.
template <class C, int EPI, int XR = 0>
__device__ __forceinline__ void grouped_epilogue(const v16i (&acc0)[C::WTM][1], const v16i (&acc1)[C::WTM][1],
                                                 const int* sRow, int g, int row0, int rows, int n0, const int* sOff,
                                                 int N, const int32_t* __restrict__ mant,
                                                 const int32_t* __restrict__ shift, const int16_t* sSilu,
                                                 int h_shift, int8_t* __restrict__ y, int ystride, int8_t* smem,
                                                 const DmaStrip* xs = nullptr) {
    constexpr int NT = C::NT, BM = C::BM + XR, BN = C::BN;
    const int tid = tid_now();
    const int32_t* gm = mant + (size_t)g * N;
    const int32_t* gs = shift + (size_t)g * N;
    int8_t* yg = y + (size_t)(sOff[g] + row0) * ystride;
    if constexpr (EPI == KT_EPI_I8) {
        w12_requant_tile8<C>(acc0, acc1, sRow, gm, gs, n0, N, [](int n) { return n; }, smem);
        if constexpr (XR != 0) w12_requant_strip8<BN>(*xs, sRow, gm, gs, n0, N, [](int n) { return n; }, smem);
        __syncthreads();
        constexpr int CH = BM * BN / 16;
        const bool vec = n0 + BN <= N && (ystride & 15) == 0;
#pragma unroll
        for (int i = 0; i < (CH + NT - 1) / NT; i++) {
            const int idx = tid + NT * i, r = idx / (BN / 16), c = (idx % (BN / 16)) * 16;
            if (idx >= CH || r >= rows) continue;
            const v4i v = *reinterpret_cast<const v4i*>(smem + r * BN + c);
            int8_t* dst = yg + (size_t)r * ystride + n0 + c;
            if (vec) {
                *reinterpret_cast<v4i*>(dst) = v;
            } else {  // bytes by shifts: an addressed vector would live in scratch memory
#pragma unroll
                for (int q = 0; q < 16; q++)
                    if (n0 + c + q < N) dst[q] = (int8_t)((uint32_t)v[q >> 2] >> (8 * (q & 3)));
            }
        }
    } else {
        const int F = N / 2;
        auto chan = [F](int n) {
            const int blk = n >> 5;
            return (blk & 1) * F + (blk >> 1) * 32 + (n & 31);
        };
        w12_requant_tile8<C>(acc0, acc1, sRow, gm, gs, n0, N, chan, smem);
        if constexpr (XR != 0) w12_requant_strip8<BN>(*xs, sRow, gm, gs, n0, N, chan, smem);
        __syncthreads();
        // the tile's columns are gate/up block pairs: hidden units n0/2 .. n0/2 + units - 1
        const int units = (N - n0 < BN ? N - n0 : BN) / 2;
        for (int task = tid; task < BM * (BN / 32); task += NT) {
            const int r = task / (BN / 32), q = task % (BN / 32);  // row, 16-unit chunk
            if (r >= rows || 16 * q >= units) continue;
            // units 16 q .. 16 q + 15: 16 consecutive gate codes at gc0 (one 32-unit block holds them), their up codes
            // 32 bytes on; every table read is issued before the first is used
            const int gc0 = (q >> 1) * 64 + (q & 1) * 16;
            const v4i gv = *reinterpret_cast<const v4i*>(smem + r * BN + gc0);
            const v4i uv = *reinterpret_cast<const v4i*>(smem + r * BN + gc0 + 32);
            int sl[16];
#pragma unroll
            for (int t2 = 0; t2 < 16; t2++)
                sl[t2] = sSilu[(int)(int8_t)((uint32_t)gv[t2 >> 2] >> (8 * (t2 & 3))) + 127];
            v4i out = {0, 0, 0, 0};
#pragma unroll
            for (int t2 = 0; t2 < 16; t2++) {
                const int uq = (int)(int8_t)((uint32_t)uv[t2 >> 2] >> (8 * (t2 & 3)));
                const uint32_t hb = (uint32_t)(uint8_t)shift_rq8(sl[t2] * uq, h_shift);
                out[t2 >> 2] |= (int)(hb << (8 * (t2 & 3)));
            }
            *reinterpret_cast<v4i*>(yg + (size_t)r * ystride + n0 / 2 + 16 * q) = out;
        }
    }
}

// One output tile of the grouped GEMM: rows row0 .. row0 + rows - 1 of group g, columns n0 .. n0 + BN - 1.
template <class C, int EPI>
__device__ __forceinline__ void grouped_tile(const __amdgpu_buffer_rsrc_t rA, uint32_t x_bytes,
                                             const int32_t* __restrict__ list, int list_stride, int g, int row0,
                                             int rows, int n0, const int* sOff, const int8_t* __restrict__ wlo,
                                             const uint8_t* __restrict__ wnib, size_t glo, int N, int kp,
                                             const int32_t* __restrict__ mant, const int32_t* __restrict__ shift,
                                             const int16_t* sSilu, int h_shift, int8_t* __restrict__ y, int ystride,
                                             int8_t* smem, int* sRow) {
    constexpr int NT = C::NT, BM = C::BM, BN = C::BN, AL = C::AL, AC = C::AC;
    static_assert(C::RING >= BM * BN, "the int8 output tile reuses the A ring");
    const int tid = tid_now(), lane = tid & 63, wave = tid >> 6;
    const int KB = kp / 32;
    uint32_t oa[AL];
#pragma unroll
    for (int i = 0; i < AL; i++) {
        const int idx = tid + NT * i, r = idx >> 2;
        if (idx < AC && r < rows) {
            const int xr = list ? list[(size_t)g * list_stride + row0 + r] : sOff[g] + row0 + r;
            oa[i] = (uint32_t)xr * (uint32_t)kp + 16 * (idx & 3);
        } else {
            oa[i] = x_bytes;  // out of range whatever the k offset: reads zero
        }
    }
    const int cb0 = n0 / 32, ncb = (N - n0 + 31) / 32 < BN / 32 ? (N - n0 + 31) / 32 : BN / 32;
    const int8_t* gl = wlo + (size_t)g * glo;
    const uint8_t* gn = wnib + (size_t)g * (glo / 2);
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(gl + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(gn + (size_t)cb0 * KB * 512, (uint32_t)ncb * KB * 512);
    const int wn = wave % C::WN;
    uint32_t ob[1] = {(uint32_t)(wn * KB) * 1024 + 16 * lane}, on[1] = {(uint32_t)(wn * KB) * 512 + 8 * lane};

    v16i acc0[C::WTM][1], acc1[C::WTM][1];
    int rsum[AL];
    w12_mainloop<C>(rA, oa, rL, rN, ob, on, kp / C::BK, smem, acc0, acc1, rsum);
    w12_row_sums<C>(rsum, sRow);
    grouped_epilogue<C, EPI>(acc0, acc1, sRow, g, row0, rows, n0, sOff, N, mant, shift, sSilu, h_shift, y, ystride,
                             smem);
}

// The 256 x 128 tile of the DMA-fed grouped kernel (w12_mainloop_dma, 8 waves): the lanes' A pieces are gathered
// rows of group g, rows at or past `rows` read zero. XR: the 288-row tile (a group's last tile absorbing a tail of
// up to 32 rows).
typedef W12Tile<2, 4, 1, 2, 4> GTileD;
template <int EPI, int XR = 0>
__device__ __forceinline__ void grouped_tile_dma(const __amdgpu_buffer_rsrc_t rA, uint32_t x_bytes,
                                                 const int32_t* __restrict__ list, int list_stride, int g, int row0,
                                                 int rows, int n0, const int* sOff, const int8_t* __restrict__ wlo,
                                                 const uint8_t* __restrict__ wnib, size_t glo, int N, int kp,
                                                 const int32_t* __restrict__ mant, const int32_t* __restrict__ shift,
                                                 const int16_t* sSilu, int h_shift, int8_t* __restrict__ y,
                                                 int ystride, int8_t* ring, int* sRow) {
    constexpr int BN = GTileD::BN;
    const int tid = tid_now(), lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KB = kp / 32;
    uint32_t va[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = dma_a_row(w, lane, j);
        if (r < rows) {
            const int xr = list ? list[(size_t)g * list_stride + row0 + r] : sOff[g] + row0 + r;
            va[j] = (uint32_t)xr * (uint32_t)kp + dma_a_chunk(lane);
        } else {
            va[j] = x_bytes;  // out of range whatever the k offset: reads zero
        }
    }
    DmaStrip xs;
    if constexpr (XR != 0) {
        const int r = dma_x_row(w, lane);
        if (r < rows) {
            const int xr = list ? list[(size_t)g * list_stride + row0 + r] : sOff[g] + row0 + r;
            xs.vx = (uint32_t)xr * (uint32_t)kp + dma_x_byte(w, lane);
        } else {
            xs.vx = x_bytes;
        }
    }
    const int cb0 = n0 / 32, ncb = (N - n0 + 31) / 32 < BN / 32 ? (N - n0 + 31) / 32 : BN / 32;
    const int8_t* gl = wlo + (size_t)g * glo;
    const uint8_t* gn = wnib + (size_t)g * (glo / 2);
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(gl + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(gn + (size_t)cb0 * KB * 512, (uint32_t)ncb * KB * 512);
    v16i acc0[4][1], acc1[4][1];
    w12_mainloop_dma<KT_DMA_NS, false, XR>(rA, rL, rN, va[0], va[1], kp, ring, acc0, acc1, sRow, &xs);
    grouped_epilogue<GTileD, EPI, XR>(acc0, acc1, sRow, g, row0, rows, n0, sOff, N, mant, shift, sSilu, h_shift, y,
                                      ystride, ring, &xs);
}

// Row tiles of a group of c rows on the DMA-fed kernel: 256-row tiles, the last absorbing a tail of up to 32 rows
// (the 288-row tile) rather than taking a tile of its own that would stream the group's weights again.
__device__ __forceinline__ int dma_row_tiles(int c) {
    const int t = c & 255;
    return c > 256 && t != 0 && t <= KT_DMA_XR ? c >> 8 : (c + 255) >> 8;
}

// The ragged grouped W12 GEMM on 256-row tiles fed by LDS DMA, for products with enough rows to give every CU a
// tile: one CTA of 8 waves per CU, each group cut into 256-row tiles whose weights cross the L2 -> CU path once per
// tile (against once per 128 rows for w12_grouped_kernel). A group's last row tile runs on the DMA tile when it
// holds more than 128 rows, else on a 128- or 64-row tile of the register mainloop (8 waves, 2 along M) in the
// same pass. Arguments, tile order and results are w12_grouped_kernel's (below).
template <int EPI>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void w12_grouped_dma_kernel(
    const int8_t* __restrict__ x, uint32_t x_bytes, const int32_t* __restrict__ list, int list_stride,
    const int32_t* __restrict__ count, int groups, const int8_t* __restrict__ wlo, const uint8_t* __restrict__ wnib,
    size_t glo, int N, int kp, const int32_t* __restrict__ mant, const int32_t* __restrict__ shift,
    const int16_t* __restrict__ silu, int h_shift, int8_t* __restrict__ y, int ystride,
    int32_t* __restrict__ off_out, int rows_one) {
    typedef W12Tile<2, 2, 1, 4, 4> GT128;
    typedef W12Tile<2, 1, 1, 4, 4> GT64;
    static_assert(GT128::NT == 512 && GT64::NT == 512 && GT128::BN == 128 && GT64::BN == 128, "one tile space");
    static_assert(GT128::RING <= KT_DMA_NS * KT_DMA_STAGE, "the register tiles' A rings fit the DMA ring");
    static_assert((256 + KT_DMA_XR) * 128 <= KT_DMA_NS * dma_stage_x<KT_DMA_XR>(), "the 288-row output tile fits");
    constexpr int NT = 512, BM = 256, BN = 128;
    extern __shared__ __attribute__((aligned(16))) int8_t ring[];
    __shared__ int sRow[BM + KT_DMA_XR];
    __shared__ int sRpre[KT_MAX_GROUPS + 1], sOff[KT_MAX_GROUPS + 1];
    __shared__ int scr[16];
    __shared__ int16_t sSilu[256];

    const int tid = threadIdx.x;
    int carry_r = 0, carry_o = 0;
    for (int g0 = 0; g0 < groups; g0 += NT) {
        const int g = g0 + tid, c = g < groups ? (count ? count[g] : rows_one) : 0;
        int er, eo, tr, to;
        block_scan2<NT>(dma_row_tiles(c), c, er, eo, tr, to, scr);
        if (g < groups) sRpre[g] = carry_r + er, sOff[g] = carry_o + eo;
        carry_r += tr, carry_o += to;
    }
    if (tid == 0) sRpre[groups] = carry_r, sOff[groups] = carry_o;
    if (EPI == KT_EPI_SWIGLU && tid < 256) sSilu[tid] = silu[tid < 255 ? tid : 254];
    __syncthreads();
    if (off_out && blockIdx.x == 0)
        for (int g = tid; g <= groups; g += NT) off_out[g] = sOff[g];

    const int tiles_n = (N + BN - 1) / BN, total = sRpre[groups] * tiles_n;
    const int nx = gridDim.x >> 3, xcd = blockIdx.x & 7, per = (total + 7) >> 3;
    const int t_end = min(total, (xcd + 1) * per);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(x, x_bytes);
    for (int t = xcd * per + (blockIdx.x >> 3); t < t_end; t += nx) {
        const int rt = t / tiles_n, n0 = (t - rt * tiles_n) * BN;
        int lo = 0, hi = groups - 1;  // the last group whose first row tile is <= rt (it is not empty)
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (sRpre[mid] <= rt) lo = mid;
            else hi = mid - 1;
        }
        const int g = lo, row0 = (rt - sRpre[g]) * BM, cnt = sOff[g + 1] - sOff[g];
        // the group's last tile holds the rest (at most BM + KT_DMA_XR rows), the others BM
        const int rows = rt == sRpre[g + 1] - 1 ? cnt - row0 : BM;
        if (rows > BM)  // uniform: a tail of at most KT_DMA_XR rows on the 288-row tile
            grouped_tile_dma<EPI, KT_DMA_XR>(rA, x_bytes, list, list_stride, g, row0, rows, n0, sOff, wlo, wnib, glo, N,
                                             kp, mant, shift, sSilu, h_shift, y, ystride, ring, sRow);
        else if (rows > GT128::BM)
            grouped_tile_dma<EPI>(rA, x_bytes, list, list_stride, g, row0, rows, n0, sOff, wlo, wnib, glo, N, kp, mant,
                                  shift, sSilu, h_shift, y, ystride, ring, sRow);
        else if (rows > GT64::BM)
            grouped_tile<GT128, EPI>(rA, x_bytes, list, list_stride, g, row0, rows, n0, sOff, wlo, wnib, glo, N, kp,
                                     mant, shift, sSilu, h_shift, y, ystride, ring, sRow);
        else
            grouped_tile<GT64, EPI>(rA, x_bytes, list, list_stride, g, row0, rows, n0, sOff, wlo, wnib, glo, N, kp,
                                    mant, shift, sSilu, h_shift, y, ystride, ring, sRow);
        __syncthreads();  // the next tile's prologue rewrites the ring
    }
}

// Ragged grouped W12 GEMM. Group g has count[g] rows (count null: one group of rows_one rows, a dense product); its
// row j is x row list[g * list_stride + j] (list != null) or x row off[g] + j (off = the exclusive prefix of count);
// its weights are the W12 planes at wlo + g * glo (lo) and wnib + g * glo / 2 (nib), n x k with per-channel scales
// mant/shift + g * n; its output row j is y row off[g] + j (row stride ystride). EPI_I8: y = the int8 requant of the
// n columns. EPI_SWIGLU: the weights are a gate/up matrix packed with the 32-row interleave (n = 2F), the scales in
// natural order (gate 0..F-1, up F..2F-1), and y = clamp(requant(silu[gq + 127] * uq, 1, h_shift)) over F columns.
// off_out (optional) receives off[0..groups]. The tile space is 128-row tiles x 128-column tiles; with TAILS =
// GT_MIXED a tile of at most 64 rows (a ragged group tail) runs the 64-row tile, at half the MFMA work, in the same
// pass (right after its group's other tiles, while their weights are in cache); GT_ALL runs every tile on the
// 128-row tile (one group: a dense product, whose only short tile is its last). Persistent:
// CTA b (XCD b % 8) takes the tiles of its XCD's contiguous share of the tile space, so an XCD's L2 serves
// consecutive column tiles of the same rows and consecutive groups' weights.
enum { GT_ALL = 0, GT_MIXED = 1, GT_HALF = 2 };

template <int EPI, int TAILS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void w12_grouped_kernel(
    const int8_t* __restrict__ x, uint32_t x_bytes, const int32_t* __restrict__ list, int list_stride,
    const int32_t* __restrict__ count, int groups, const int8_t* __restrict__ wlo, const uint8_t* __restrict__ wnib,
    size_t glo, int N, int kp, const int32_t* __restrict__ mant, const int32_t* __restrict__ shift,
    const int16_t* __restrict__ silu, int h_shift, int8_t* __restrict__ y, int ystride,
    int32_t* __restrict__ off_out, int rows_one) {
    // the tile space and the computing tile: 128-row tiles (GT_MIXED: GTileH for a tail of at most 64 rows), or
    // 64-row tiles throughout (GT_HALF: one group whose 128-row tiles would leave CUs idle, a prefill batch)
    typedef typename std::conditional<TAILS == GT_HALF, GTileH, GTile>::type C;
    typedef C CT;
    static_assert(GTileH::NT == C::NT && GTileH::BN == C::BN && GTileH::RING <= C::RING, "one tile space");
    constexpr int NT = C::NT, BM = C::BM, BN = C::BN;
    __shared__ __attribute__((aligned(16))) int8_t smem[CT::RING];
    __shared__ int sRow[CT::BM];
    __shared__ int sRpre[KT_MAX_GROUPS + 1], sOff[KT_MAX_GROUPS + 1];
    __shared__ int scr[8];
    __shared__ int16_t sSilu[256];

    const int tid = threadIdx.x;
    int carry_r = 0, carry_o = 0;
    for (int g0 = 0; g0 < groups; g0 += NT) {
        const int g = g0 + tid, c = g < groups ? (count ? count[g] : rows_one) : 0;
        int er, eo, tr, to;
        block_scan2<NT>((c + BM - 1) / BM, c, er, eo, tr, to, scr);
        if (g < groups) sRpre[g] = carry_r + er, sOff[g] = carry_o + eo;
        carry_r += tr, carry_o += to;
    }
    if (tid == 0) sRpre[groups] = carry_r, sOff[groups] = carry_o;
    if (EPI == KT_EPI_SWIGLU) sSilu[tid] = silu[tid < 255 ? tid : 254];
    __syncthreads();
    if (off_out && blockIdx.x == 0)
        for (int g = tid; g <= groups; g += NT) off_out[g] = sOff[g];

    const int tiles_n = (N + BN - 1) / BN, total = sRpre[groups] * tiles_n;
    const int nx = gridDim.x >> 3, xcd = blockIdx.x & 7, per = (total + 7) >> 3;
    const int t_end = min(total, (xcd + 1) * per);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(x, x_bytes);
    for (int t = xcd * per + (blockIdx.x >> 3); t < t_end; t += nx) {
        const int rt = t / tiles_n, n0 = (t - rt * tiles_n) * BN;
        int lo = 0, hi = groups - 1;  // the last group whose first row tile is <= rt (it is not empty)
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (sRpre[mid] <= rt) lo = mid;
            else hi = mid - 1;
        }
        const int g = lo, row0 = (rt - sRpre[g]) * BM, cnt = sOff[g + 1] - sOff[g];
        const int rows = cnt - row0 < BM ? cnt - row0 : BM;
        if (TAILS == GT_MIXED && rows <= GTileH::BM)  // uniform: a ragged tail on the 64-row tile
            grouped_tile<GTileH, EPI>(rA, x_bytes, list, list_stride, g, row0, rows, n0, sOff, wlo, wnib, glo, N, kp,
                                      mant, shift, sSilu, h_shift, y, ystride, smem, sRow);
        else
            grouped_tile<CT, EPI>(rA, x_bytes, list, list_stride, g, row0, rows, n0, sOff, wlo, wnib, glo, N, kp,
                                  mant, shift, sSilu, h_shift, y, ystride, smem, sRow);
        __syncthreads();  // the next tile's prologue rewrites the ring
    }
}

// One CTA per token: y = 4096 d[off[E] + t] + sum_i cw_i d[off[e_i] + pos_i] (int32 is exact: |cw| < 2^15,
// top_k <= 32), out = clamp(requant(y, 1, out_shift)), 16 columns per thread.
__global__ __launch_bounds__(256) void moe_combine_kernel(const int8_t* __restrict__ d, const int32_t* __restrict__ off,
                                                          const int32_t* __restrict__ sel,
                                                          const int32_t* __restrict__ cw,
                                                          const int32_t* __restrict__ pos, int H, int E, int top_k,
                                                          int out_shift, int8_t* __restrict__ out) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const int8_t* ds = d + (size_t)(off[E] + t) * H;
    for (int c = tid; c < H / 16; c += 256) {
        int y[16];
        const v4i vs = *reinterpret_cast<const v4i*>(ds + 16 * c);
        const int8_t* bs = reinterpret_cast<const int8_t*>(&vs);
#pragma unroll
        for (int q = 0; q < 16; q++) y[q] = 4096 * bs[q];
        for (int i = 0; i < top_k; i++) {
            const int e = sel[(size_t)t * top_k + i], w = cw[(size_t)t * top_k + i];
            const int8_t* dr = d + (size_t)(off[e] + pos[(size_t)t * top_k + i]) * H;
            const v4i v = *reinterpret_cast<const v4i*>(dr + 16 * c);
            const int8_t* b = reinterpret_cast<const int8_t*>(&v);
#pragma unroll
            for (int q = 0; q < 16; q++) y[q] += w * b[q];
        }
        v4i o;
        int8_t* ob = reinterpret_cast<int8_t*>(&o);
#pragma unroll
        for (int q = 0; q < 16; q++) ob[q] = (int8_t)shift_rq8(y[q], out_shift);
        *reinterpret_cast<v4i*>(out + (size_t)t * H + 16 * c) = o;
    }
}

// ------------------------------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------------------------------

hipError_t launch_moe_route(const int32_t* logits, int T, int E, int top_k, const int16_t* sig, int32_t* sel,
                            int32_t* cw, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    if (E < 1 || E > 1024 || top_k < 1 || top_k > E || top_k > 32) return hipErrorInvalidValue;
    moe_route_kernel<<<dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s>>>(logits, T, E, top_k, sig, sel, cw);
    return hipGetLastError();
}

hipError_t launch_moe_bucket(const int32_t* sel, int T, int E, int top_k, int32_t* list, int32_t* pos,
                             int32_t* count, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    if (E < 1 || E + 1 > KT_MAX_GROUPS || top_k < 1 || top_k > E) return hipErrorInvalidValue;
    if (top_k <= 8)
        moe_bucket_kernel<8><<<dim3((unsigned)(E + 1)), dim3(BK_NT), 0, s>>>(sel, T, E, top_k, list, pos, count);
    else
        moe_bucket_kernel<0><<<dim3((unsigned)(E + 1)), dim3(BK_NT), 0, s>>>(sel, T, E, top_k, list, pos, count);
    return hipGetLastError();
}

// Whether the device gives one CTA the DMA-fed grouped kernel's LDS; queried once per process.
static bool grouped_dma_lds_ok() {
    static int ok = -1;
    if (ok < 0) {
        hipFuncAttributes fa;
        int dev = 0, mx = 0;
        ok = hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
             hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(&w12_grouped_dma_kernel<KT_EPI_SWIGLU>)) ==
                 hipSuccess &&
             fa.sharedSizeBytes + (size_t)KT_DMA_NS * dma_stage_x<KT_DMA_XR>() <= (size_t)mx;
    }
    return ok == 1;
}

hipError_t launch_w12_grouped(const int8_t* x, size_t x_bytes, const int32_t* list, int list_stride,
                              const int32_t* count, int groups, int64_t max_rows, const int8_t* wlo,
                              const uint8_t* wnib, size_t glo, int N, int kp, const int32_t* mant,
                              const int32_t* shift, int epi, const int16_t* silu, int h_shift, int8_t* y,
                              int ystride, int32_t* off_out, hipStream_t s) {
    if (groups <= 0 || N <= 0) return hipSuccess;
    if (groups > KT_MAX_GROUPS || kp <= 0 || kp % 64 || kp > KT_SMALL_KP || x_bytes + kp >= 0xFFFFFFF0ull ||
        max_rows < 0 || max_rows > INT32_MAX || (count == nullptr && groups != 1))
        return hipErrorInvalidValue;
    if (epi == KT_EPI_SWIGLU && (N % 64 || !silu || h_shift < 1 || h_shift > 30 || ystride % 16))
        return hipErrorInvalidValue;
    const int64_t tiles_n = (N + GTile::BN - 1) / GTile::BN;
    const int64_t ub = ((max_rows + GTile::BM - 1) / GTile::BM + groups) * tiles_n;  // row tiles <= rows/BM + groups
    if (ub * GTile::BN > INT32_MAX) return hipErrorInvalidValue;
    const int64_t grid = ub < 512 ? (ub + 7) / 8 * 8 : 512;  // two CTAs per CU, a multiple of 8 (XCDs)
    if (epi != KT_EPI_I8 && epi != KT_EPI_SWIGLU) return hipErrorInvalidValue;
    // enough 256-row tiles (at full groups) to give every CU one: the DMA-fed kernel, one CTA per CU
    if (max_rows / 256 * tiles_n >= 256 && grouped_dma_lds_ok()) {
        const size_t lds = (size_t)KT_DMA_NS * dma_stage_x<KT_DMA_XR>();  // the 288-row tile's stages
        const int64_t ub2 = ((max_rows + 255) / 256 + groups) * tiles_n;
        const unsigned grid2 = (unsigned)(ub2 < 256 ? (ub2 + 7) / 8 * 8 : 256);
        if (epi == KT_EPI_I8)
            w12_grouped_dma_kernel<KT_EPI_I8><<<dim3(grid2), dim3(512), lds, s>>>(
                x, (uint32_t)x_bytes, list, list_stride, count, groups, wlo, wnib, glo, N, kp, mant, shift, silu,
                h_shift, y, ystride, off_out, (int)max_rows);
        else
            w12_grouped_dma_kernel<KT_EPI_SWIGLU><<<dim3(grid2), dim3(512), lds, s>>>(
                x, (uint32_t)x_bytes, list, list_stride, count, groups, wlo, wnib, glo, N, kp, mant, shift, silu,
                h_shift, y, ystride, off_out, (int)max_rows);
        return hipGetLastError();
    }
#define KT_GROUPED(E, T, off)                                                                                        \
    w12_grouped_kernel<E, T><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, (uint32_t)x_bytes, list, list_stride,   \
                                                                       count, groups, wlo, wnib, glo, N, kp, mant, \
                                                                       shift, silu, h_shift, y, ystride, off,      \
                                                                       (int)max_rows)
    const int64_t tiles_h = (max_rows + GTileH::BM - 1) / GTileH::BM * tiles_n;
    if (groups == 1 && (max_rows + GTile::BM - 1) / GTile::BM * tiles_n < 512) {
        // a short dense batch, fewer 128-row tiles than CTA slots (two per CU): 64-row tiles, twice the tiles
        const unsigned grid_h = (unsigned)(tiles_h < 512 ? (tiles_h + 7) / 8 * 8 : 512);
        if (epi == KT_EPI_I8)
            w12_grouped_kernel<KT_EPI_I8, GT_HALF><<<dim3(grid_h), dim3(256), 0, s>>>(
                x, (uint32_t)x_bytes, list, list_stride, count, groups, wlo, wnib, glo, N, kp, mant, shift, silu,
                h_shift, y, ystride, off_out, (int)max_rows);
        else
            w12_grouped_kernel<KT_EPI_SWIGLU, GT_HALF><<<dim3(grid_h), dim3(256), 0, s>>>(
                x, (uint32_t)x_bytes, list, list_stride, count, groups, wlo, wnib, glo, N, kp, mant, shift, silu,
                h_shift, y, ystride, off_out, (int)max_rows);
        return hipGetLastError();
    }
    if (groups == 1) {
        if (epi == KT_EPI_I8) KT_GROUPED(KT_EPI_I8, GT_ALL, off_out);
        else KT_GROUPED(KT_EPI_SWIGLU, GT_ALL, off_out);
    } else {
        if (epi == KT_EPI_I8) KT_GROUPED(KT_EPI_I8, GT_MIXED, off_out);
        else KT_GROUPED(KT_EPI_SWIGLU, GT_MIXED, off_out);
    }
#undef KT_GROUPED
    return hipGetLastError();
}

hipError_t launch_moe_combine(const int8_t* d, const int32_t* off, const int32_t* sel, const int32_t* cw,
                              const int32_t* pos, int T, int H, int E, int top_k, int out_shift, int8_t* out,
                              hipStream_t s) {
    if (T <= 0) return hipSuccess;
    if (H % 16 || top_k < 1 || top_k > 32 || out_shift < 1 || out_shift > 30) return hipErrorInvalidValue;
    moe_combine_kernel<<<dim3((unsigned)T), dim3(256), 0, s>>>(d, off, sel, cw, pos, H, E, top_k, out_shift, out);
    return hipGetLastError();
}

}  // namespace kt
