// Exact integer GEMM kernels for CDNA4 (gfx950): the MI355X backend of tritify's linear accumulate
// Y[r,o] = sum_k X[r,k] * W[o,k] (crates/01-engine/kt-core/src/backend.rs:46-58).
//
// Everything here is integer arithmetic. Two operand families:
//
// 1. Digit planes (the LinearBackend path, any i32 codes): a code is P balanced base-256 digits d_i in [-128,127],
//    v = sum_i 256^i d_i (P = 1, 3 or 5 per operand). The product of two codes is sum_{i,j} 256^(i+j) x_i w_j, so
//    each plane pair is one int8 x int8 -> int32 MFMA product; pairs with equal i+j share one int32 accumulator
//    ("group" g = i+j). Groups are recombined in wrapping i64 as sum_g 256^g C_g -- exact modulo 2^64, which is the
//    reference's own release-mode i64 sum. The host splits k into chunks short enough that no int32 group sum can
//    wrap and launches one kernel per chunk, each adding its i64 result into y.
//    Layout of a planed operand: [plane][row][kp] int8, kp = k rounded up to 64, zero padded.
//
// 2. W12 (benchmark configs: int8 activations x 12-bit weight codes in [-2048, 2047]), the format and the mainloop
//    of kt_w12_core.h: the dense GEMM for large M and the skinny GEMM for batch decode live here, the grouped (MoE)
//    and im2col GEMMs in their own files.
//
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kt_kernels.h"
#include "kt_w12_core.h"

namespace kt {

// ------------------------------------------------------------------------------------------------------------------
// Packing kernels
// ------------------------------------------------------------------------------------------------------------------

// i32 codes [rows][k] -> P balanced base-256 digit planes [P][rows][kp]; padding k..kp is zero. `wrong_carry`
// truncates the carry (a planted defect for the firing controls only).
__global__ void pack_planes_kernel(const int32_t* __restrict__ codes, int64_t rows, int64_t k, int64_t kp, int p,
                                   int wrong_carry, int8_t* __restrict__ out) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * kp) return;
    int64_t r = idx / kp, c = idx - r * kp;
    int64_t v = c < k ? codes[r * k + c] : 0;
    for (int i = 0; i < p; i++) {
        int64_t d = ((v + 128) & 255) - 128;
        out[((int64_t)i * rows + r) * kp + c] = (int8_t)d;
        v = wrong_carry ? v / 256 : (v - d) >> 8;
    }
}

// i32 codes [n][k] in [-2048, 2047] -> fragment-tiled W12 planes (lo np*kp bytes, nib np*kp/2 bytes, np = n rounded
// up to 32). One thread per fragment lane: 16 lo bytes and 8 nib bytes; padding rows and k get lo = 0, hi = 0.
// ilv > 0 interleaves two halves of ilv rows each (a SwiGLU gate/up matrix, n = 2 ilv, ilv a multiple of 32):
// packed row block 2j holds source rows 32j.. (gate), block 2j+1 source rows ilv + 32j.. (up).
__global__ void w12_pack_kernel(const int32_t* __restrict__ codes, int64_t n, int64_t k, int64_t kp, int64_t ilv,
                                int8_t* __restrict__ lo, uint8_t* __restrict__ nib) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // fragment-lane index
    const int64_t KB = kp / 32, total = (n + 31) / 32 * KB * 64;
    if (idx >= total) return;
    const int64_t frag = idx >> 6, l = idx & 63, nb = frag / KB, kb = frag - nb * KB;
    const int64_t r = nb * 32 + (l & 31), c0 = kb * 32 + 16 * (l >> 5);
    const int64_t src = ilv > 0 ? (nb & 1) * ilv + (nb >> 1) * 32 + (l & 31) : r;
    uint32_t lw[4] = {0, 0, 0, 0}, nw[2] = {0, 0};
    for (int t = 0; t < 16; t++) {
        const int64_t c = c0 + t;
        uint32_t lb = 0, hb = 0;
        if (r < n && c < k) {
            const int32_t v = codes[src * k + c];
            lb = (uint32_t)((v & 255) - 128) & 255;
            hb = ((uint32_t)(v + 2048) >> 8) & 15;
        }
        lw[t >> 2] |= lb << (8 * (t & 3));
        nw[t >> 3] |= hb << (8 * (t & 3) + 4 * ((t >> 2) & 1));
    }
    *reinterpret_cast<v4i*>(lo + idx * 16) = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
    *reinterpret_cast<v2i*>(nib + idx * 8) = v2i{(int)nw[0], (int)nw[1]};
}

// i32 codes [n][k] in [-2048, 2047] -> the balanced W12B planes: hi = (v + 128) >> 8 in [-8, 8], lo = v - 256 hi in
// [-128, 127] (v = lo + 256 hi exactly), each plane fragment-tiled as W12's lo plane (np * kp bytes). One thread per
// fragment lane: 16 lo bytes and 16 hi bytes; padding rows and k are 0 in both.
__global__ void w12b_pack_kernel(const int32_t* __restrict__ codes, int64_t n, int64_t k, int64_t kp,
                                 int8_t* __restrict__ lo, int8_t* __restrict__ hi) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // fragment-lane index
    const int64_t KB = kp / 32, total = (n + 31) / 32 * KB * 64;
    if (idx >= total) return;
    const int64_t frag = idx >> 6, l = idx & 63, nb = frag / KB, kb = frag - nb * KB;
    const int64_t r = nb * 32 + (l & 31), c0 = kb * 32 + 16 * (l >> 5);
    uint32_t lw[4] = {0, 0, 0, 0}, hw[4] = {0, 0, 0, 0};
    for (int t = 0; t < 16; t++) {
        const int64_t c = c0 + t;
        uint32_t lb = 0, hb = 0;
        if (r < n && c < k) {
            const int32_t v = codes[r * k + c], h = (v + 128) >> 8;
            lb = (uint32_t)(v - 256 * h) & 255;
            hb = (uint32_t)h & 255;
        }
        lw[t >> 2] |= lb << (8 * (t & 3));
        hw[t >> 2] |= hb << (8 * (t & 3));
    }
    *reinterpret_cast<v4i*>(lo + idx * 16) = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
    *reinterpret_cast<v4i*>(hi + idx * 16) = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
}

// ------------------------------------------------------------------------------------------------------------------
// Digit-plane GEMM (LinearBackend path). CTA = 4 waves in 2x2; each wave WTM x WTN tiles of 32x32; BK = 64.
// Processes k in [k0, k1) (multiples of 64) and writes y = result (first chunk) or y += result.
// ------------------------------------------------------------------------------------------------------------------
// With ql non-null (the last k-chunk of a device QuantLinear call) the epilogue also adds the bias in units of c,
// (bs * c^-1).apply(bias[n]) when ql->mode == 0, and raises the call's output maximum (ql_raise_ymax) to the
// largest |result| (layers.rs:314-321).
// Split k (gridDim.y = S > 1, a QuantLinear call whose tiles leave CUs idle): CTA (t, s) takes the s-th of S
// contiguous runs of k-tiles and adds its partial result into y with 64-bit atomics (y starts at zero; wrapping
// addition is exact in any order); the last of the S CTAs of tile t to arrive (tile_cnt[t], zero at the start)
// reads the finished sums and does the bias and maximum part of the epilogue.
// Two waves per SIMD (two CTAs per CU) wherever the accumulators and operands fit 256 VGPRs; the 5 x 5 planes and
// the 1 x 5 planes on 1 x 2 wave tiles need more and run one wave per SIMD.
template <int PX, int PW, int WTM, int WTN>
constexpr int plane_gemm_waves() { return (PX == 5 && PW == 5) || (PX == 1 && PW == 5 && WTN == 2) ? 1 : 2; }

template <int PX, int PW, int WTM, int WTN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(plane_gemm_waves<PX, PW, WTM, WTN>(), 2))) void plane_gemm_kernel(const int8_t* __restrict__ xa, const int8_t* __restrict__ wb,
                                                         int64_t* __restrict__ y, int M, int N, int kp, int k0,
                                                         int k1, int accumulate, int drop_top,
                                                         const int64_t* __restrict__ ql_bias, QlState* ql_all,
                                                         unsigned* __restrict__ tile_cnt, QlSeg seg) {
    constexpr int BK = 64, CPR = BK / 16;
    constexpr int BM = 64 * WTM, BN = 64 * WTN;
    constexpr int NG = PX + PW - 1;
    constexpr int AL = BM * CPR / 256, BL = BN * CPR / 256;  // 16-byte chunks per thread per plane
    static_assert(AL >= 1 && BL >= 1, "tile too small for 256 threads");
    __shared__ __attribute__((aligned(16))) int8_t sA[2][PX][BM * BK];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][PW][BN * BK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_n = (N + BN - 1) / BN, tiles_m = (int)gridDim.x / tiles_n;  // gridDim.x = tiles_m * tiles_n
    // Block b runs on XCD b % 8. XCD x takes a contiguous run of the tile numbers (a bijection for any tile count),
    // numbered row tile fastest, so the row tiles of one column tile read its weight planes through one L2.
    const int nt = (int)gridDim.x, q8 = nt >> 3, r8 = nt & 7, xcd = (int)blockIdx.x & 7;
    const int t = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + ((int)blockIdx.x >> 3);
    const int m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
    QlState* ql = ql_all ? ql_all + ql_seg_of(seg, n0) : nullptr;  // this tile's call
    const size_t xplane = (size_t)M * kp, wplane = (size_t)N * kp;

    v16i acc[NG][WTM][WTN];
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
        for (int i = 0; i < WTM; i++)
#pragma unroll
            for (int j = 0; j < WTN; j++) acc[g][i][j] = v16i{};

    v4i ra[PX][AL], rb[PW][BL];
    auto gload_tile = [&](int k) {
#pragma unroll
        for (int p = 0; p < PX; p++)
#pragma unroll
            for (int i = 0; i < AL; i++) {
                int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
                int gr = m0 + r;
                ra[p][i] = gr < M ? gload16(xa + p * xplane + (size_t)gr * kp + k + 16 * c) : v4i{};
            }
#pragma unroll
        for (int q = 0; q < PW; q++)
#pragma unroll
            for (int i = 0; i < BL; i++) {
                int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
                int gr = n0 + r;
                rb[q][i] = gr < N ? gload16(wb + q * wplane + (size_t)gr * kp + k + 16 * c) : v4i{};
            }
    };
    auto lstore_tile = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PX; p++)
#pragma unroll
            for (int i = 0; i < AL; i++) {
                int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
                lds_write16(sA[buf][p], lds_off<CPR>(r, c), ra[p][i]);
            }
#pragma unroll
        for (int q = 0; q < PW; q++)
#pragma unroll
            for (int i = 0; i < BL; i++) {
                int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
                lds_write16(sB[buf][q], lds_off<CPR>(r, c), rb[q][i]);
            }
    };

    // this CTA's run of k-tiles: [kb, kb + nk * BK), nk >= 1 by the launcher's choice of S
    const int nk_all = (k1 - k0) / BK, per = (nk_all + (int)gridDim.y - 1) / (int)gridDim.y;
    const int kb = k0 + (int)blockIdx.y * per * BK;
    const int nk = nk_all - (int)blockIdx.y * per < per ? nk_all - (int)blockIdx.y * per : per;
    gload_tile(kb);
    lstore_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload_tile(kb + (kt + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            const int chunk = 2 * ks + (lane >> 5);
            v4i a[PX][WTM], b[PW][WTN];
#pragma unroll
            for (int p = 0; p < PX; p++)
#pragma unroll
                for (int i = 0; i < WTM; i++) {
                    int r = wm * 32 * WTM + i * 32 + (lane & 31);
                    a[p][i] = lds_read16(sA[cur][p], lds_off<CPR>(r, chunk));
                }
#pragma unroll
            for (int q = 0; q < PW; q++)
#pragma unroll
                for (int j = 0; j < WTN; j++) {
                    int r = wn * 32 * WTN + j * 32 + (lane & 31);
                    b[q][j] = lds_read16(sB[cur][q], lds_off<CPR>(r, chunk));
                }
#pragma unroll
            for (int p = 0; p < PX; p++)
#pragma unroll
                for (int q = 0; q < PW; q++)
#pragma unroll
                    for (int i = 0; i < WTM; i++)
#pragma unroll
                        for (int j = 0; j < WTN; j++) acc[p + q][i][j] = mfma32(a[p][i], b[q][j], acc[p + q][i][j]);
        }
        if (kt + 1 < nk) lstore_tile(cur ^ 1);
        __syncthreads();
    }

    int64_t lmax = 0;
    const bool badd = ql && ql_bias && ql->mode == 0, split = gridDim.y > 1;
    if (split) {  // partial sums into y, then the tile's last CTA goes on with the finished sums
#pragma unroll
        for (int i = 0; i < WTM; i++)
#pragma unroll
            for (int j = 0; j < WTN; j++) {
                const int n = n0 + wn * 32 * WTN + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + wm * 32 * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    uint64_t v = 0;
#pragma unroll
                    for (int g = 0; g < NG; g++) {
                        if (8 * g >= 64) continue;  // 256^g = 0 mod 2^64
                        if (drop_top && g == NG - 1) continue;
                        v += (uint64_t)(int64_t)acc[g][i][j][r] << (8 * g);
                    }
                    if (m < M && n < N)
                        atomicAdd(reinterpret_cast<unsigned long long*>(y + (size_t)m * N + n), (unsigned long long)v);
                }
            }
        // The hand-off in the memory model. The partial sums are agent-scope atomic read-modify-writes; each wave
        // releases them at workgroup scope (its own atomics performed) before the barrier, which orders them before
        // thread 0's arrival on the tile's counter, an agent-scope acquire-release. The CTA that completes the
        // count has acquired every other CTA's sums there; the barrier after it carries that to all its waves,
        // which read the sums with agent-scope atomic loads.
        __shared__ int s_last;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(&tile_cnt[blockIdx.x], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                     gridDim.y - 1;
        __syncthreads();
        if (!s_last) return;  // uniform
    }
#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++) {
            const int n = n0 + wn * 32 * WTN + j * 32 + (lane & 31);
            const uint64_t bc = badd && n < N ? (uint64_t)scale_apply(ql->f_mant, ql->f_shift, ql_bias[n]) : 0;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 32 * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M && n < N) {
                    int64_t* p = y + (size_t)m * N + n;
                    uint64_t f;
                    if (split) {  // the finished sum, read at the scope the other CTAs' atomics were performed
                        f = __hip_atomic_load(reinterpret_cast<uint64_t*>(p), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        uint64_t v = 0;
#pragma unroll
                        for (int g = 0; g < NG; g++) {
                            if (8 * g >= 64) continue;  // 256^g = 0 mod 2^64
                            if (drop_top && g == NG - 1) continue;
                            v += (uint64_t)(int64_t)acc[g][i][j][r] << (8 * g);
                        }
                        f = accumulate ? (uint64_t)*p + v : v;
                    }
                    if (ql) {
                        f += bc;
                        const int64_t a = (int64_t)f < 0 ? (int64_t)(0 - f) : (int64_t)f;  // i64::abs, wrapping
                        lmax = a > lmax ? a : lmax;
                    }
                    if (!split || bc != 0) *p = (int64_t)f;
                }
            }
        }
    if (ql) {  // the CTA's largest |result| into the call's maximum
        __shared__ int64_t s_max[4];
        lmax = wave_max_i64(lmax);
        if (lane == 0) s_max[wave] = lmax;
        __syncthreads();
        if (tid == 0) {
            int64_t b = s_max[0];
            for (int q = 1; q < 4; q++) b = s_max[q] > b ? s_max[q] : b;
            if (b > 0) ql_raise_ymax(ql, b);
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// The digit-plane product for a few rows (M <= MM <= KT_PLANE_SKINNY_M: decode rows, where a 64-row MFMA tile would
// do 64 rows of work for one): a wave per PS_CPW output columns, its lanes striding k[k0, k1) in 16-byte chunks of
// every plane row (coalesced 1 KB per load instruction), int32 plane-group sums per lane with sdot4 (the host's
// flush bound keeps every partial of a group within int32, as for the MFMA accumulators), a butterfly across the
// wave, then plane_gemm_kernel's epilogue: groups recombined modulo 2^64, drop_top, accumulate, the QuantLinear
// bias and maximum. No k split.
// ------------------------------------------------------------------------------------------------------------------
#define KT_PLANE_SKINNY_M 4
constexpr int PS_CPW = 2;  // output columns per wave

template <int PX, int PW, int MM>
__global__ __launch_bounds__(256) void plane_skinny_kernel(const int8_t* __restrict__ xa, const int8_t* __restrict__ wb,
                                                           int64_t* __restrict__ y, int M, int N, int kp, int k0,
                                                           int k1, int accumulate, int drop_top,
                                                           const int64_t* __restrict__ ql_bias, QlState* ql_all,
                                                           QlSeg seg) {
    constexpr int NG = PX + PW - 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = ((int)blockIdx.x * 4 + wave) * PS_CPW;  // the wave's first column
    QlState* ql = ql_all ? ql_all + ql_seg_of(seg, (int)blockIdx.x * 4 * PS_CPW) : nullptr;  // this CTA's call
    const size_t xplane = (size_t)M * kp, wplane = (size_t)N * kp;
    const int nch = (k1 - k0) / 16;
    int acc[PS_CPW][MM][NG];
#pragma unroll
    for (int c = 0; c < PS_CPW; c++)
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int g = 0; g < NG; g++) acc[c][m][g] = 0;
    for (int q = lane; q < nch; q += 64) {
        const size_t ko = (size_t)k0 + 16 * (size_t)q;
        v4i xv[PX][MM], wv[PS_CPW][PW];
#pragma unroll
        for (int i = 0; i < PX; i++)
#pragma unroll
            for (int m = 0; m < MM; m++)
                xv[i][m] = m < M ? *reinterpret_cast<const v4i*>(xa + i * xplane + (size_t)m * kp + ko) : v4i{};
#pragma unroll
        for (int c = 0; c < PS_CPW; c++)
#pragma unroll
            for (int j = 0; j < PW; j++)
                wv[c][j] = nb + c < N ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(
                                            wb + j * wplane + (size_t)(nb + c) * kp + ko))  // read once: non-temporal
                                      : v4i{};
#pragma unroll
        for (int c = 0; c < PS_CPW; c++)
#pragma unroll
            for (int m = 0; m < MM; m++)
#pragma unroll
                for (int i = 0; i < PX; i++)
#pragma unroll
                    for (int j = 0; j < PW; j++) {
                        int d = acc[c][m][i + j];
#pragma unroll
                        for (int e = 0; e < 4; e++) d = __builtin_amdgcn_sdot4(xv[i][m][e], wv[c][j][e], d, false);
                        acc[c][m][i + j] = d;
                    }
    }
#pragma unroll
    for (int c = 0; c < PS_CPW; c++)
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int g = 0; g < NG; g++)
                acc[c][m][g] = wave_sum_i32(acc[c][m][g]);
    const bool badd = ql && ql_bias && ql->mode == 0;
    int64_t lmax = 0;
    if (lane == 0) {
#pragma unroll
        for (int c = 0; c < PS_CPW; c++) {
            const int n = nb + c;
            if (n >= N) continue;
            const uint64_t bc = badd ? (uint64_t)scale_apply(ql->f_mant, ql->f_shift, ql_bias[n]) : 0;
#pragma unroll
            for (int m = 0; m < MM; m++) {
                if (m >= M) continue;
                uint64_t v = 0;
#pragma unroll
                for (int g = 0; g < NG; g++) {
                    if (8 * g >= 64) continue;  // 256^g = 0 mod 2^64
                    if (drop_top && g == NG - 1) continue;
                    v += (uint64_t)(int64_t)acc[c][m][g] << (8 * g);
                }
                int64_t* p = y + (size_t)m * N + n;
                uint64_t f = accumulate ? (uint64_t)*p + v : v;
                if (ql) {
                    f += bc;
                    const int64_t a = (int64_t)f < 0 ? (int64_t)(0 - f) : (int64_t)f;  // i64::abs, wrapping
                    lmax = a > lmax ? a : lmax;
                }
                *p = (int64_t)f;
            }
        }
    }
    if (ql) {  // the CTA's largest |result| into the call's maximum
        __shared__ int64_t s_max[4];
        if (lane == 0) s_max[wave] = lmax;
        __syncthreads();
        if (tid == 0) {
            int64_t b = s_max[0];
            for (int w2 = 1; w2 < 4; w2++) b = s_max[w2] > b ? s_max[w2] : b;
            if (b > 0) ql_raise_ymax(ql, b);
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// W12 GEMM (M > 128). x int8 [M][kp] (zero padded); W12 fragment-tiled lo / nib; the mainloop of kt_w12_core.h.
// Tiles are numbered so that the CTAs the hardware places on one XCD (block b -> XCD b % 8) form a compact group
// of GM tile-rows, sharing A rows and B columns in that XCD's L2.
// ------------------------------------------------------------------------------------------------------------------

// One W12 output from its two plane sums and the row-sum term: v = s_lo + 256 s_hi + corr (corr = -1920 sum x).
// SMALL: every partial sum and v fit int32 (kp <= 8128: |v| <= 8128 * 2048 * 128 < 2^31), so v is formed in 32 bits
// and the requant product |v| * mant (< 2^62) in 64 -- a handful of instructions per output.
template <int OUT, bool SMALL>
__device__ __forceinline__ void store_w12(void* y, size_t idx, int s_lo, int s_hi, int64_t corr, int32_t mant,
                                          int32_t sh) {
    if constexpr (SMALL) {
        const int v = w12_value(s_lo, s_hi, (int)corr);
        if constexpr (OUT == KT_OUT_I64) {
            reinterpret_cast<int64_t*>(y)[idx] = (int64_t)v;
        } else {
            const uint32_t a = v < 0 ? 0u - (uint32_t)v : (uint32_t)v;
            const uint64_t prod = (uint64_t)a * (uint32_t)mant;
            int64_t q;
            if (sh <= 0) q = (int64_t)(prod << (-sh));
            else q = (int64_t)((prod + ((uint64_t)1 << (sh - 1))) >> sh);  // sh <= 63: prod < 2^62
            if (v < 0) q = -q;
            if constexpr (OUT == KT_OUT_I32 || OUT == KT_OUT_I32_ADD) {
                q = q > INT32_MAX ? INT32_MAX : (q < INT32_MIN ? INT32_MIN : q);
                if constexpr (OUT == KT_OUT_I32_ADD) q = sat_add32(reinterpret_cast<int32_t*>(y)[idx], q);
                reinterpret_cast<int32_t*>(y)[idx] = (int32_t)q;
            } else {
                q = q > 127 ? 127 : (q < -127 ? -127 : q);
                reinterpret_cast<int8_t*>(y)[idx] = (int8_t)q;
            }
        }
    } else {
        const int64_t v = (int64_t)s_lo + 256 * (int64_t)s_hi + corr;
        store_out<OUT>(y, idx, v, &mant, &sh, 0);
    }
}

__device__ __forceinline__ void tile_coords(int M, int N, int BM, int BN, int& m0, int& n0) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, nt = tiles_m * tiles_n;
    int bid = blockIdx.x;
    if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);  // consecutive ids on one XCD
    constexpr int GM = 4;
    const int group = bid / (GM * tiles_n), first_m = group * GM;
    const int gsize = tiles_m - first_m < GM ? tiles_m - first_m : GM;
    const int in_group = bid - group * GM * tiles_n;
    m0 = (first_m + in_group % gsize) * BM;
    n0 = (in_group / gsize) * BN;
}

// Tile shape of the large-M W12 GEMM: waves per SIMD the register allocation targets, 32x32 tiles per wave.
#ifndef KT_W12_WTM
#define KT_W12_WTM 4
#endif
#ifndef KT_W12_WTN
#define KT_W12_WTN 1
#endif
#ifndef KT_W12_WAVES
#define KT_W12_WAVES 2
#endif
#ifndef KT_W12_WM
#define KT_W12_WM 1
#endif
#ifndef KT_W12_NSLOT
#define KT_W12_NSLOT 4
#endif

// The dense W12 GEMM's epilogue: recombine the two planes with the row-sum term (sRow), requantize per output channel
// and store the CTA tile at (m0, n0). OUT_I8 stages the int8 tile in `smem` (BM x BN bytes, free once the mainloop
// is done) and applies `sLut` when `lut` is non-null.
template <class C, int OUT, bool SMALL>
__device__ __forceinline__ void w12_gemm_epilogue(const v16i (&acc0)[C::WTM][C::WTN],
                                                  const v16i (&acc1)[C::WTM][C::WTN], const int* sRow, int8_t* smem,
                                                  const int8_t* sLut, void* __restrict__ y, int M, int N, int m0,
                                                  int n0, const int32_t* __restrict__ mant,
                                                  const int32_t* __restrict__ shift, const int8_t* __restrict__ lut) {
    constexpr int NT = C::NT, BM = C::BM, BN = C::BN, WTM = C::WTM, WTN = C::WTN, WN = C::WN;
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
    const int wave = (tid >> 6) % WN, rw0 = ((tid >> 6) / WN) * 32 * WTM;
    const bool full = m0 + BM <= M && n0 + BN <= N;
    if constexpr (OUT == KT_OUT_I8 && SMALL) {
        // requantize (and map through the code table) into an int8 tile in LDS (the A ring is no longer read),
        // then store it with 16-byte writes
        if (lut) w12_requant_tile8<C, true>(acc0, acc1, sRow, mant, shift, n0, N, [](int n) { return n; }, smem, sLut);
        else w12_requant_tile8<C, false>(acc0, acc1, sRow, mant, shift, n0, N, [](int n) { return n; }, smem);
        __syncthreads();
        constexpr int CH = BM * BN / 16;  // 16-byte chunks of the tile
#pragma unroll
        for (int i = 0; i < (CH + NT - 1) / NT; i++) {
            const int idx = tid + NT * i;
            if (CH % NT != 0 && idx >= CH) break;
            const int rt = idx / (BN / 16), c = (idx % (BN / 16)) * 16, m = m0 + rt, n = n0 + c;
            const v4i v = *reinterpret_cast<const v4i*>(smem + rt * BN + c);
            // bytes are moved with shifts, never through the vector's address: an addressed vector becomes a
            // per-thread LDS slot whose indexing reads the dispatch packet, a long stall before the stores
            int8_t* dst = reinterpret_cast<int8_t*>(y) + (size_t)m * N + n;
            if (full && (N & 15) == 0) {
                *reinterpret_cast<v4i*>(dst) = v;
            } else if (m < M) {
#pragma unroll
                for (int t = 0; t < 16; t++)
                    if (n + t < N) dst[t] = (int8_t)((uint32_t)v[t >> 2] >> (8 * (t & 3)));
            }
        }
    } else if constexpr ((OUT == KT_OUT_I32 || OUT == KT_OUT_I32_ADD) && SMALL) {
#pragma unroll
        for (int j = 0; j < WTN; j++) {
            const int n = n0 + wave * 32 * WTN + j * 32 + (lane & 31);
            const ColQ q = col_q(n < N ? mant[n] : 0, n < N ? shift[n] : 1);
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int rt = rw0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3), m = m0 + rt;
                    const int v = w12_value(acc0[i][j][r], acc1[i][j][r], w12_corr(sRow[rt]));
                    const int32_t o = col_requant<true>(v, q);
                    if (full || (m < M && n < N)) {
                        int32_t* p = reinterpret_cast<int32_t*>(y) + (size_t)m * N + n;
                        *p = OUT == KT_OUT_I32_ADD ? sat_add32(*p, o) : o;
                    }
                }
        }
    } else {
        int32_t cm[WTN], cs[WTN];
#pragma unroll
        for (int j = 0; j < WTN; j++) {
            const int n = n0 + wave * 32 * WTN + j * 32 + (lane & 31);
            cm[j] = (OUT != KT_OUT_I64 && n < N) ? mant[n] : 0;
            cs[j] = (OUT != KT_OUT_I64 && n < N) ? shift[n] : 0;
        }
#pragma unroll
        for (int i = 0; i < WTM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int rt = rw0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);  // row within the CTA tile
                const int64_t corr = -1920 * (int64_t)sRow[rt];  // past int32 for k > 8738
                const int m = m0 + rt;
#pragma unroll
                for (int j = 0; j < WTN; j++) {
                    const int n = n0 + wave * 32 * WTN + j * 32 + (lane & 31);
                    if (full || (m < M && n < N))
                        store_w12<OUT, SMALL>(y, (size_t)m * N + n, acc0[i][j][r], acc1[i][j][r], corr, cm[j], cs[j]);
                }
            }
    }
}

// An optional int8 -> int8 table (`lut`, 255 entries indexed by q + 127) is applied after the int8 requant: the
// activation-code epilogue (GELU of config 5). lut is read only for OUT == KT_OUT_I8 and may be null.
template <int WM, int WTM, int WTN, int WAVES, int NSLOT, int OUT, bool SMALL, int WN = 4>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WAVES, WAVES))) void w12_gemm_kernel(
    const int8_t* __restrict__ x, const int8_t* __restrict__ wlo, const uint8_t* __restrict__ wnib,
    void* __restrict__ y, int M, int N, int kp, const int32_t* __restrict__ mant, const int32_t* __restrict__ shift,
    const int8_t* __restrict__ lut) {
    typedef W12Tile<WM, WTM, WTN, NSLOT, WN> C;
    constexpr int NT = C::NT, BM = C::BM, BN = C::BN, AL = C::AL, AC = C::AC;
    constexpr int SO = OUT == KT_OUT_I8 ? BM * BN : 0;  // the int8 output tile reuses the A ring after the loop
    __shared__ __attribute__((aligned(16))) int8_t smem[C::RING > SO ? C::RING : SO];
    __shared__ int sRow[BM];
    __shared__ int8_t sLut[256];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = (tid >> 6) % WN;
    int m0, n0;
    tile_coords(M, N, BM, BN, m0, n0);
    const int KB = kp / 32;
    if (OUT == KT_OUT_I8 && SMALL)
        for (int i = tid; i < 256; i += NT) sLut[i] = lut ? lut[i < 255 ? i : 254] : 0;

    // A: the CTA's rows; rows past the matrix read as zero (their offsets are past the descriptor)
    const uint32_t rows_a = (uint32_t)(M - m0 < BM ? M - m0 : BM);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(x + (size_t)m0 * kp, rows_a * (uint32_t)kp);
    uint32_t oa[AL];
#pragma unroll
    for (int i = 0; i < AL; i++) {
        const int idx = tid + NT * i;
        oa[i] = idx < AC ? (uint32_t)(idx >> 2) * (uint32_t)kp + 16 * (idx & 3) : KT_OOB;
    }
    // B: the CTA's column blocks (fragment-tiled); blocks past the matrix read as zero
    const int cb0 = n0 / 32, ncb = (N - n0 + 31) / 32 < BN / 32 ? (N - n0 + 31) / 32 : BN / 32;
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(wnib + (size_t)cb0 * KB * 512, (uint32_t)ncb * KB * 512);
    uint32_t ob[WTN], on[WTN];
#pragma unroll
    for (int j = 0; j < WTN; j++) {
        ob[j] = (uint32_t)((wave * WTN + j) * KB) * 1024 + 16 * lane;
        on[j] = (uint32_t)((wave * WTN + j) * KB) * 512 + 8 * lane;
    }

    v16i acc0[WTM][WTN], acc1[WTM][WTN];
    int rsum[AL];
    w12_mainloop<C>(rA, oa, rL, rN, ob, on, kp / C::BK, smem, acc0, acc1, rsum);
    w12_row_sums<C>(rsum, sRow);

    w12_gemm_epilogue<C, OUT, SMALL>(acc0, acc1, sRow, smem, sLut, y, M, N, m0, n0, mant, shift, lut);
}

// Dense W12 GEMM on 256 x 128 CTA tiles fed by LDS DMA (w12_mainloop_dma): one CTA of 8 waves per CU, every operand
// byte moved once per CTA; the epilogue is the 128 x 128 kernel's. Dynamic LDS: KT_DMA_NS stages, which the int8
// output tile reuses.
#ifndef KT_W12_DMA
#define KT_W12_DMA 1
#endif
// BAL: the weights are the balanced W12B planes (wnib is the hi plane, int8, laid out as lo).
template <int OUT, bool SMALL, bool BAL = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void w12_gemm_dma_kernel(
    const int8_t* __restrict__ x, const int8_t* __restrict__ wlo, const uint8_t* __restrict__ wnib,
    void* __restrict__ y, int M, int N, int kp, const int32_t* __restrict__ mant, const int32_t* __restrict__ shift,
    const int8_t* __restrict__ lut) {
    typedef W12Tile<2, 4, 1, 2, 4> C;  // 256 x 128, 8 waves (the tile's NSLOT is not used by this mainloop)
    static_assert(C::BM == 256 && C::BN == 128 && C::NT == 512, "the DMA mainloop's tile");
    static_assert(KT_DMA_NS * KT_DMA_STAGE >= C::BM * C::BN, "the int8 output tile fits the ring");
    constexpr uint32_t HB = BAL ? 1024 : 512;  // bytes of the hi plane per k32 block of a column block
    extern __shared__ __attribute__((aligned(16))) int8_t ring[];
    __shared__ int sRow[C::BM];
    __shared__ int8_t sLut[256];
    const int tid = threadIdx.x;
    int m0, n0;
    tile_coords(M, N, C::BM, C::BN, m0, n0);
    const int KB = kp / 32;
    if (OUT == KT_OUT_I8 && SMALL)
        for (int i = tid; i < 256; i += C::NT) sLut[i] = lut ? lut[i < 255 ? i : 254] : 0;
    // rows and column blocks past the matrix read as zero (their offsets are past the descriptors)
    const uint32_t rows_a = (uint32_t)(M - m0 < C::BM ? M - m0 : C::BM);
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(x + (size_t)m0 * kp, rows_a * (uint32_t)kp);
    const int cb0 = n0 / 32, ncb = (N - n0 + 31) / 32 < 4 ? (N - n0 + 31) / 32 : 4;
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(wnib + (size_t)cb0 * KB * HB, (uint32_t)ncb * KB * HB);
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t va0 = (uint32_t)dma_a_row(w, lane, 0) * (uint32_t)kp + dma_a_chunk(lane);
    v16i acc0[4][1], acc1[4][1];
    w12_mainloop_dma<KT_DMA_NS, BAL>(rA, rL, rN, va0, va0 + 16u * (uint32_t)kp, kp, ring, acc0, acc1, sRow);
    w12_gemm_epilogue<C, OUT, SMALL>(acc0, acc1, sRow, ring, sLut, y, M, N, m0, n0, mant, shift, lut);
}

// Whether the device gives one CTA the DMA kernel's LDS (static arrays + the ring); queried once per process.
static bool dma_lds_ok() {
    static int ok = -1;
    if (ok < 0) {
        hipFuncAttributes fa;
        int dev = 0, mx = 0;
        ok = hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
             hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(&w12_gemm_dma_kernel<KT_OUT_I8, true>)) ==
                 hipSuccess &&
             fa.sharedSizeBytes + (size_t)KT_DMA_NS * KT_DMA_STAGE_BAL <= (size_t)mx;
    }
    return ok == 1;
}

// ------------------------------------------------------------------------------------------------------------------
// W12 skinny GEMM (M <= 16 * MT <= 128, batch decode and short prefill chunks). Bandwidth-bound: the weights are read once,
// so the grid must reach every CU with enough loads in flight and end without a cross-CTA reduction. A CTA owns half
// a column block (16 columns: fragment lanes 16 hb + c + 32 h, i.e. two 256-byte runs of each 1 KB lo fragment and
// two 128-byte runs of each 512-byte nib fragment; the two halves of a block read disjoint bytes) over all of k, so
// N = 4096 gives 256 CTAs. Its NW waves take pairs of k32 blocks round-robin, U pairs in flight per wave. On the
// 16x16x64 MFMA, lane l = c + 16 g supplies column c (B) / row c (A) for k-group g = (k32 block 2p + g / 2,
// k-half g % 2): exactly the lanes the half block's bytes arrive in, so no operand moves between lanes. Rows past
// M read as zero through the x buffer descriptor (kp is a multiple of 64, so a column block has an even number of
// k32 blocks and np whole pairs). The waves meet in LDS in i64; the per-channel scales are fetched
// at the start, so the epilogue waits on no memory.
//
// FOLD_O (one row, residual-add output): before this product's requantized dots are added, the residual takes the
// requantized o-projection sums the decode attention step left in fo.acc (y[n] = sat(sat(y[n] + requant_o(acc[n]))
// + requant(dot)), the two residual additions in the reference's order), and the thread that owns column n clears
// acc[n] for the next step.
// ------------------------------------------------------------------------------------------------------------------
struct FoldO {
    int32_t* acc;          // d int32: the o projection's dot sums (W12 offset included)
    const int32_t* mant;   // the o projection's per-channel scales
    const int32_t* shift;
};

template <int MT, int NW, int U, int OUT, bool SMALL, bool NORM = false, bool FOLD_O = false>
__global__ __launch_bounds__(64 * NW) void w12_skinny_kernel(const int8_t* __restrict__ x,
                                                             const int8_t* __restrict__ wlo,
                                                             const uint8_t* __restrict__ wnib, void* __restrict__ y,
                                                             int M, int N, int kp, const int32_t* __restrict__ mant,
                                                             const int32_t* __restrict__ shift,
                                                             const int8_t* __restrict__ lut, int d, FoldO fo = {}) {
    constexpr int NT = 64 * NW, OUTS = MT * 256;  // threads; outputs of the CTA (MT row tiles x 16 columns)
    static_assert(OUTS % NT == 0 || NT % OUTS == 0, "the threads tile the outputs");
    static_assert(!NORM || (MT == 1 && SMALL), "the RMSNorm prologue serves M <= 16 with int32 dots");
    static_assert(!FOLD_O || (MT == 1 && SMALL && !NORM && OUT == KT_OUT_I32_ADD), "FOLD_O: one-row residual add");
    typedef typename std::conditional<SMALL, int32_t, int64_t>::type part_t;  // SMALL: every dot fits int32
    __shared__ part_t sP[NW][OUTS];
    __shared__ int32_t sX[NW][MT * 16];
    extern __shared__ __attribute__((aligned(16))) int8_t sQ[];  // NORM: the normalized rows, M x kp
    __shared__ uint64_t sNss[NORM ? NW * 32 : 1], sNrq[NORM ? 32 : 1];
    int32_t pre[2];  // NORM: row 0 of the residual, loaded first
    if constexpr (NORM) norm_preload<64 * NW, 2>(reinterpret_cast<const int32_t*>(x), d, pre);
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar load offsets
    const int cb = blockIdx.x >> 1, hb = blockIdx.x & 1, n0 = cb * 32 + 16 * hb;
    const int KB = kp / 32;

    // the epilogue's channel scales, fetched now
    const int oc = tid & 15, on = n0 + oc;  // every output of this thread is in column on (NT is a multiple of 16)
    const int32_t om = (OUT != KT_OUT_I64 && tid < OUTS && on < N) ? mant[on] : 0;
    const int32_t os = (OUT != KT_OUT_I64 && tid < OUTS && on < N) ? shift[on] : 0;
    // the residual an I32_ADD output adds to, loaded now (one output per thread when OUTS <= NT): the epilogue then
    // has no dependent load; only this thread reads or writes that element
    constexpr bool PRE_Y = OUT == KT_OUT_I32_ADD && SMALL && OUTS <= NT;
    int32_t yres = 0;
    if constexpr (PRE_Y) {
        if (tid < OUTS && (tid >> 4) < M && on < N) yres = reinterpret_cast<const int32_t*>(y)[(size_t)(tid >> 4) * N + on];
    }
    int32_t fa = 0, fm = 0, fs = 0;  // FOLD_O: row 0's o sum and its scale, loaded now as well
    if constexpr (FOLD_O) {
        if (tid < 16 && on < N) fa = fo.acc[on], fm = fo.mant[on], fs = fo.shift[on];
    }

    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cb * KB * 1024, (uint32_t)KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(wnib + (size_t)cb * KB * 512, (uint32_t)KB * 512);
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(x, (uint32_t)M * (uint32_t)kp);
    const int c = lane & 15, g = lane >> 4, kbq = g >> 1, h = g & 1;
    const int slot = 16 * hb + c + 32 * h;
    const uint32_t oL = 16 * slot + 1024 * kbq, oN = 8 * slot + 512 * kbq;
    uint32_t oX[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) oX[t] = (uint32_t)(c + 16 * t) * (uint32_t)kp + 32 * kbq + 16 * h;

    v4i acc0[MT], acc1[MT];
    int sx[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc0[t] = acc1[t] = v4i{}, sx[t] = 0;

    v4i L[U], X[U][MT];
    v2i D[U];
    const int np = (KB + 1) / 2, nb = (np + NW * U - 1) / (NW * U);
    // batch b: U pairs of k32 blocks per wave, all loads in flight before the first MFMA. The RMSNorm variant runs
    // exactly one batch (the host guarantees it), as straight-line code: no loop header to wait at, so the residual
    // row's loads are the only ones its prologue waits for.
    auto batch = [&](const int b) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            // a pair past the end re-reads the last pair (its x is masked below): every load stays in the buffers
            const int p = w + NW * (U * b + u);
            const uint32_t pl = (uint32_t)(p < np ? p : np - 1);
            L[u] = bload16nt(rL, oL, pl * 2048u);  // the weights: read once per launch
            D[u] = bload8nt(rN, oN, pl * 1024u);
            if constexpr (!NORM) {
#pragma unroll
                for (int t = 0; t < MT; t++) X[u][t] = bload16(rX, oX[t], pl * 64u);
            }
        }
        if constexpr (NORM) {  // x rows from LDS, normalized there while the first weight loads are in flight
            __builtin_amdgcn_sched_barrier(0);
            norm_rows_to_lds<NT, 2>(reinterpret_cast<const int32_t*>(x), M, d, kp, sQ, sNss, sNrq, pre);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = w + NW * (U * b + u);
                const uint32_t pl = (uint32_t)(p < np ? p : np - 1);
                X[u][0] = c < M ? *reinterpret_cast<const v4i*>(sQ + (size_t)c * kp + pl * 64u + 32 * kbq + 16 * h)
                                : v4i{};
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int mask = 2 * (w + NW * (U * b + u)) + kbq < KB ? -1 : 0;  // x past k is not in the row sums
            const v4i hi = unpack_hi(D[u]);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i a = X[u][t] & mask;
                sx[t] += sum4(a);
                acc0[t] = mfma16(a, L[u], acc0[t]);
                acc1[t] = mfma16(a, hi, acc1[t]);
            }
        }
    };
    if constexpr (NORM) {
        batch(0);
    } else {
        int b = 0;
        do batch(b);
        while (++b < nb);
    }

    // the wave's partials (lane l, register r: row 4 g + r of the tile, column c) and row sums into LDS
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if constexpr (SMALL)  // modulo 2^32: the CTA's total is exact
                sP[w][(t * 16 + 4 * g + r) * 16 + c] = (int32_t)((uint32_t)acc0[t][r] + ((uint32_t)acc1[t][r] << 8));
            else
                sP[w][(t * 16 + 4 * g + r) * 16 + c] = (int64_t)acc0[t][r] + 256 * (int64_t)acc1[t][r];
        }
        const int s = add_xor32(add_xor16(sx[t]));
        if (lane < 16) sX[w][t * 16 + lane] = s;
    }
    __syncthreads();
    const ColQ cq = col_q(om, os);
#pragma unroll
    for (int o = tid; o < OUTS; o += NT) {
        const int m = o >> 4;  // output (m, oc)
        if constexpr (SMALL) {
            uint32_t v = 0, rs = 0;
#pragma unroll
            for (int q = 0; q < NW; q++) v += (uint32_t)sP[q][o], rs += (uint32_t)sX[q][m];
            const int vi = (int)(v - 1920u * rs);
            if (m < M && on < N) {
                const size_t idx = (size_t)m * N + on;
                if constexpr (OUT == KT_OUT_I64) reinterpret_cast<int64_t*>(y)[idx] = vi;
                else if constexpr (OUT == KT_OUT_I32) reinterpret_cast<int32_t*>(y)[idx] = col_requant<true>(vi, cq);
                else if constexpr (OUT == KT_OUT_I32_ADD) {
                    int32_t* p = reinterpret_cast<int32_t*>(y) + idx;
                    int32_t base = PRE_Y ? yres : *p;
                    if constexpr (FOLD_O) {  // M == 1: this is row 0, column on
                        base = sat_add32(base, col_requant<true>(fa, col_q(fm, fs)));
                        fo.acc[on] = 0;
                    }
                    *p = sat_add32(base, col_requant<true>(vi, cq));
                }
                else {
                    const int q = col_requant<false>(vi, cq);
                    reinterpret_cast<int8_t*>(y)[idx] = lut ? lut[q + 127] : (int8_t)q;
                }
            }
        } else {
            int64_t v = 0, rs = 0;
#pragma unroll
            for (int q = 0; q < NW; q++) v += sP[q][o], rs += sX[q][m];
            v -= 1920 * rs;
            if (m < M && on < N) store_out<OUT>(y, (size_t)m * N + on, v, &om, &os, 0);
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// W12 skinny GEMM for 64 < M <= 128 with x staged through LDS. Loaded straight into the MFMA operand lanes (the skinny
// kernel above), each x load instruction touches 16 rows x 64 bytes, half of every 128-byte line it requests, and
// every one of the N / 16 CTAs reads all of x: at N = K = 4096, 128 MB of x requests for 25 MB of weights, and the
// requests, not the bytes, set the time. Here a CTA owns 64 rows x one 32-column block (CTAs 8 apart, on one XCD,
// share the block's weights: rows 0-63 and 64-127), so x is read N / 32 times, and everything arrives by LDS DMA in
// stages of 256 k (SK_STAGE bytes: x, then the block's lo and nib planes for those k, which are contiguous in the
// packed layout). Each x DMA instruction moves 4 rows x 256 contiguous bytes (8 whole lines), lane L landing at row
// L / 16, 16-byte chunk position L % 16 of the stage, fetching chunk (L % 16) ^ (row % 16) (the swizzle that keeps the
// fragment reads conflict-free). Every wave issues the same SK_DMAS DMA instructions per stage and none writes a
// register, so one s_waitcnt vmcnt per stage, in the instruction stream, is the only wait: a ring of SK_NS stages
// keeps SK_NS - 1 in flight. Offsets past a buffer (rows past M, k past kp, stages past the end) read as zero, so
// nothing needs masking. Wave w takes pair w % 4 of a stage's four k64 pairs and column half w / 4, all 4 row tiles,
// and the row sums of tiles 2 (w / 4) and 2 (w / 4) + 1; the waves' partial sums then meet in the ring's LDS.
// ------------------------------------------------------------------------------------------------------------------
// 3 stages: 11.6-12.1 us at M = 128, N = K = 4096, against 12.2 for 4 and 12.6-12.9 for 5
constexpr int SK_NS = 3, SK_X = 64 * 256, SK_LO = 32 * 256, SK_NIB = 32 * 128;  // ring stages; bytes per stage
constexpr int SK_STAGE = SK_X + SK_LO + SK_NIB, SK_DMAS = 4;                     // 28 KB; DMAs per wave per stage

template <int OUT>
__global__ __launch_bounds__(512) void w12_skinny_lds_kernel(const int8_t* __restrict__ x,
                                                             const int8_t* __restrict__ wlo,
                                                             const uint8_t* __restrict__ wnib, void* __restrict__ y,
                                                             int M, int N, int kp, const int32_t* __restrict__ mant,
                                                             const int32_t* __restrict__ shift,
                                                             const int8_t* __restrict__ lut) {
    constexpr int NT = 512, OUTS = 64 * 32;  // 64 rows x 32 columns
    static_assert(SK_NS * SK_STAGE >= 8 * 64 * 16 * 4, "the waves' partials fit the ring");
    extern __shared__ __attribute__((aligned(16))) int8_t ring[];
    __shared__ int32_t sX[4][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x, rh = (b >> 3) & 1, cb = (b & 7) | ((b >> 4) << 3);
    const int m0 = 64 * rh, n0 = 32 * cb;
    if (n0 >= N) return;  // past the last column block: the whole CTA idles
    const int KB = kp / 32, nst = (kp + 255) / 256;  // k32 blocks, stages
    const int Mr = M - m0 < 64 ? M - m0 : 64;        // rows of this CTA (>= 1: M > 64)

    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cb * KB * 1024, (uint32_t)KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(wnib + (size_t)cb * KB * 512, (uint32_t)KB * 512);
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(x + (size_t)m0 * kp, (uint32_t)Mr * (uint32_t)kp);
    const int c = lane & 15, g = lane >> 4, kbq = g >> 1, h = g & 1;
    const int pp = w & 3, ch = w >> 2;  // the wave's pair within a stage; its column half
    const int slot = 16 * ch + c + 32 * h;

    // DMA lanes. x: instruction i (0, 1) of wave w moves rows 8 w + 4 i + lane / 16, chunk position lane % 16; lo: wave
    // w moves bytes 1024 w .. 1024 w + 1023 of the stage's 8 KB; nib: lanes 0-31 of wave w move bytes 512 w .. 512 w +
    // 511 of its 4 KB. Every offset is a VGPR (the SGPR offset stays 0, uniform), so the range check sees all of it.
    uint32_t vX[2];
    int qX[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = 8 * w + 4 * i + (lane >> 4);
        qX[i] = (lane & 15) ^ (r & 15);
        vX[i] = r < Mr ? (uint32_t)r * (uint32_t)kp + 16u * qX[i] : KT_OOB;  // rows past M read as zero
    }
    const uint32_t vL = 1024u * w + 16u * lane, vN = 512u * w + 16u * (lane & 31);
    auto issue = [&](auto S, int st) {
        constexpr int sl = decltype(S)::value;
        int8_t* sb = ring + sl * SK_STAGE;
        const uint32_t k0 = 256u * (uint32_t)st;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t v = vX[i] != KT_OOB && k0 + 16u * qX[i] < (uint32_t)kp ? vX[i] + k0 : KT_OOB;
            dma16(rX, sb + 2048 * w + 1024 * i, v, 0);
        }
        dma16(rL, sb + SK_X + 1024 * w, vL + (uint32_t)SK_LO * st, 0);
        if (lane < 32) dma16(rN, sb + SK_X + SK_LO + 512 * w, vN + (uint32_t)SK_NIB * st, 0);
    };

    v4i acc0[4], acc1[4];
    int sx0 = 0, sx1 = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) acc0[t] = acc1[t] = v4i{};
    // fragment offsets within a stage
    int oA[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int R = 16 * t + c, q = 4 * pp + g;
        oA[t] = R * 256 + ((q ^ (R & 15)) << 4);
    }
    const int oL = SK_X + 2048 * pp + 1024 * kbq + 16 * slot, oN = SK_X + SK_LO + 1024 * pp + 512 * kbq + 8 * slot;

    static_for<0, SK_NS - 1>([&](auto S) { issue(S, decltype(S)::value); });
    int st = 0;
    do {
        static_for<0, SK_NS>([&](auto S) {
            constexpr int sl = decltype(S)::value;
            const int s = st + sl;
            if (s < nst) {
                // stage s has landed once the DMAs of the SK_NS - 2 later stages are all that remain
                asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(SK_DMAS * (SK_NS - 2)) : "memory");
                // every wave is past stage s - 1: its buffer takes stage s + SK_NS - 1
                issue(slot_t<(sl + SK_NS - 1) % SK_NS>{}, s + SK_NS - 1);
                const int8_t* sb = ring + sl * SK_STAGE;
                v4i a[4];
#pragma unroll
                for (int t = 0; t < 4; t++) a[t] = *reinterpret_cast<const v4i*>(sb + oA[t]);
                const v4i lo = *reinterpret_cast<const v4i*>(sb + oL);
                const v4i hi = unpack_hi(*reinterpret_cast<const v2i*>(sb + oN));
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    acc0[t] = mfma16(a[t], lo, acc0[t]);
                    acc1[t] = mfma16(a[t], hi, acc1[t]);
                }
                if (ch == 0) sx0 += sum4(a[0]), sx1 += sum4(a[1]);
                else sx0 += sum4(a[2]), sx1 += sum4(a[3]);
            }
        });
        st += SK_NS;
    } while (st < nst);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // the ring is free (stages past the end landed)

    // the wave's partials (64 rows x its 16 columns) and its two tiles' row sums, into LDS
    int32_t* sP = reinterpret_cast<int32_t*>(ring);  // [8 waves][64 rows][16 columns]
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int r = 0; r < 4; r++)
            sP[(w * 64 + 16 * t + 4 * g + r) * 16 + c] = (int32_t)((uint32_t)acc0[t][r] + ((uint32_t)acc1[t][r] << 8));
    }
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        const int sv = add_xor32(add_xor16(tt ? sx1 : sx0));
        if (lane < 16) sX[pp][16 * (2 * ch + tt) + lane] = sv;
    }
    __syncthreads();
    const int cc = tid & 31, on = n0 + cc;  // every output of this thread is in column on
    const int32_t om = (OUT != KT_OUT_I64 && on < N) ? mant[on] : 0;
    const int32_t os = (OUT != KT_OUT_I64 && on < N) ? shift[on] : 0;
    const ColQ cq = col_q(om, os);
#pragma unroll
    for (int o = tid; o < OUTS; o += NT) {
        const int m = o >> 5, hc = cc >> 4, c16 = cc & 15;  // output (m0 + m, on); waves 4 hc .. 4 hc + 3 hold it
        uint32_t v = 0, rs = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) v += (uint32_t)sP[((4 * hc + q) * 64 + m) * 16 + c16], rs += (uint32_t)sX[q][m];
        const int vi = (int)(v - 1920u * rs);
        if (m < Mr && on < N) {
            const size_t idx = (size_t)(m0 + m) * N + on;
            if constexpr (OUT == KT_OUT_I64) reinterpret_cast<int64_t*>(y)[idx] = vi;
            else if constexpr (OUT == KT_OUT_I32) reinterpret_cast<int32_t*>(y)[idx] = col_requant<true>(vi, cq);
            else if constexpr (OUT == KT_OUT_I32_ADD) {
                int32_t* py = reinterpret_cast<int32_t*>(y) + idx;
                *py = sat_add32(*py, col_requant<true>(vi, cq));
            } else {
                const int qv = col_requant<false>(vi, cq);
                reinterpret_cast<int8_t*>(y)[idx] = lut ? lut[qv + 127] : (int8_t)qv;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// W12 skinny SwiGLU (M <= 16 * MT): the skinny kernel over a gate/up matrix packed with the 32-row interleave. A CTA
// owns 16 hidden units u0 .. u0 + 15: half hb of gate block 2j and the same half of up block 2j + 1 (adjacent in
// memory), both streamed in one pass over k. Epilogue: g, u = int8 requant per channel (gate channel u, up channel
// F + u), h = clamp(requant(silu[g + 127] * u, 1, h_shift)). Every dot is SMALL (kp <= 8128).
// ------------------------------------------------------------------------------------------------------------------
//
// FOLD_O (with NORM, one row, d <= 2 * 64 NW): the residual row is normalized with the o projection's requantized
// sums in fo.acc added first (r + requant_o(acc), saturating): the residual the reference's o QuantLinear leaves.
// The residual itself is not written here (other CTAs are reading it); the residual-add product after this one
// folds the same sums into it.
template <int MT, int NW, int U, bool NORM = false, bool FOLD_O = false>
__global__ __launch_bounds__(64 * NW) void w12_skinny_swiglu_kernel(
    const int8_t* __restrict__ x, const int8_t* __restrict__ wlo, const uint8_t* __restrict__ wnib,
    int8_t* __restrict__ y, int ystride, int M, int F, int kp, const int32_t* __restrict__ mant,
    const int32_t* __restrict__ shift, const int16_t* __restrict__ silu, int h_shift, int d, FoldO fo = {}) {
    constexpr int NT = 64 * NW, OUTS = MT * 256;
    static_assert(OUTS % NT == 0 || NT % OUTS == 0, "the threads tile the outputs");
    static_assert(!NORM || MT == 1, "the RMSNorm prologue serves M <= 16");
    static_assert(!FOLD_O || NORM, "FOLD_O folds into the RMSNorm prologue");
    __shared__ int32_t sPg[NW][OUTS], sPu[NW][OUTS];
    __shared__ int32_t sX[NW][MT * 16];
    __shared__ int16_t sSilu[256];
    extern __shared__ __attribute__((aligned(16))) int8_t sQ[];  // NORM: the normalized rows, M x kp
    __shared__ uint64_t sNss[NORM ? NW * 32 : 1], sNrq[NORM ? 32 : 1];
    int32_t pre[2];  // NORM: row 0 of the residual, loaded first
    if constexpr (NORM) norm_preload<64 * NW, 2>(reinterpret_cast<const int32_t*>(x), d, pre);
    int32_t fa[2] = {0, 0}, fm[2] = {0, 0}, fs[2] = {0, 0};  // FOLD_O: the o sums and scales of the same values
    if constexpr (FOLD_O) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = (int)threadIdx.x + j * NT;
            if (i < d) fa[j] = fo.acc[i], fm[j] = fo.mant[i], fs[j] = fo.shift[i];
        }
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int u0 = 16 * blockIdx.x, cbg = 2 * (u0 >> 5), hb = (u0 >> 4) & 1;
    const int KB = kp / 32;
    static_assert(NT >= 256, "one SiLU table entry per thread");
    const int16_t silu_v = tid < 256 ? silu[tid < 255 ? tid : 254] : 0;  // to LDS after the mainloop: no wait here

    const int oc = tid & 15, ou = u0 + oc;
    const int32_t gm = tid < OUTS ? mant[ou] : 0, gs = tid < OUTS ? shift[ou] : 0;
    const int32_t um = tid < OUTS ? mant[F + ou] : 0, us = tid < OUTS ? shift[F + ou] : 0;

    // gate block cbg and up block cbg + 1 are adjacent: one descriptor over both
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cbg * KB * 1024, 2u * (uint32_t)KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(wnib + (size_t)cbg * KB * 512, 2u * (uint32_t)KB * 512);
    const __amdgpu_buffer_rsrc_t rX = make_rsrc(x, (uint32_t)M * (uint32_t)kp);
    const int c = lane & 15, g = lane >> 4, kbq = g >> 1, h = g & 1;
    const int slot = 16 * hb + c + 32 * h;
    const uint32_t oL = 16 * slot + 1024 * kbq, oN = 8 * slot + 512 * kbq;
    const uint32_t uL = oL + (uint32_t)KB * 1024, uN = oN + (uint32_t)KB * 512;
    uint32_t oX[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) oX[t] = (uint32_t)(c + 16 * t) * (uint32_t)kp + 32 * kbq + 16 * h;

    v4i ag0[MT], ag1[MT], au0[MT], au1[MT];
    int sx[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) ag0[t] = ag1[t] = au0[t] = au1[t] = v4i{}, sx[t] = 0;

    v4i Lg[U], Lu[U], X[U][MT];
    v2i Dg[U], Du[U];
    const int np = KB / 2, nb = (np + NW * U - 1) / (NW * U);
    auto batch = [&](const int b) {  // as in w12_skinny_kernel; the RMSNorm variant runs one batch, loop-free
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int p = w + NW * (U * b + u);
            const uint32_t pl = (uint32_t)(p < np ? p : np - 1);
            Lg[u] = bload16nt(rL, oL, pl * 2048u);  // the weights: read once per launch
            Dg[u] = bload8nt(rN, oN, pl * 1024u);
            Lu[u] = bload16nt(rL, uL, pl * 2048u);
            Du[u] = bload8nt(rN, uN, pl * 1024u);
            if constexpr (!NORM) {
#pragma unroll
                for (int t = 0; t < MT; t++) X[u][t] = bload16(rX, oX[t], pl * 64u);
            }
        }
        if constexpr (NORM) {  // x rows from LDS, normalized there while the first weight loads are in flight
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (FOLD_O) {  // values past d stay 0: requant of a zero sum is 0
#pragma unroll
                for (int j = 0; j < 2; j++) pre[j] = sat_add32(pre[j], col_requant<true>(fa[j], col_q(fm[j], fs[j])));
            }
            norm_rows_to_lds<NT, 2>(reinterpret_cast<const int32_t*>(x), M, d, kp, sQ, sNss, sNrq, pre);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int p = w + NW * (U * b + u);
                const uint32_t pl = (uint32_t)(p < np ? p : np - 1);
                X[u][0] = c < M ? *reinterpret_cast<const v4i*>(sQ + (size_t)c * kp + pl * 64u + 32 * kbq + 16 * h)
                                : v4i{};
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int mask = 2 * (w + NW * (U * b + u)) + kbq < KB ? -1 : 0;
            const v4i hg = unpack_hi(Dg[u]), hu = unpack_hi(Du[u]);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i a = X[u][t] & mask;
                sx[t] += sum4(a);
                ag0[t] = mfma16(a, Lg[u], ag0[t]);
                ag1[t] = mfma16(a, hg, ag1[t]);
                au0[t] = mfma16(a, Lu[u], au0[t]);
                au1[t] = mfma16(a, hu, au1[t]);
            }
        }
    };
    if constexpr (NORM) {
        batch(0);
    } else {
        int b = 0;
        do batch(b);
        while (++b < nb);
    }

#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int o = (t * 16 + 4 * g + r) * 16 + c;
            sPg[w][o] = (int32_t)((uint32_t)ag0[t][r] + ((uint32_t)ag1[t][r] << 8));
            sPu[w][o] = (int32_t)((uint32_t)au0[t][r] + ((uint32_t)au1[t][r] << 8));
        }
        const int s = add_xor32(add_xor16(sx[t]));
        if (lane < 16) sX[w][t * 16 + lane] = s;
    }
    if (tid < 256) sSilu[tid] = silu_v;
    __syncthreads();
    const ColQ qg = col_q(gm, gs), qu = col_q(um, us);
#pragma unroll
    for (int o = tid; o < OUTS; o += NT) {
        const int m = o >> 4;
        uint32_t vg = 0, vu = 0, rs = 0;
#pragma unroll
        for (int q = 0; q < NW; q++) vg += (uint32_t)sPg[q][o], vu += (uint32_t)sPu[q][o], rs += (uint32_t)sX[q][m];
        const int gq = col_requant<false>((int)(vg - 1920u * rs), qg);
        const int uq = col_requant<false>((int)(vu - 1920u * rs), qu);
        if (m < M) y[(size_t)m * ystride + ou] = (int8_t)shift_rq8((int)sSilu[gq + 127] * uq, h_shift);
    }
}

// ------------------------------------------------------------------------------------------------------------------
// Lane-layout probe of the 32x32x32 and 16x16x64 int8 MFMAs (test hook): a and b are 64 lanes x 16 bytes each;
// c32 gets the 64 x 16 raw accumulator registers of one 32x32x32 product, c16 the 64 x 4 of one 16x16x64 product.
// ------------------------------------------------------------------------------------------------------------------
__global__ void mfma_probe_kernel(const int8_t* a, const int8_t* b, int32_t* c32, int32_t* c16) {
    const int l = threadIdx.x;
    v4i av = gload16(a + 16 * l), bv = gload16(b + 16 * l);
    v16i c = mfma32(av, bv, v16i{});
    v4i d = mfma16(av, bv, v4i{});
#pragma unroll
    for (int r = 0; r < 16; r++) c32[16 * l + r] = c[r];
#pragma unroll
    for (int r = 0; r < 4; r++) c16[4 * l + r] = d[r];
}

// ------------------------------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------------------------------

static inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

hipError_t launch_pack_planes(const int32_t* codes, int64_t rows, int64_t k, int p, int wrong_carry, int8_t* out,
                              hipStream_t s) {
    const int64_t kp = ceil_div(k, 64) * 64, total = rows * kp;
    if (total == 0) return hipSuccess;
    pack_planes_kernel<<<dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s>>>(codes, rows, k, kp, p, wrong_carry,
                                                                                  out);
    return hipGetLastError();
}

hipError_t launch_w12_pack(const int32_t* codes, int64_t n, int64_t k, int64_t ilv, int8_t* lo, uint8_t* nib,
                           hipStream_t s) {
    const int64_t kp = ceil_div(k, 64) * 64, total = ceil_div(n, 32) * (kp / 32) * 64;
    if (total == 0) return hipSuccess;
    if (ilv > 0 && (ilv % 32 || n != 2 * ilv)) return hipErrorInvalidValue;
    w12_pack_kernel<<<dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s>>>(codes, n, k, kp, ilv, lo, nib);
    return hipGetLastError();
}

// The tile shape of the digit-plane GEMM for px x pw planes: accumulators within ~160 registers (2x2 tiles of 32x32
// per wave for <= 2 plane-sum groups, 1x2 for <= 5, 1x1 beyond), and half-width tiles when 64 x 128 tiles would
// leave CUs idle (N = 896 at M = 512). Returns the number of tiles.
static int64_t plane_gemm_shape(int px, int pw, int M, int N, int& wtm, int& wtn) {
    const int ng = px + pw - 1;
    wtm = ng <= 2 ? 2 : 1, wtn = ng <= 5 ? 2 : 1;
    if (wtn == 2 && ceil_div(N, 64 * wtn) * ceil_div(M, 64 * wtm) < 256) wtn = 1;
    return ceil_div(N, 64 * wtn) * ceil_div(M, 64 * wtm);
}

int plane_gemm_splits(int px, int pw, int M, int N, int k0, int k1) {
    int wtm, wtn;
    const int64_t tiles = plane_gemm_shape(px, pw, M, N, wtm, wtn);
    const int nk = (k1 - k0) / 64;
    // the split costs atomic passes over the M x N outputs: worth it for long k (down: 76 k-tiles) or one row tile
    // (decode), not for short k over many rows (N = 896 at M = 512, K = 896: measured slower)
    if (M <= KT_PLANE_SKINNY_M || tiles >= 128 || nk < 2 || (nk < 24 && M > 64)) return 1;  // a few rows: skinny
    int want = (int)(256 / tiles);
    want = want > 4 ? 4 : (want < 1 ? 1 : want);
    want = want > nk ? nk : want;
    const int per = (nk + want - 1) / want;
    return (nk + per - 1) / per;  // every run of k-tiles is non-empty
}

int plane_gemm_cta_cols(int px, int pw, int M, int N) {
    if (M <= KT_PLANE_SKINNY_M) return 4 * PS_CPW;
    int wtm, wtn;
    plane_gemm_shape(px, pw, M, N, wtm, wtn);
    return 64 * wtn;
}

template <int PX, int PW>
static hipError_t plane_gemm_px_pw(const int8_t* xa, const int8_t* wb, int64_t* y, int M, int N, int kp, int k0,
                                   int k1, int accumulate, int drop_top, const int64_t* ql_bias, QlState* ql,
                                   int splits, unsigned* cnt, const QlSeg& seg, hipStream_t s) {
    if (M <= KT_PLANE_SKINNY_M) {
        if (splits != 1) return hipErrorInvalidValue;
        const dim3 grid((unsigned)ceil_div(N, 4 * PS_CPW));
        if (M == 1)
            plane_skinny_kernel<PX, PW, 1><<<grid, dim3(256), 0, s>>>(xa, wb, y, M, N, kp, k0, k1, accumulate,
                                                                     drop_top, ql_bias, ql, seg);
        else
            plane_skinny_kernel<PX, PW, KT_PLANE_SKINNY_M><<<grid, dim3(256), 0, s>>>(xa, wb, y, M, N, kp, k0, k1,
                                                                                     accumulate, drop_top, ql_bias,
                                                                                     ql, seg);
        return hipGetLastError();
    }
    int wtm, wtn;
    const int64_t tiles = plane_gemm_shape(PX, PW, M, N, wtm, wtn);
    const dim3 grid((unsigned)tiles, (unsigned)splits);
    constexpr int NG = PX + PW - 1, WTM = NG <= 2 ? 2 : 1;
    if (wtn == 1)
        plane_gemm_kernel<PX, PW, WTM, 1><<<grid, dim3(256), 0, s>>>(xa, wb, y, M, N, kp, k0, k1, accumulate,
                                                                     drop_top, ql_bias, ql, cnt, seg);
    else if constexpr (NG <= 5)
        plane_gemm_kernel<PX, PW, WTM, 2><<<grid, dim3(256), 0, s>>>(xa, wb, y, M, N, kp, k0, k1, accumulate,
                                                                     drop_top, ql_bias, ql, cnt, seg);
    return hipGetLastError();
}

hipError_t launch_plane_gemm(int px, int pw, const int8_t* xa, const int8_t* wb, int64_t* y, int M, int N, int kp,
                             int k0, int k1, int accumulate, int drop_top, hipStream_t s, const int64_t* ql_bias,
                             QlState* ql, int splits, unsigned* tile_cnt, const QlSeg* seg) {
    const QlSeg one{1, {0, N, N, N, N}};
    const QlSeg& sg = seg ? *seg : one;
    if (sg.n < 1 || sg.n > KT_QL_MAX_SEG) return hipErrorInvalidValue;
    if (M <= 0 || N <= 0 || k1 <= k0) return hipSuccess;
    if ((k0 % 64) || (k1 % 64) || k1 > kp || ceil_div(M, 64) * ceil_div(N, 64) > INT32_MAX) return hipErrorInvalidValue;
    if (splits != 1 && (splits != plane_gemm_splits(px, pw, M, N, k0, k1) || !tile_cnt || accumulate))
        return hipErrorInvalidValue;
#define KT_CASE(a, b) \
    if (px == a && pw == b)                                                                                  \
        return plane_gemm_px_pw<a, b>(xa, wb, y, M, N, kp, k0, k1, accumulate, drop_top, ql_bias, ql, splits, \
                                      tile_cnt, sg, s);
    KT_CASE(1, 1) KT_CASE(1, 3) KT_CASE(1, 5) KT_CASE(3, 1) KT_CASE(3, 3) KT_CASE(3, 5) KT_CASE(5, 1) KT_CASE(5, 3)
    KT_CASE(5, 5)
#undef KT_CASE
    return hipErrorInvalidValue;
}

// Whether the device gives one CTA the LDS-staged skinny kernel's ring; queried once per process.
static bool skinny_lds_ok() {
    static int ok = -1;
    if (ok < 0) {
        hipFuncAttributes fa;
        int dev = 0, mx = 0;
        ok = hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
             hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(&w12_skinny_lds_kernel<KT_OUT_I8>)) ==
                 hipSuccess &&
             fa.sharedSizeBytes + (size_t)SK_NS * SK_STAGE <= (size_t)mx;
    }
    return ok == 1;
}

template <int OUT>
static hipError_t w12_linear_out(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int N, int kp,
                                 const int32_t* mant, const int32_t* shift, const int8_t* lut, void* y, hipStream_t s) {
    if (lut && (OUT != KT_OUT_I8 || kp > KT_SMALL_KP)) return hipErrorInvalidValue;
    if (M <= KT_W12_SKINNY_MAX_M) {
        const int64_t ctas = 2 * ceil_div(N, 32);
        if (ctas > INT32_MAX || (int64_t)M * kp > (int64_t)UINT32_MAX || kp > KT_W12_SKINNY_MAX_K)
            return hipErrorInvalidValue;
        dim3 grid((unsigned)ctas);
#define KT_SKINNY(mt, nw, u)                                                                                        \
    if (M <= 16 * mt) {                                                                                             \
        if (kp <= KT_SMALL_KP)                                                                                      \
            w12_skinny_kernel<mt, nw, u, OUT, true><<<grid, dim3(64 * nw), 0, s>>>(x, lo, nib, y, M, N, kp, mant,   \
                                                                                   shift, lut, 0);                  \
        else                                                                                                        \
            w12_skinny_kernel<mt, nw, u, OUT, false><<<grid, dim3(64 * nw), 0, s>>>(x, lo, nib, y, M, N, kp, mant,  \
                                                                                    shift, nullptr, 0);             \
        return hipGetLastError();                                                                                   \
    }
        if (kp > 2048 && ctas < 256) {  // long k, few CTAs (M <= 16): 16 waves x 5 pairs, up to kp 5120 in one batch
            KT_SKINNY(1, 16, 5)
        }
        if (kp <= 1024) {  // short k at M <= 16: 8 waves x 2 pairs cover kp in one batch with fewer clamped re-reads
            KT_SKINNY(1, 8, 2)
        }
        // 65-128 rows with int32 dots: x staged through LDS (w12_skinny_lds_kernel)
        if (M > 64 && kp <= KT_SMALL_KP && skinny_lds_ok()) {
            // CTA b: rows 64 ((b >> 3) & 1), column block (b & 7) | ((b >> 4) << 3): 16 * ceil(ncb / 8) CTAs, the
            // ones past the last column block idle
            const int64_t ncb = ceil_div(N, 32), grid_l = 16 * ceil_div(ncb, 8);
            w12_skinny_lds_kernel<OUT><<<dim3((unsigned)grid_l), dim3(512), (size_t)SK_NS * SK_STAGE, s>>>(
                x, lo, nib, y, M, N, kp, mant, shift, lut);
            return hipGetLastError();
        }
        // otherwise 65-128 rows: 8 waves x 2 pairs (21.8 us at M = 128, N = K = 4096, against 22.4 for 4 waves x 4
        // pairs, 25.3 for 4 x 8 and 31.0 for 8 x 4)
        KT_SKINNY(1, 8, 4) KT_SKINNY(2, 8, 4) KT_SKINNY(4, 8, 2) KT_SKINNY(8, 8, 2)
#undef KT_SKINNY
    }
    const bool small = kp <= KT_SMALL_KP;
    constexpr int WM = KT_W12_WM, WTM = KT_W12_WTM, WTN = KT_W12_WTN, WV = KT_W12_WAVES, NS = KT_W12_NSLOT;
    const int64_t tiles4 = ceil_div(N, 32 * WTN * 4) * ceil_div(M, 32 * WTM * WM);
    // Fewer 128 x 128 tiles than CUs: 64 x 128 tiles, or 64 x 64 (128 threads) when even those leave CUs idle, so
    // small products (prefill projections, the SAM MLP) spread over the chip
    const int64_t tiles_h = ceil_div(N, 128) * ceil_div(M, 64), tiles_q = ceil_div(N, 64) * ceil_div(M, 64);
    const int64_t tiles_e = ceil_div(N, 64) * ceil_div(M, 32);
    if (tiles4 < 256 && small) {
        if (tiles_h >= 256 || tiles_q <= tiles_h) {
            w12_gemm_kernel<1, 2, 1, WV, NS, OUT, true><<<dim3((unsigned)tiles_h), dim3(256), 0, s>>>(
                x, lo, nib, y, M, N, kp, mant, shift, lut);
        } else if (tiles_q < 256 && tiles_e <= 512) {
            // even 64 x 64 tiles leave CUs idle: 32 x 64 tiles, twice the CTAs (config 3's prefill o and down)
            w12_gemm_kernel<1, 1, 1, WV, NS, OUT, true, 2><<<dim3((unsigned)tiles_e), dim3(128), 0, s>>>(
                x, lo, nib, y, M, N, kp, mant, shift, lut);
        } else {
            w12_gemm_kernel<1, 2, 1, WV, NS, OUT, true, 2><<<dim3((unsigned)tiles_q), dim3(128), 0, s>>>(
                x, lo, nib, y, M, N, kp, mant, shift, lut);
        }
        return hipGetLastError();
    }
#if KT_W12_DMA
    // enough 256 x 128 tiles to give at least 7/8 of the CUs one: the DMA-fed kernel (config 5's MLP in, 224 tiles:
    // 4-6% faster than its 448 tiles of 128 x 128, which leave the same CU time idle in their second round)
    const int64_t tiles_d = ceil_div(N, 128) * ceil_div(M, 256);
    if (tiles_d >= 224 && dma_lds_ok()) {
        const size_t lds = (size_t)KT_DMA_NS * KT_DMA_STAGE;
        if (small)
            w12_gemm_dma_kernel<OUT, true><<<dim3((unsigned)tiles_d), dim3(512), lds, s>>>(x, lo, nib, y, M, N, kp,
                                                                                       mant, shift, lut);
        else
            w12_gemm_dma_kernel<OUT, false><<<dim3((unsigned)tiles_d), dim3(512), lds, s>>>(x, lo, nib, y, M, N, kp,
                                                                                        mant, shift, nullptr);
        return hipGetLastError();
    }
#endif
    dim3 grid((unsigned)tiles4), block(256 * WM);
    if (small)
        w12_gemm_kernel<WM, WTM, WTN, WV, NS, OUT, true><<<grid, block, 0, s>>>(x, lo, nib, y, M, N, kp, mant, shift, lut);
    else
        w12_gemm_kernel<WM, WTM, WTN, WV, NS, OUT, false><<<grid, block, 0, s>>>(x, lo, nib, y, M, N, kp, mant, shift,
                                                                                 nullptr);
    return hipGetLastError();
}

hipError_t launch_w12_linear(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int N, int kp,
                             const int32_t* mant, const int32_t* shift, const int8_t* lut, int out_kind, void* y,
                             hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (kp <= 0 || (kp % 64) || ceil_div(M, 64) * ceil_div(N, 64) > INT32_MAX) return hipErrorInvalidValue;
    switch (out_kind) {
        case KT_OUT_I64: return w12_linear_out<KT_OUT_I64>(x, lo, nib, M, N, kp, mant, shift, lut, y, s);
        case KT_OUT_I32: return w12_linear_out<KT_OUT_I32>(x, lo, nib, M, N, kp, mant, shift, lut, y, s);
        case KT_OUT_I32_ADD: return w12_linear_out<KT_OUT_I32_ADD>(x, lo, nib, M, N, kp, mant, shift, lut, y, s);
        case KT_OUT_I8: return w12_linear_out<KT_OUT_I8>(x, lo, nib, M, N, kp, mant, shift, lut, y, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_w12b_pack(const int32_t* codes, int64_t n, int64_t k, int8_t* lo, int8_t* hi, hipStream_t s) {
    const int64_t kp = ceil_div(k, 64) * 64, total = ceil_div(n, 32) * (kp / 32) * 64;
    if (total == 0) return hipSuccess;
    w12b_pack_kernel<<<dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s>>>(codes, n, k, kp, lo, hi);
    return hipGetLastError();
}

// The balanced-plane product: always the DMA-fed 256 x 128 kernel (built for m that gives every CU a tile; any m
// and n are correct: rows and columns past them read as zero and are not stored).
template <int OUT>
static hipError_t w12b_linear_out(const int8_t* x, const int8_t* lo, const int8_t* hi, int M, int N, int kp,
                                  const int32_t* mant, const int32_t* shift, void* y, hipStream_t s) {
    if (!dma_lds_ok()) return hipErrorInvalidConfiguration;
    const int64_t tiles_d = ceil_div(N, 128) * ceil_div(M, 256);
    if (tiles_d > INT32_MAX) return hipErrorInvalidValue;
    const size_t lds = (size_t)KT_DMA_NS * KT_DMA_STAGE_BAL;
    const uint8_t* h = reinterpret_cast<const uint8_t*>(hi);
    if (kp <= KT_SMALL_KP)
        w12_gemm_dma_kernel<OUT, true, true><<<dim3((unsigned)tiles_d), dim3(512), lds, s>>>(x, lo, h, y, M, N, kp,
                                                                                          mant, shift, nullptr);
    else
        w12_gemm_dma_kernel<OUT, false, true><<<dim3((unsigned)tiles_d), dim3(512), lds, s>>>(x, lo, h, y, M, N, kp,
                                                                                           mant, shift, nullptr);
    return hipGetLastError();
}

hipError_t launch_w12b_linear(const int8_t* x, const int8_t* lo, const int8_t* hi, int M, int N, int kp,
                              const int32_t* mant, const int32_t* shift, int out_kind, void* y, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (kp <= 0 || (kp % 64)) return hipErrorInvalidValue;
    switch (out_kind) {
        case KT_OUT_I64: return w12b_linear_out<KT_OUT_I64>(x, lo, hi, M, N, kp, mant, shift, y, s);
        case KT_OUT_I32: return w12b_linear_out<KT_OUT_I32>(x, lo, hi, M, N, kp, mant, shift, y, s);
        case KT_OUT_I32_ADD: return w12b_linear_out<KT_OUT_I32_ADD>(x, lo, hi, M, N, kp, mant, shift, y, s);
        case KT_OUT_I8: return w12b_linear_out<KT_OUT_I8>(x, lo, hi, M, N, kp, mant, shift, y, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_w12_swiglu(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int F, int kp,
                             const int32_t* mant, const int32_t* shift, const int16_t* silu, int h_shift, int8_t* y,
                             int ystride, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    if (F <= 0 || F % 32 || kp <= 0 || kp % 64 || kp > KT_SMALL_KP || h_shift < 1 || h_shift > 30 || ystride < F ||
        (int64_t)M * kp > (int64_t)UINT32_MAX)
        return hipErrorInvalidValue;
    if (M <= KT_W12_SKINNY_MAX_M) {
        dim3 grid((unsigned)(F / 16));
#define KT_SWIGLU(mt, nw, u)                                                                                         \
    if (M <= 16 * mt) {                                                                                              \
        w12_skinny_swiglu_kernel<mt, nw, u><<<grid, dim3(64 * nw), 0, s>>>(x, lo, nib, y, ystride, M, F, kp, mant,  \
                                                                           shift, silu, h_shift, 0);                 \
        return hipGetLastError();                                                                                    \
    }
        if (kp <= 1024) {
            KT_SWIGLU(1, 8, 2)
        }
        KT_SWIGLU(1, 8, 4) KT_SWIGLU(2, 8, 2) KT_SWIGLU(4, 8, 1) KT_SWIGLU(8, 4, 2)
#undef KT_SWIGLU
    }
    return hipErrorInvalidValue;  // the caller takes the grouped kernel (one group) for longer batches
}

// The RMSNorm-fused skinny products (M <= 16): x is the int32 residual, M rows of d values; kp = d rounded up to 64.
static bool norm_shape_ok(int M, int d, int kp) {  // one batch of 8 waves x 4 pairs of k32 blocks: kp <= 2048
    return M >= 1 && M <= 16 && d >= 1 && kp == (d + 63) / 64 * 64 && kp <= KT_NORM_MAX_D &&
           (int64_t)M * kp <= KT_NORM_LDS_MAX;
}

template <int U>
static hipError_t linear_norm_u(const int8_t* x, int M, int d, int kp, const int8_t* lo, const uint8_t* nib, int N,
                                const int32_t* mant, const int32_t* shift, int out_kind, void* y, hipStream_t s) {
    dim3 grid((unsigned)(2 * ceil_div(N, 32))), block(64 * 8);
    const size_t lds = (size_t)M * kp;
    switch (out_kind) {
        case KT_OUT_I64:
            w12_skinny_kernel<1, 8, U, KT_OUT_I64, true, true><<<grid, block, lds, s>>>(x, lo, nib, y, M, N, kp, mant,
                                                                                       shift, nullptr, d);
            break;
        case KT_OUT_I32:
            w12_skinny_kernel<1, 8, U, KT_OUT_I32, true, true><<<grid, block, lds, s>>>(x, lo, nib, y, M, N, kp, mant,
                                                                                       shift, nullptr, d);
            break;
        case KT_OUT_I8:
            w12_skinny_kernel<1, 8, U, KT_OUT_I8, true, true><<<grid, block, lds, s>>>(x, lo, nib, y, M, N, kp, mant,
                                                                                      shift, nullptr, d);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// U (pairs of k32 blocks per wave) is the smallest that covers kp in one batch of 8 waves: fewer clamped re-reads.
hipError_t launch_w12_linear_norm(const int32_t* r, int M, int d, const int8_t* lo, const uint8_t* nib, int N,
                                  const int32_t* mant, const int32_t* shift, int out_kind, void* y, hipStream_t s) {
    const int kp = (d + 63) / 64 * 64;
    if (N <= 0 || !norm_shape_ok(M, d, kp) || 2 * ceil_div(N, 32) > INT32_MAX) return hipErrorInvalidValue;
    const int8_t* x = reinterpret_cast<const int8_t*>(r);
    if (kp <= 1024) return linear_norm_u<2>(x, M, d, kp, lo, nib, N, mant, shift, out_kind, y, s);
    return linear_norm_u<4>(x, M, d, kp, lo, nib, N, mant, shift, out_kind, y, s);
}

hipError_t launch_w12_swiglu_norm(const int32_t* r, int M, int d, const int8_t* lo, const uint8_t* nib, int F,
                                  const int32_t* mant, const int32_t* shift, const int16_t* silu, int h_shift,
                                  int8_t* y, int ystride, hipStream_t s) {
    const int kp = (d + 63) / 64 * 64;
    if (F <= 0 || F % 32 || !norm_shape_ok(M, d, kp) || h_shift < 1 || h_shift > 30 || ystride < F)
        return hipErrorInvalidValue;
    dim3 grid((unsigned)(F / 16)), block(64 * 8);
    const int8_t* x = reinterpret_cast<const int8_t*>(r);
    if (kp <= 1024)
        w12_skinny_swiglu_kernel<1, 8, 2, true><<<grid, block, (size_t)M * kp, s>>>(x, lo, nib, y, ystride, M, F, kp,
                                                                                    mant, shift, silu, h_shift, d);
    else
        w12_skinny_swiglu_kernel<1, 8, 4, true><<<grid, block, (size_t)M * kp, s>>>(x, lo, nib, y, ystride, M, F, kp,
                                                                                    mant, shift, silu, h_shift, d);
    return hipGetLastError();
}

// The decode step's gate/up product with the attention's o sums folded into the normalized residual: one row,
// d <= 1024 (the two preloaded values per thread cover the row).
hipError_t launch_w12_swiglu_norm_o(const int32_t* r, int d, const int8_t* lo, const uint8_t* nib, int F,
                                    const int32_t* mant, const int32_t* shift, const int16_t* silu, int h_shift,
                                    int8_t* y, const int32_t* oacc, const int32_t* omant, const int32_t* oshift,
                                    hipStream_t s) {
    const int kp = (d + 63) / 64 * 64;
    if (F <= 0 || F % 32 || !norm_shape_ok(1, d, kp) || kp > 1024 || h_shift < 1 || h_shift > 30 || !oacc ||
        !omant || !oshift)
        return hipErrorInvalidValue;
    const FoldO fo{const_cast<int32_t*>(oacc), omant, oshift};  // read only here
    w12_skinny_swiglu_kernel<1, 8, 2, true, true><<<dim3((unsigned)(F / 16)), dim3(512), (size_t)kp, s>>>(
        reinterpret_cast<const int8_t*>(r), lo, nib, y, F, 1, F, kp, mant, shift, silu, h_shift, d, fo);
    return hipGetLastError();
}

// The decode step's residual-add product (one row) that also folds the o sums into the residual and clears them;
// the launch shapes of w12_linear_out for M = 1.
hipError_t launch_w12_linear_add_o(const int8_t* x, const int8_t* lo, const uint8_t* nib, int N, int kp,
                                   const int32_t* mant, const int32_t* shift, int32_t* y, int32_t* oacc,
                                   const int32_t* omant, const int32_t* oshift, hipStream_t s) {
    if (N <= 0 || kp <= 0 || kp % 64 || kp > KT_SMALL_KP || !oacc || !omant || !oshift) return hipErrorInvalidValue;
    const int64_t ctas = 2 * ceil_div(N, 32);
    if (ctas > INT32_MAX) return hipErrorInvalidValue;
    const FoldO fo{oacc, omant, oshift};
    const dim3 grid((unsigned)ctas);
    if (kp > 2048 && ctas < 256)
        w12_skinny_kernel<1, 16, 5, KT_OUT_I32_ADD, true, false, true><<<grid, dim3(1024), 0, s>>>(
            x, lo, nib, y, 1, N, kp, mant, shift, nullptr, 0, fo);
    else if (kp <= 1024)
        w12_skinny_kernel<1, 8, 2, KT_OUT_I32_ADD, true, false, true><<<grid, dim3(512), 0, s>>>(
            x, lo, nib, y, 1, N, kp, mant, shift, nullptr, 0, fo);
    else
        w12_skinny_kernel<1, 8, 4, KT_OUT_I32_ADD, true, false, true><<<grid, dim3(512), 0, s>>>(
            x, lo, nib, y, 1, N, kp, mant, shift, nullptr, 0, fo);
    return hipGetLastError();
}

// A pure read of `bytes` (a multiple of 16) with the GEMV's load form: KT_STREAM_READ_CTAS CTAs of 512 threads, CTA b
// over the b-th contiguous chunk (a multiple of 16 bytes), 16-byte buffer loads, 4 per thread in flight before any is
// used; out[b] = the XOR of the chunk's 32-bit words (so no load can be dropped). A measurement of what the memory
// delivers to this load form with no compute, beside the products that stream the same bytes. (Over 25 MB, a sweep of
// 4-32 loads per thread, 256-1024 threads and 256-2048 CTAs found none faster than this shape by more than 1%.)
__global__ __launch_bounds__(512) void stream_read_kernel(const uint8_t* __restrict__ src, uint32_t bytes,
                                                          uint32_t chunk, uint32_t* __restrict__ out) {
    __shared__ uint32_t red[8];
    const uint32_t b = blockIdx.x, off = b * chunk;
    const uint32_t len = off >= bytes ? 0u : (bytes - off < chunk ? bytes - off : chunk);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src + (len ? off : 0u), len);  // loads past len read as zero
    v4i acc = {};
    for (uint32_t o = 16u * threadIdx.x; o < len; o += 4u * 512u * 16u) {
        v4i v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = bload16(r, o + (uint32_t)u * 512u * 16u, 0);
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u];
    }
    uint32_t x = (uint32_t)(acc.x ^ acc.y ^ acc.z ^ acc.w);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) x ^= (uint32_t)__shfl_xor((int)x, d);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) t ^= red[q];
        out[b] = t;
    }
}

hipError_t launch_stream_read(const uint8_t* src, uint32_t bytes, uint32_t* out, hipStream_t s) {
    const uint32_t chunk = (uint32_t)ceil_div(ceil_div((int64_t)bytes, KT_STREAM_READ_CTAS), 16) * 16u;
    stream_read_kernel<<<dim3(KT_STREAM_READ_CTAS), dim3(512), 0, s>>>(src, bytes, chunk ? chunk : 16u, out);
    return hipGetLastError();
}

hipError_t launch_mfma_probe(const int8_t* a, const int8_t* b, int32_t* c32, int32_t* c16, hipStream_t s) {
    mfma_probe_kernel<<<dim3(1), dim3(64), 0, s>>>(a, b, c32, c16);
    return hipGetLastError();
}

}  // namespace kt
