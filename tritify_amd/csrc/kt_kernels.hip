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
// 2. W12 (int8 activations x 12-bit weight codes in [-2048, 2047]):
//    lo plane [n][kp] int8 = (v & 255) - 128, nib plane [n][kp/2] holding hi = (v + 2048) >> 8 in [0, 15], so that
//    v = lo + 256*hi - 1920 and sum_k x*v = S_lo + 256*S_hi - 1920*sum_k x. In each 16-byte nib group (32 k-values
//    of one row) dword q has k = 8q..8q+3 in its low nibbles and k = 8q+4..8q+7 in its high nibbles, so one AND and
//    one shift+AND unpack eight codes into two int8 dwords in natural k order.
//
// MFMA: v_mfma_i32_32x32x32_i8 (GEMM) and, for skinny M, v_mfma_i32_16x16x64_i8. A lane's 16 operand bytes are
// 16 consecutive k of one row (A) / one column (B); the hardware pairs A and B bytes with the same k-slot, so any
// lane->k assignment that is the same for A and B gives the exact dot product. The C layout of the 32x32 MFMA is
// lane l, register r -> row 8*(r/4) + 4*(l/32) + (r%4), column l%32; of the 16x16 MFMA: row 4*(l/16) + r, col l%16
// (checked by the layout test in tests/test_gpu.py).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kt_kernels.h"

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
// MFMA operand reads (consecutive lanes = consecutive rows, same chunk) fall in distinct banks.
template <int CPR>
__device__ __forceinline__ int swz(int r) {
    if constexpr (CPR == 4) return ((r >> 1) ^ (r >> 3)) & 3;
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
__device__ __forceinline__ v2i gload8(const uint8_t* p) { return *reinterpret_cast<const v2i*>(p); }

// 16 nibble bytes (32 codes of one nib group) -> two 16-byte chunks of the hi plane in natural k order.
__device__ __forceinline__ void unpack_nib(v4i d, v4i& h0, v4i& h1) {
    const int m = 0x0F0F0F0F;
    h0 = v4i{d.x & m, (d.x >> 4) & m, d.y & m, (d.y >> 4) & m};
    h1 = v4i{d.z & m, (d.z >> 4) & m, d.w & m, (d.w >> 4) & m};
}

__device__ __forceinline__ int sum4(v4i v) {
    const int ones = 0x01010101;
    int s = __builtin_amdgcn_sdot4(v.x, ones, 0, false);
    s = __builtin_amdgcn_sdot4(v.y, ones, s, false);
    s = __builtin_amdgcn_sdot4(v.z, ones, s, false);
    return __builtin_amdgcn_sdot4(v.w, ones, s, false);
}

// round(acc * mant / 2^shift), half away from zero, widening product (crates/00-kernels/kt-int/src/lib.rs:78-86).
__device__ __forceinline__ int64_t requant_dev(int64_t acc, int64_t mant, int shift) {
    __int128 prod = (__int128)acc * (__int128)mant;
    if (shift <= 0) return (int64_t)(prod << (-shift));
    __int128 half = (__int128)1 << (shift - 1);
    __int128 r = prod >= 0 ? (prod + half) >> shift : -(((-prod) + half) >> shift);
    return (int64_t)r;
}

template <int OUT>
__device__ __forceinline__ void store_out(void* y, size_t idx, int64_t v, const int32_t* mant, const int32_t* shift,
                                          int n) {
    if constexpr (OUT == KT_OUT_I64) {
        reinterpret_cast<int64_t*>(y)[idx] = v;
    } else {
        int64_t q = requant_dev(v, mant[n], shift[n]);
        if constexpr (OUT == KT_OUT_I32) {
            q = q > INT32_MAX ? INT32_MAX : (q < INT32_MIN ? INT32_MIN : q);
            reinterpret_cast<int32_t*>(y)[idx] = (int32_t)q;
        } else {
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            reinterpret_cast<int8_t*>(y)[idx] = (int8_t)q;
        }
    }
}

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

// i32 codes [n][k] in [-2048, 2047] -> W12 planes (lo [n][kp], nib [n][kp/2]). One thread per nib byte.
__global__ void w12_pack_kernel(const int32_t* __restrict__ codes, int64_t n, int64_t k, int64_t kp,
                                int8_t* __restrict__ lo, uint8_t* __restrict__ nib) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t per_row = kp / 2;
    if (idx >= n * per_row) return;
    int64_t r = idx / per_row, b = idx - r * per_row;
    int64_t g = b >> 4, bi = b & 15;
    int64_t c0 = g * 32 + (bi >> 2) * 8 + (bi & 3), c1 = c0 + 4;
    int8_t l0 = 0, l1 = 0;  // padding (k..kp) is lo = 0, hi = 0
    uint32_t h0 = 0, h1 = 0;
    if (c0 < k) {
        int32_t v = codes[r * k + c0];
        l0 = (int8_t)((v & 255) - 128);
        h0 = ((uint32_t)(v + 2048) >> 8) & 15;
    }
    if (c1 < k) {
        int32_t v = codes[r * k + c1];
        l1 = (int8_t)((v & 255) - 128);
        h1 = ((uint32_t)(v + 2048) >> 8) & 15;
    }
    lo[r * kp + c0] = l0;
    lo[r * kp + c1] = l1;
    nib[idx] = (uint8_t)(h0 | (h1 << 4));
}

// ------------------------------------------------------------------------------------------------------------------
// Digit-plane GEMM (LinearBackend path). CTA = 4 waves in 2x2; each wave WTM x WTN tiles of 32x32; BK = 64.
// Processes k in [k0, k1) (multiples of 64) and writes y = result (first chunk) or y += result.
// ------------------------------------------------------------------------------------------------------------------
template <int PX, int PW, int WTM, int WTN>
__global__ __launch_bounds__(256) void plane_gemm_kernel(const int8_t* __restrict__ xa, const int8_t* __restrict__ wb,
                                                         int64_t* __restrict__ y, int M, int N, int kp, int k0,
                                                         int k1, int accumulate, int drop_top) {
    constexpr int BK = 64, CPR = BK / 16;
    constexpr int BM = 64 * WTM, BN = 64 * WTN;
    constexpr int NG = PX + PW - 1;
    constexpr int AL = BM * CPR / 256, BL = BN * CPR / 256;  // 16-byte chunks per thread per plane
    static_assert(AL >= 1 && BL >= 1, "tile too small for 256 threads");
    __shared__ __attribute__((aligned(16))) int8_t sA[2][PX][BM * BK];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][PW][BN * BK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_n = (N + BN - 1) / BN;
    const int m0 = (blockIdx.x / tiles_n) * BM, n0 = (blockIdx.x % tiles_n) * BN;
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
                if (m < M && n < N) {
                    int64_t* p = y + (size_t)m * N + n;
                    *p = accumulate ? (int64_t)((uint64_t)*p + v) : (int64_t)v;
                }
            }
        }
}

// ------------------------------------------------------------------------------------------------------------------
// W12 GEMM (BASELINE path, M >= 16). x int8 [M][lda] (lda = kp, zero padded), W12 lo [N][kp], nib [N][kp/2].
// CTA = 4 waves in 2x2, each WTM x WTN tiles of 32x32; the hi plane is unpacked once per CTA on its way into LDS.
// The row sums of x (for the -1920*sum_k x term) come from the A staging registers.
// ------------------------------------------------------------------------------------------------------------------
template <int WTM, int WTN, int BK, int OUT>
__global__ __launch_bounds__(256) void w12_gemm_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ wlo,
                                                       const uint8_t* __restrict__ wnib, void* __restrict__ y,
                                                       int M, int N, int kp, const int32_t* __restrict__ mant,
                                                       const int32_t* __restrict__ shift) {
    constexpr int CPR = BK / 16;
    constexpr int BM = 64 * WTM, BN = 64 * WTN;
    constexpr int AL = BM * CPR / 256, BL = BN * CPR / 256;
    constexpr int NC = BN * (BK / 32), NL = (NC + 255) / 256;  // 16-byte nib chunks of a tile
    static_assert(AL >= 1 && BL >= 1, "tile too small for 256 threads");
    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * BK];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][2][BN * BK];
    __shared__ int sRow[BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_n = (N + BN - 1) / BN;
    const int m0 = (blockIdx.x / tiles_n) * BM, n0 = (blockIdx.x % tiles_n) * BN;
    const size_t ldn = (size_t)kp / 2;

    v16i acc0[WTM][WTN], acc1[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++) acc0[i][j] = acc1[i][j] = v16i{};

    int rsum[AL];
#pragma unroll
    for (int i = 0; i < AL; i++) rsum[i] = 0;

    v4i ra[AL], rl[BL], rn[NL];
    auto gload_tile = [&](int k) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
            int gr = m0 + r;
            ra[i] = gr < M ? gload16(x + (size_t)gr * kp + k + 16 * c) : v4i{};
        }
#pragma unroll
        for (int i = 0; i < BL; i++) {
            int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
            int gr = n0 + r;
            rl[i] = gr < N ? gload16(wlo + (size_t)gr * kp + k + 16 * c) : v4i{};
        }
#pragma unroll
        for (int i = 0; i < NL; i++) {
            int idx = tid + 256 * i, r = idx / (BK / 32), g = idx % (BK / 32);
            int gr = n0 + r;
            rn[i] = (idx < NC && gr < N) ? gload16(reinterpret_cast<const int8_t*>(wnib) + (size_t)gr * ldn + k / 2 + 16 * g)
                           : v4i{};
        }
    };
    auto lstore_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
            lds_write16(sA[buf], lds_off<CPR>(r, c), ra[i]);
            rsum[i] += sum4(ra[i]);
        }
#pragma unroll
        for (int i = 0; i < BL; i++) {
            int idx = tid + 256 * i, r = idx / CPR, c = idx % CPR;
            lds_write16(sB[buf][0], lds_off<CPR>(r, c), rl[i]);
        }
#pragma unroll
        for (int i = 0; i < NL; i++) {
            int idx = tid + 256 * i, r = idx / (BK / 32), g = idx % (BK / 32);
            if (NC % 256 != 0 && idx >= NC) continue;
            v4i h0, h1;
            unpack_nib(rn[i], h0, h1);
            lds_write16(sB[buf][1], lds_off<CPR>(r, 2 * g), h0);
            lds_write16(sB[buf][1], lds_off<CPR>(r, 2 * g + 1), h1);
        }
    };

    const int nk = kp / BK;
    gload_tile(0);
    lstore_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload_tile((kt + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            const int chunk = 2 * ks + (lane >> 5);
            v4i a[WTM], b0[WTN], b1[WTN];
#pragma unroll
            for (int i = 0; i < WTM; i++) {
                int r = wm * 32 * WTM + i * 32 + (lane & 31);
                a[i] = lds_read16(sA[cur], lds_off<CPR>(r, chunk));
            }
#pragma unroll
            for (int j = 0; j < WTN; j++) {
                int r = wn * 32 * WTN + j * 32 + (lane & 31);
                b0[j] = lds_read16(sB[cur][0], lds_off<CPR>(r, chunk));
                b1[j] = lds_read16(sB[cur][1], lds_off<CPR>(r, chunk));
            }
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int j = 0; j < WTN; j++) {
                    acc0[i][j] = mfma32(a[i], b0[j], acc0[i][j]);
                    acc1[i][j] = mfma32(a[i], b1[j], acc1[i][j]);
                }
        }
        if (kt + 1 < nk) lstore_tile(cur ^ 1);
        __syncthreads();
    }

    // row sums: the CPR threads of one row are consecutive lanes of one wave
#pragma unroll
    for (int i = 0; i < AL; i++) {
        int s = rsum[i];
#pragma unroll
        for (int o = 1; o < CPR; o <<= 1) s += __shfl_xor(s, o);
        int idx = tid + 256 * i;
        if ((idx % CPR) == 0) sRow[idx / CPR] = s;
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++) {
            const int n = n0 + wn * 32 * WTN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int rl_ = wm * 32 * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int m = m0 + rl_;
                int64_t v = (int64_t)acc0[i][j][r] + 256 * (int64_t)acc1[i][j][r] - 1920 * (int64_t)sRow[rl_];
                if (m < M && n < N) store_out<OUT>(y, (size_t)m * N + n, v, mant, shift, n);
            }
        }
}

// ------------------------------------------------------------------------------------------------------------------
// W12 GEMV (batch decode, M <= 8). Bandwidth-bound: each wave owns NR output channels and streams their packed
// codes with coalesced 16-byte (lo) and 8-byte (nib) loads -- lane j of chunk i reads k = 1024 i + 16 j .. +16 --
// dots them against x with v_dot4_i32_i8, and reduces the lanes with DPP and ds_swizzle.
// ------------------------------------------------------------------------------------------------------------------

// Sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ int wave_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]: lane ^ 1
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]: lane ^ 2
    v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true); // row_half_mirror: the other quad of 8
    v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true); // row_mirror: the other half of the row of 16
    v += __builtin_amdgcn_ds_swizzle(v, 0x401F);             // xor 16 within 32 lanes
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 32);
}

template <int MR, int NR, int OUT>
__global__ __launch_bounds__(256) void w12_gemv_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ wlo,
                                                       const uint8_t* __restrict__ wnib, void* __restrict__ y,
                                                       int M, int N, int kp, const int32_t* __restrict__ mant,
                                                       const int32_t* __restrict__ shift) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nbase = (blockIdx.x * 4 + wave) * NR;
    if (nbase >= N) return;  // whole wave leaves; no barrier follows
    const size_t ldn = (size_t)kp / 2;
    const int mask = 0x0F0F0F0F, ones = 0x01010101;

    int slo[MR][NR], shi[MR][NR], sx[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
        sx[m] = 0;
#pragma unroll
        for (int r = 0; r < NR; r++) slo[m][r] = shi[m][r] = 0;
    }

    constexpr int U = 4;  // chunks in flight per row
    for (int c0 = 0; c0 * 1024 < kp; c0 += U) {
        v4i L[U][NR];
        v2i D[U][NR];
        v4i X[U][MR];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int kk = (c0 + u) * 1024 + 16 * lane;
            const bool ok = kk < kp;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const int n = nbase + r;
                const bool v = ok && n < N;
                L[u][r] = v ? gload16(wlo + (size_t)n * kp + kk) : v4i{};
                D[u][r] = v ? gload8(wnib + (size_t)n * ldn + kk / 2) : v2i{};
            }
#pragma unroll
            for (int m = 0; m < MR; m++) X[u][m] = (ok && m < M) ? gload16(x + (size_t)m * kp + kk) : v4i{};
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int m = 0; m < MR; m++) {
                sx[m] = __builtin_amdgcn_sdot4(X[u][m].x, ones, sx[m], false);
                sx[m] = __builtin_amdgcn_sdot4(X[u][m].y, ones, sx[m], false);
                sx[m] = __builtin_amdgcn_sdot4(X[u][m].z, ones, sx[m], false);
                sx[m] = __builtin_amdgcn_sdot4(X[u][m].w, ones, sx[m], false);
            }
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const int h0 = D[u][r].x & mask, h1 = (D[u][r].x >> 4) & mask;
                const int h2 = D[u][r].y & mask, h3 = (D[u][r].y >> 4) & mask;
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    int s = slo[m][r], t = shi[m][r];
                    s = __builtin_amdgcn_sdot4(X[u][m].x, L[u][r].x, s, false);
                    s = __builtin_amdgcn_sdot4(X[u][m].y, L[u][r].y, s, false);
                    s = __builtin_amdgcn_sdot4(X[u][m].z, L[u][r].z, s, false);
                    s = __builtin_amdgcn_sdot4(X[u][m].w, L[u][r].w, s, false);
                    t = __builtin_amdgcn_sdot4(X[u][m].x, h0, t, false);
                    t = __builtin_amdgcn_sdot4(X[u][m].y, h1, t, false);
                    t = __builtin_amdgcn_sdot4(X[u][m].z, h2, t, false);
                    t = __builtin_amdgcn_sdot4(X[u][m].w, h3, t, false);
                    slo[m][r] = s;
                    shi[m][r] = t;
                }
            }
        }
    }

#pragma unroll
    for (int m = 0; m < MR; m++) {
        if (m >= M) break;
        const int64_t xs = wave_sum(sx[m]);
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int n = nbase + r;
            const int64_t v = (int64_t)wave_sum(slo[m][r]) + 256 * (int64_t)wave_sum(shi[m][r]) - 1920 * xs;
            if (lane == 0 && n < N) store_out<OUT>(y, (size_t)m * N + n, v, mant, shift, n);
        }
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

hipError_t launch_w12_pack(const int32_t* codes, int64_t n, int64_t k, int8_t* lo, uint8_t* nib, hipStream_t s) {
    const int64_t kp = ceil_div(k, 64) * 64, total = n * (kp / 2);
    if (total == 0) return hipSuccess;
    w12_pack_kernel<<<dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s>>>(codes, n, k, kp, lo, nib);
    return hipGetLastError();
}

template <int PX, int PW>
static hipError_t plane_gemm_px_pw(const int8_t* xa, const int8_t* wb, int64_t* y, int M, int N, int kp, int k0,
                                   int k1, int accumulate, int drop_top, hipStream_t s) {
    constexpr int NG = PX + PW - 1;
    // keep the accumulators within ~160 registers: 2x2 tiles for <= 2 groups, 1x2 for <= 5, 1x1 beyond
    constexpr int WTM = NG <= 2 ? 2 : 1;
    constexpr int WTN = NG <= 5 ? 2 : 1;
    constexpr int BM = 64 * WTM, BN = 64 * WTN;
    dim3 grid((unsigned)(ceil_div(N, BN) * ceil_div(M, BM)));
    plane_gemm_kernel<PX, PW, WTM, WTN><<<grid, dim3(256), 0, s>>>(xa, wb, y, M, N, kp, k0, k1, accumulate, drop_top);
    return hipGetLastError();
}

hipError_t launch_plane_gemm(int px, int pw, const int8_t* xa, const int8_t* wb, int64_t* y, int M, int N, int kp,
                             int k0, int k1, int accumulate, int drop_top, hipStream_t s) {
    if (M <= 0 || N <= 0 || k1 <= k0) return hipSuccess;
    if ((k0 % 64) || (k1 % 64) || k1 > kp || ceil_div(M, 64) * ceil_div(N, 64) > INT32_MAX) return hipErrorInvalidValue;
#define KT_CASE(a, b) \
    if (px == a && pw == b) return plane_gemm_px_pw<a, b>(xa, wb, y, M, N, kp, k0, k1, accumulate, drop_top, s);
    KT_CASE(1, 1) KT_CASE(1, 3) KT_CASE(1, 5) KT_CASE(3, 1) KT_CASE(3, 3) KT_CASE(3, 5) KT_CASE(5, 1) KT_CASE(5, 3)
    KT_CASE(5, 5)
#undef KT_CASE
    return hipErrorInvalidValue;
}

template <int OUT>
static hipError_t w12_linear_out(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int N, int kp,
                                 const int32_t* mant, const int32_t* shift, void* y, hipStream_t s) {
    if (M <= 8) {
        constexpr int NR = 4;
        dim3 grid((unsigned)ceil_div(N, 4 * NR));
#define KT_GEMV(mr) \
    if (M <= mr) { \
        w12_gemv_kernel<mr, NR, OUT><<<grid, dim3(256), 0, s>>>(x, lo, nib, y, M, N, kp, mant, shift); \
        return hipGetLastError(); \
    }
        KT_GEMV(1) KT_GEMV(2) KT_GEMV(4) KT_GEMV(8)
#undef KT_GEMV
    }
    if (M <= 64) {
        dim3 grid((unsigned)(ceil_div(N, 64) * ceil_div(M, 64)));
        w12_gemm_kernel<1, 1, 64, OUT><<<grid, dim3(256), 0, s>>>(x, lo, nib, y, M, N, kp, mant, shift);
        return hipGetLastError();
    }
    dim3 grid((unsigned)(ceil_div(N, 128) * ceil_div(M, 128)));
    w12_gemm_kernel<2, 2, 64, OUT><<<grid, dim3(256), 0, s>>>(x, lo, nib, y, M, N, kp, mant, shift);
    return hipGetLastError();
}

hipError_t launch_w12_linear(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int N, int kp,
                             const int32_t* mant, const int32_t* shift, int out_kind, void* y, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (kp <= 0 || (kp % 64) || ceil_div(M, 64) * ceil_div(N, 64) > INT32_MAX) return hipErrorInvalidValue;
    switch (out_kind) {
        case KT_OUT_I64: return w12_linear_out<KT_OUT_I64>(x, lo, nib, M, N, kp, mant, shift, y, s);
        case KT_OUT_I32: return w12_linear_out<KT_OUT_I32>(x, lo, nib, M, N, kp, mant, shift, y, s);
        case KT_OUT_I8: return w12_linear_out<KT_OUT_I8>(x, lo, nib, M, N, kp, mant, shift, y, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_mfma_probe(const int8_t* a, const int8_t* b, int32_t* c32, int32_t* c16, hipStream_t s) {
    mfma_probe_kernel<<<dim3(1), dim3(64), 0, s>>>(a, b, c32, c16);
    return hipGetLastError();
}

}  // namespace kt
