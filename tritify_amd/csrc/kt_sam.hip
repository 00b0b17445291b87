// SAM 2.1's image path on gfx950: the patch-embed convolution as an im2col-fused W12 GEMM.
//
// The reference runs Conv2d::forward_int as a direct loop over (ic, ky, kx) per output element on the CPU
// (crates/01-engine/kt-core/src/conv.rs:68-130), output [c_out, OH, OW]. Here one CTA owns 128 consecutive output
// positions of one output row and 128 output channels: it stages the image rows those positions read (u8 pixels
// through the per-channel entry code table, zero outside the image -- the reference's skipped taps) into LDS, builds
// the im2col A tile [128 positions][k = (ic, ky, kx)] from that patch in the MFMA operand layout, multiplies it
// against the W12 weights (B fragments straight from global memory into registers), adds the bias in accumulator
// units, requantizes per output channel and stores the tile transposed, 128 contiguous positions per channel.
// k = ci * kh * kw <= 256, so the whole reduction is at most four 64-wide k tiles held in LDS at once.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kt_kernels.h"
#include "kt_w12_core.h"

namespace kt {

constexpr int CONV_PATCH_MAX = 16384;  // bytes of the staged image rows (ci * kh * (stride * 127 + kw))

template <int KTILES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_patch_kernel(const uint8_t* __restrict__ img, const int8_t* __restrict__ lut,
                                                         int CI, int H, int W, int KH, int KW, int S, int P, int OH,
                                                         int OW, const int8_t* __restrict__ wlo,
                                                         const uint8_t* __restrict__ wnib, int CO,
                                                         const int32_t* __restrict__ bias,
                                                         const int32_t* __restrict__ mant,
                                                         const int32_t* __restrict__ shift, int8_t* __restrict__ out) {
    constexpr int BM = 128, BN = 128, KP = 64 * KTILES, KB = KP / 32, CPT = 2 * KTILES;  // chunks per thread
    constexpr int NTILE = KTILES < 3 ? 3 : KTILES;
    constexpr int SOP = BM + 16;  // output tile row stride: rows 144 bytes apart spread the byte stores over banks
    static_assert(NTILE * BM * 64 >= BN * SOP, "the output tile reuses the A tiles");
    __shared__ __attribute__((aligned(16))) int8_t sA[NTILE][BM * 64];
    __shared__ int8_t sPatch[CONV_PATCH_MAX];
    __shared__ int8_t sLut[4 * 256];
    __shared__ int sKoff[KP];
    __shared__ int sRow[BM];

    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, wave = tid >> 6;
    const int segs = (OW + BM - 1) / BM, oy = blockIdx.x / segs, ox0 = (blockIdx.x - oy * segs) * BM;
    const int n0 = blockIdx.y * BN;
    const int KK = CI * KH * KW, L = S * (BM - 1) + KW, ix0 = ox0 * S - P;

    // B fragments of the whole k range, issued first so they land while the patch is staged
    const int cb0 = n0 / 32, ncb = (CO - n0 + 31) / 32 < BN / 32 ? (CO - n0 + 31) / 32 : BN / 32;
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    const __amdgpu_buffer_rsrc_t rN = make_rsrc(wnib + (size_t)cb0 * KB * 512, (uint32_t)ncb * KB * 512);
    v4i bl[KTILES][2];
    v2i bn[KTILES][2];
#pragma unroll
    for (int t = 0; t < KTILES; t++)
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            bl[t][ks] = bload16(rL, (uint32_t)(wave * KB) * 1024 + 16 * lane, (2 * t + ks) * 1024u);
            bn[t][ks] = bload8(rN, (uint32_t)(wave * KB) * 512 + 8 * lane, (2 * t + ks) * 512u);
        }

    for (int i = tid; i < CI * 256; i += 256) sLut[i] = lut[i];
    // The staged rows cover image columns from a = ix0 rounded down to a multiple of 4 (dword loads when W % 4 == 0),
    // so patch column j of the segment sits at byte o + j of its LDS row (row stride LP bytes).
    const bool vec = (W & 3) == 0;
    const int a = vec ? ix0 & ~3 : ix0, o = ix0 - a, ND = (L + o + 3) >> 2, LP = vec ? 4 * ND : L;
    for (int kk = tid; kk < KP; kk += 256) {
        if (kk < KK) {
            const int ic = kk / (KH * KW), r = kk - ic * KH * KW, ky = r / KW, kx = r - ky * KW;
            sKoff[kk] = (ic * KH + ky) * LP + kx + o;
        } else {
            sKoff[kk] = -1;
        }
    }
    // the image rows of this output row segment, as entry codes (zero outside the image), every load of a pass in
    // flight before the first use
    constexpr int RB = 24;
    const int nrows = CI * KH;
    if (vec) {  // thread d < ND: dword d of every row (4 pixels, inside or outside the image together)
        const int col = a + 4 * tid;
        const bool col_in = tid < ND && col >= 0 && col < W;
        for (int r0 = 0; r0 < nrows; r0 += RB) {
            int v[RB];
            int ic = r0 / KH, ky = r0 - ic * KH;  // of row r0 + rr, advanced without divisions
            int ics[RB];
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                const int iy = oy * S - P + ky;
                const bool in = r0 + rr < nrows && col_in && iy >= 0 && iy < H;
                v[rr] = in ? *reinterpret_cast<const int*>(img + ((size_t)ic * H + iy) * W + col) : 0;
                ics[rr] = in ? ic : -1;
                if (++ky == KH) ky = 0, ic++;
            }
            if (r0 == 0) __syncthreads();  // the entry table is in LDS
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                if (r0 + rr >= nrows || tid >= ND) continue;
                int q = 0;
                if (ics[rr] >= 0) {
                    const int8_t* lt = sLut + ics[rr] * 256;
#pragma unroll
                    for (int b = 0; b < 4; b++) q |= ((int)(uint8_t)lt[(v[rr] >> (8 * b)) & 255]) << (8 * b);
                }
                *reinterpret_cast<int*>(sPatch + (r0 + rr) * LP + 4 * tid) = q;
            }
        }
    } else {  // byte loads, one byte per thread and row per pass
        bool first = true;
        for (int j = tid; j - tid < L; j += 256) {
            const int ix = ix0 + j;
            const bool col_in = j < L && ix >= 0 && ix < W;
            for (int r0 = 0; r0 < nrows; r0 += RB) {
                int v[RB];
                int ic = r0 / KH, ky = r0 - ic * KH;
#pragma unroll
                for (int rr = 0; rr < RB; rr++) {
                    const int iy = oy * S - P + ky;
                    // a pixel, plus 256 x its channel for the table lookup; -1 for a tap outside the image
                    v[rr] = r0 + rr < nrows && col_in && iy >= 0 && iy < H
                                ? (int)img[((size_t)ic * H + iy) * W + ix] + 256 * ic
                                : -1;
                    if (++ky == KH) ky = 0, ic++;
                }
                if (first) __syncthreads();  // the entry table is in LDS
                first = false;
#pragma unroll
                for (int rr = 0; rr < RB; rr++) {
                    const int row = r0 + rr;
                    if (row < nrows && j < L) sPatch[row * LP + j] = v[rr] >= 0 ? sLut[v[rr]] : 0;
                }
            }
        }
        if (first) __syncthreads();
    }
    __syncthreads();
    // im2col: thread (row m = tid / 2) builds CPT 16-byte chunks of its row and their sum
    {
        const int m = tid >> 1, c0 = (tid & 1) * CPT;
        int s = 0;
#pragma unroll
        for (int c = 0; c < CPT; c++) {
            const int cc = c0 + c;
            v4i v;
            int8_t* b = reinterpret_cast<int8_t*>(&v);
#pragma unroll
            for (int t = 0; t < 16; t++) {
                const int ko = sKoff[16 * cc + t];
                b[t] = ko >= 0 ? sPatch[ko + S * m] : 0;
            }
            s += sum4(v);
            lds_write16(sA[cc >> 2], lds_off<4>(m, cc & 3), v);
        }
        s += __shfl_xor(s, 1);
        if ((tid & 1) == 0) sRow[m] = s;
    }
    __syncthreads();

    v16i acc0[4], acc1[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc0[i] = acc1[i] = v16i{};
#pragma unroll
    for (int t = 0; t < KTILES; t++)
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const v4i b0 = bl[t][ks], b1 = unpack_hi(bn[t][ks]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v4i a = lds_read16(sA[t], lds_off<4>(i * 32 + (lane & 31), 2 * ks + half));
                acc0[i] = mfma32(a, b0, acc0[i]);
                acc1[i] = mfma32(a, b1, acc1[i]);
            }
        }
    __syncthreads();  // every wave is done with sA: it becomes the output tile [BN][BM]

    int8_t* sO = &sA[0][0];
    {
        const int c = wave * 32 + (lane & 31), n = n0 + c;
        const ColQ q = col_q(n < CO ? mant[n] : 0, n < CO ? shift[n] : 1);
        const int b = n < CO && bias ? bias[n] : 0;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                const int v = w12_value(acc0[i][r], acc1[i][r], -1920 * sRow[m]) + b;
                sO[c * SOP + m] = (int8_t)col_requant<false>(v, q);
            }
    }
    __syncthreads();
    const bool full = ox0 + BM <= OW && (OW & 15) == 0;
    for (int idx = tid; idx < BN * BM / 16; idx += 256) {
        const int c = idx / (BM / 16), m = (idx - c * (BM / 16)) * 16, n = n0 + c;
        if (n >= CO) continue;
        const v4i v = *reinterpret_cast<const v4i*>(sO + c * SOP + m);
        int8_t* dst = out + ((size_t)n * OH + oy) * OW + ox0 + m;
        if (full) {
            *reinterpret_cast<v4i*>(dst) = v;
        } else {
            const int8_t* bb = reinterpret_cast<const int8_t*>(&v);
            for (int t = 0; t < 16 && ox0 + m + t < OW; t++) dst[t] = bb[t];
        }
    }
}

hipError_t launch_conv_patch(const uint8_t* img, const int8_t* lut, int CI, int H, int W, int KH, int KW, int S, int P,
                             const int8_t* wlo, const uint8_t* wnib, int CO, const int32_t* bias, const int32_t* mant,
                             const int32_t* shift, int8_t* out, hipStream_t s) {
    if (CI < 1 || CI > 4 || KH < 1 || KW < 1 || S < 1 || P < 0 || H + 2 * P < KH || W + 2 * P < KW || CO < 1)
        return hipErrorInvalidValue;
    const int KK = CI * KH * KW;
    // staged rows: L = S * 127 + KW bytes, plus up to 6 of dword alignment, at most 1024 (one dword per thread)
    const int64_t Lrow = (int64_t)S * 127 + KW + 6;
    if (KK > 256 || Lrow > 1024 || (int64_t)CI * KH * Lrow > CONV_PATCH_MAX) return hipErrorInvalidValue;
    const int OH = (H + 2 * P - KH) / S + 1, OW = (W + 2 * P - KW) / S + 1;
    const int64_t segs = (OW + 127) / 128;
    if ((int64_t)OH * segs > INT32_MAX || (int64_t)CI * H * W > INT32_MAX) return hipErrorInvalidValue;
    dim3 grid((unsigned)(OH * segs), (unsigned)((CO + 127) / 128));
    const int kt = (KK + 63) / 64;
    if (kt == 1)
        conv_patch_kernel<1><<<grid, dim3(256), 0, s>>>(img, lut, CI, H, W, KH, KW, S, P, OH, OW, wlo, wnib, CO, bias,
                                                        mant, shift, out);
    else if (kt == 2)
        conv_patch_kernel<2><<<grid, dim3(256), 0, s>>>(img, lut, CI, H, W, KH, KW, S, P, OH, OW, wlo, wnib, CO, bias,
                                                        mant, shift, out);
    else if (kt == 3)
        conv_patch_kernel<3><<<grid, dim3(256), 0, s>>>(img, lut, CI, H, W, KH, KW, S, P, OH, OW, wlo, wnib, CO, bias,
                                                        mant, shift, out);
    else
        conv_patch_kernel<4><<<grid, dim3(256), 0, s>>>(img, lut, CI, H, W, KH, KW, S, P, OH, OW, wlo, wnib, CO, bias,
                                                        mant, shift, out);
    return hipGetLastError();
}

}  // namespace kt
