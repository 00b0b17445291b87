// SAM 2.1's image path on gfx950 (benchmark config 5): the patch-embed convolution as an im2col-fused W12 GEMM.
//
// The reference runs Conv2d::forward_int as a direct loop over (ic, ky, kx) per output element on the CPU
// (crates/01-engine/kt-core/src/conv.rs:68-130), output [c_out, OH, OW]. Here one CTA of 8 waves owns 128 consecutive
// output positions of one output row and 128 output channels.
//
// The weights are two int8 digit planes (code = lo + 256 hi), so the two MFMA products recombine with one shift-add
// and no row-sum term. Their k order is (ic, ky, kx) with the taps of each kernel row padded to kwp = kw rounded up
// to 4 (code 0 in the pad), so the taps of one kernel row for one output position are kwp / 4 whole dwords of an
// image row. The CTA stages the ci * kh image rows its positions read into LDS as entry codes (zero outside the
// image, the reference's skipped taps). Each row is staged as 4 / gcd(stride, 4) copies, copy c shifted by c * gcd(stride, 4) bytes, so that
// position m's taps start on a dword boundary of copy (stride * m) mod 4 / gcd(stride, 4). The MFMA A operand (16 k
// bytes per lane) is then four dwords read in place from the staged rows; no im2col tile is built. B fragments go from
// global memory straight into registers. The low-digit accumulators start at the bias; the epilogue requantizes per
// output channel and stores the tile transposed, 128 contiguous positions per channel.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kt_kernels.h"
#include "kt_w12_core.h"

namespace kt {

constexpr int CONV_BM = 128, CONV_BN = 128;
constexpr int CONV_SOP = 136;          // output tile row stride: 34 dwords put a wave's dword stores in 64 banks
constexpr int CONV_STAGE_MAX = 41472;  // bytes of staged image rows (copies x rows x row stride)
constexpr int CONV_IPT = 2;            // staging items (4 dwords of every copy of one row) per thread and pass

// The staging geometry of one launch, formed on the host.
struct PatchPlan {
    int CI, H, W, KH, S, P, OH, OW, CO, segs;
    int NR;          // image rows the taps read: CI * KH (row r = (ic, ky))
    int RMAX;        // staged rows: every row the k tiles address; rows NR.. are zero
    int LPDU;        // dwords of a staged row that the 128 positions read
    int NQ;          // staging items per row: LPDU / 4 rounded up (4 dwords each)
    int LPB;         // bytes between staged rows
    int CSB;         // bytes between copies
    int NC, GSH;     // copies per row; log2 of the phase step between copies (NC << GSH == 4)
    uint32_t m_nq;   // ceil(2^32 / NQ): it / NQ as one multiply-high for it * NQ < 2^32
    uint32_t m_kh;   // ceil(2^32 / KH)
};

// The entry codes of four pixels: lut[channel * 256 + pixel] for each byte of raw (icoff = channel << 8). Each table
// index is one byte permute (the pixel byte beside the channel byte); the four codes are joined by three more.
__device__ __forceinline__ uint32_t entry4(uint32_t raw, const int8_t* lut, uint32_t icoff) {
    uint32_t c[4];
#pragma unroll
    for (int b = 0; b < 4; b++) c[b] = (uint8_t)lut[__builtin_amdgcn_perm(icoff, raw, 0x0C0C0500u | b)];
    const uint32_t lo = __builtin_amdgcn_perm(c[1], c[0], 0x0C0C0400u), hi = __builtin_amdgcn_perm(c[3], c[2], 0x0C0C0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// The smallest |v| whose requant exceeds 127: ((a * mt + bias) >> shr) >= 128 exactly when
// a >= ceil((2^(shr + 7) - bias) / mt). 2^32 - 1 when no |v| <= 2^31 reaches it.
__device__ __forceinline__ uint32_t rq8_threshold(const ColQ& q) {
    if (q.mt == 0 || q.shr + 7 >= 64) return 0xFFFFFFFFu;  // mt = 0: bias >> shr = 0
    const uint64_t lim = (uint64_t)1 << (q.shr + 7);        // bias < 2^shr < lim
    const uint64_t t = (lim - q.bias + q.mt - 1) / q.mt;
    return t > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)t;
}

// col_requant<false>(v, q) with the clamp as one compare against rq8_threshold(q).
__device__ __forceinline__ int32_t rq8(uint32_t v, const ColQ& q, uint32_t sat) {
    const bool vneg = (int32_t)v < 0;
    const uint32_t a = vneg ? 0u - v : v;
    const uint32_t m = a >= sat ? 127u : (uint32_t)(((uint64_t)a * q.mt + q.bias) >> q.shr);
    return vneg != q.neg ? -(int32_t)m : (int32_t)m;
}

template <int KTILES, int DPR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void conv_patch_kernel(
    const uint8_t* __restrict__ img, const int8_t* __restrict__ lut, const PatchPlan p,
    const int8_t* __restrict__ wlo, const int8_t* __restrict__ whi, const int32_t* __restrict__ bias,
    const int32_t* __restrict__ mant, const int32_t* __restrict__ shift, int8_t* __restrict__ out) {
    constexpr int BM = CONV_BM, BN = CONV_BN, SOP = CONV_SOP, KB = 2 * KTILES;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    // the entry table is static LDS, so its address folds into the lookups' offset field
    __shared__ __attribute__((aligned(256))) int8_t sLut[4 * 256];  // [4][256] entry codes
    int8_t* sO = smem;                                    // [BN][SOP] output tile
    int* sCol = reinterpret_cast<int*>(smem + BN * SOP);  // [BN][8] requant constants of each column
    int8_t* sPatch = smem + BN * SOP + 32 * BN;           // [NC][RMAX] staged rows

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ct = wave & 3, rh = wave >> 2;
    const int oy = blockIdx.x / p.segs, ox0 = (blockIdx.x - oy * p.segs) * BM;
    const int n0 = blockIdx.y * BN;

    // The column constants of the epilogue, formed by the first two waves (one column per thread) from loads issued
    // before the image loads, so they are ready long before the epilogue.
    int32_t cm = 0, cs = 1, cbias = 0;
    if (tid < BN && n0 + tid < p.CO) {
        cm = mant[n0 + tid], cs = shift[n0 + tid];
        if (bias) cbias = bias[n0 + tid];
    }
    int8_t lv[2];
#pragma unroll
    for (int u = 0; u < 2; u++) lv[u] = tid + 512 * u < p.CI * 256 ? lut[tid + 512 * u] : 0;

    // Staging. Item it = (row r, quad q) writes dwords 4q .. 4q + 3 of every copy of staged row r. Raw dword t of an
    // item holds the pixels of image columns a + 4 (4q + t) .. + 3, where a = the segment's first tap column ix0
    // rounded down to a multiple of 4 when whole dwords can be loaded (W % 4 == 0; o = ix0 - a), else a = ix0 (byte
    // loads, o = 0). Copy c's dword 4q + i is bytes 4i + o + (c << GSH) .. + 3 of the item's raw dwords, so an item
    // translates each of its 5 or 6 raw dwords through the entry table once.
    const int total = p.RMAX * p.NQ;
    const bool vec = (p.W & 3) == 0;
    const int ix0 = ox0 * p.S - p.P, a = vec ? ix0 & ~3 : ix0, o = ix0 - a;
    const bool need5 = o + ((p.NC - 1) << p.GSH) > 4;  // a copy starts past raw dword 1
    // Loads go through a buffer resource over the image: a pixel outside the image (or a raw dword no copy reads) is
    // an out-of-range offset that returns 0 without a branch, so every load of a pass is in flight before the first
    // is used.
    const __amdgpu_buffer_rsrc_t rI = make_rsrc(img, (uint32_t)(p.CI * p.H * p.W));
    // item `it`: its raw dwords and flags: channel << 24 | which pixels lie in the image (whole dwords: bit t for raw
    // dword t; byte loads: bits 4t .. 4t + 3 for its bytes)
    auto load_item = [&](int it, uint32_t (&raw)[6], int& flags, auto vec_tag) {
        constexpr bool VEC = decltype(vec_tag)::value;
        const int r = (int)__umulhi((uint32_t)it, p.m_nq), d = 4 * (it - r * p.NQ);
        const int ic = (int)__umulhi((uint32_t)r, p.m_kh), iy = oy * p.S - p.P + (r - ic * p.KH);
        // bitwise, not short-circuit: the offsets below become selects, the loads stay unconditional
        const bool row_ok = (it < total) & (r < p.NR) & ((unsigned)iy < (unsigned)p.H);
        const int rowoff = (ic * p.H + iy) * p.W;
        int vm = (row_ok ? ic : 0) << 24;
#pragma unroll
        for (int t = 0; t < 6; t++) {
            const bool used = row_ok & (t < 5 || need5);
            const int col = a + 4 * (d + t);
            if constexpr (VEC) {
                const bool ok = used & ((unsigned)col < (unsigned)p.W);
                raw[t] = __builtin_amdgcn_raw_buffer_load_b32(rI, ok ? rowoff + col : (int)KT_OOB, 0, 0);
                vm |= ok ? 1 << t : 0;
            } else {
                raw[t] = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const bool ok = used & ((unsigned)(col + b) < (unsigned)p.W);
                    raw[t] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rI, ok ? rowoff + col + b : (int)KT_OOB,
                                                                             0, 0) << (8 * b);
                    vm |= ok ? 1 << (4 * t + b) : 0;
                }
            }
        }
        flags = vm;
    };
    // the item's entry codes into dwords 4q .. 4q + 3 of every copy of row r (one 16-byte store per copy)
    auto store_item = [&](int it, const uint32_t (&raw)[6], int flags, auto vec_tag) {
        constexpr bool VEC = decltype(vec_tag)::value;
        const int r = (int)__umulhi((uint32_t)it, p.m_nq), d = 4 * (it - r * p.NQ);
        uint32_t T[6] = {0, 0, 0, 0, 0, 0};
        if (flags & 0xFFFFFF) {  // some pixel of the item lies in the image
            const uint32_t icoff = (uint32_t)(flags >> 24) << 8;
#pragma unroll
            for (int t = 0; t < 6; t++) {
                if (t == 5 && !need5) continue;
                const uint32_t e = entry4(raw[t], sLut, icoff);
                if constexpr (VEC) {
                    T[t] = (flags >> t) & 1 ? e : 0u;
                } else {
                    uint32_t m = 0;  // the bytes that lie in the image
#pragma unroll
                    for (int b = 0; b < 4; b++) m |= (flags >> (4 * t + b)) & 1 ? 0xFFu << (8 * b) : 0u;
                    T[t] = e & m;
                }
            }
        }
        int8_t* dst = sPatch + r * p.LPB + 4 * d;
        {
            const int sh = o;  // copy 0 starts inside raw dword 0
            *reinterpret_cast<v4i*>(dst) = v4i{(int)__builtin_amdgcn_alignbyte(T[1], T[0], sh),
                                               (int)__builtin_amdgcn_alignbyte(T[2], T[1], sh),
                                               (int)__builtin_amdgcn_alignbyte(T[3], T[2], sh),
                                               (int)__builtin_amdgcn_alignbyte(T[4], T[3], sh)};
        }
        for (int c = 1; c < p.NC; c++) {
            const int sh = o + (c << p.GSH);
            const bool up = sh >= 4;
            uint32_t U[5];
#pragma unroll
            for (int t = 0; t < 5; t++) U[t] = up ? T[t + 1] : T[t];
            *reinterpret_cast<v4i*>(dst + c * p.CSB) = v4i{(int)__builtin_amdgcn_alignbyte(U[1], U[0], sh & 3),
                                                           (int)__builtin_amdgcn_alignbyte(U[2], U[1], sh & 3),
                                                           (int)__builtin_amdgcn_alignbyte(U[3], U[2], sh & 3),
                                                           (int)__builtin_amdgcn_alignbyte(U[4], U[3], sh & 3)};
        }
    };
    auto put_tables = [&]() {
#pragma unroll
        for (int u = 0; u < 2; u++)
            if (tid + 512 * u < p.CI * 256) sLut[tid + 512 * u] = lv[u];
        if (tid < BN) {
            const ColQ8 q8 = col_q8(cm, cs);
            const ColQ& q = q8.q;
            const uint64_t mb = (uint64_t)__double_as_longlong(q8.ms);
            *reinterpret_cast<v4i*>(sCol + 8 * tid) =
                v4i{(int)q.mt, (int)q8.hsb, cbias, (int)(q.shr | (q.neg ? 256u : 0u) | (q8.fp ? 512u : 0u))};
            *reinterpret_cast<v4i*>(sCol + 8 * tid + 4) =
                v4i{(int)(uint32_t)q.bias, (int)(uint32_t)(q.bias >> 32), (int)(uint32_t)mb, (int)(uint32_t)(mb >> 32)};
        }
        __syncthreads();  // the entry table is in LDS
    };
    if (vec) {  // whole dwords: every load of a pass in flight before the first use
        auto pass = [&](int base, bool first) {
            uint32_t raw[CONV_IPT][6];
            int flags[CONV_IPT];
#pragma unroll
            for (int q = 0; q < CONV_IPT; q++)
                load_item(base + q * 512 + tid, raw[q], flags[q], std::integral_constant<bool, true>{});
            if (first) {
                // the tables' work waits for the column loads: keep it behind the image loads
                __builtin_amdgcn_sched_barrier(0);
                put_tables();
            }
#pragma unroll
            for (int q = 0; q < CONV_IPT; q++)
                if (base + q * 512 + tid < total)
                    store_item(base + q * 512 + tid, raw[q], flags[q], std::integral_constant<bool, true>{});
        };
        pass(0, true);  // peeled, so that the tables' work is not hoisted above the loads
        for (int base = 512 * CONV_IPT; base < total; base += 512 * CONV_IPT) pass(base, false);
    } else {  // byte loads (rows not dword aligned), one item at a time
        put_tables();
        for (int it = tid; it < total; it += 512) {
            uint32_t raw[6];
            int flags;
            load_item(it, raw, flags, std::integral_constant<bool, false>{});
            store_item(it, raw, flags, std::integral_constant<bool, false>{});
        }
    }
    // B fragments of the whole k range (wave column tile ct), issued once the staging registers are free; the
    // weights are shared by every CTA, so these mostly hit L2 while the last waves finish staging
    const int cb0 = n0 / 32, ncb = min((p.CO - n0 + 31) / 32, BN / 32);
    const __amdgpu_buffer_rsrc_t rL = make_rsrc(wlo + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    const __amdgpu_buffer_rsrc_t rH = make_rsrc(whi + (size_t)cb0 * KB * 1024, (uint32_t)ncb * KB * 1024);
    constexpr int BW = KB < 4 ? KB : 4;  // 32-k blocks of B in flight: block kb + BW is loaded as kb is consumed
    v4i bl[KB], bh[KB];
    auto load_b = [&](int kb) {
        bl[kb] = bload16(rL, (uint32_t)(ct * KB) * 1024 + 16 * lane, kb * 1024u);
        bh[kb] = bload16(rH, (uint32_t)(ct * KB) * 1024 + 16 * lane, kb * 1024u);
    };
#pragma unroll
    for (int kb = 0; kb < BW; kb++) load_b(kb);
    __syncthreads();  // the staged rows are complete

    // MFMA over the staged rows: wave (ct, rh) owns columns 32 ct.. and the i-tiles 2 rh, 2 rh + 1 (32 positions
    // each). Lane (j, h) reads for position m = 32 i + j the k dwords g = 8 kb + 4 h + (0..3): dword g % DPR of
    // kernel row g / DPR.
    const int j = lane & 31, h = lane >> 5;
    int mb[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int sm = p.S * ((2 * rh + i) * 32 + j);
        mb[i] = ((sm & 3) >> p.GSH) * p.CSB + (sm >> 2) * 4;
    }
    // the low-digit accumulators start at the column's bias (accumulator units), so it needs no add per value
    const int cb = sCol[8 * (ct * 32 + j) + 2];
    v16i acc0[2], acc1[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) acc0[i][r] = cb;
        acc1[i] = v16i{};
    }
    // The first half of the waves issues its MFMAs first, so its epilogue (VALU) overlaps the other half's MFMAs.
    if (rh == 0) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            v4i av;
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                int off;
                if constexpr (4 % DPR == 0) {
                    constexpr int RPH = 4 / DPR;  // kernel rows per 16-byte chunk
                    off = ((8 * kb + ii) / DPR + RPH * h) * p.LPB + 4 * ((8 * kb + ii) % DPR);
                } else {
                    const int g = 8 * kb + 4 * h + ii;
                    off = (g / DPR) * p.LPB + 4 * (g % DPR);
                }
                av[ii] = *reinterpret_cast<const int*>(sPatch + mb[i] + off);
            }
            acc0[i] = mfma32(av, bl[kb], acc0[i]);
            acc1[i] = mfma32(av, bh[kb], acc1[i]);
        }
        if (kb + BW < KB) load_b(kb + BW);
    }
    if (rh == 0) __builtin_amdgcn_s_setprio(0);

    {
        const int c = ct * 32 + j;
        const v4i k4 = *reinterpret_cast<const v4i*>(sCol + 8 * c);
        const v4i k8 = *reinterpret_cast<const v4i*>(sCol + 8 * c + 4);
        ColQ q;
        q.mt = (uint32_t)k4.x, q.shr = (uint32_t)k4.w & 255u, q.neg = (k4.w >> 8) & 1;
        q.bias = (uint64_t)(uint32_t)k8.x | (uint64_t)(uint32_t)k8.y << 32;
        const uint32_t hsb = (uint32_t)k4.y;
        const double ms = __longlong_as_double((long long)((uint64_t)(uint32_t)k8.z | (uint64_t)(uint32_t)k8.w << 32));
        // four codes (each in [-127, 127]) into the bytes of one dword, three byte permutes
        auto pack4 = [](const int (&y)[4]) {
            const uint32_t lo = __builtin_amdgcn_perm((uint32_t)y[1], (uint32_t)y[0], 0x0C0C0400u);
            const uint32_t hi = __builtin_amdgcn_perm((uint32_t)y[3], (uint32_t)y[2], 0x0C0C0400u);
            return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        };
        const bool all_fp = __all((k4.w >> 9) & 1);
        // the clamp threshold of the integer path, needed only when a column of the wave is off the double path
        const uint32_t sat = all_fp ? 0u : rq8_threshold(q);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int m0 = (2 * rh + i) * 32 + 8 * g4 + 4 * h;
                int v[4], y[4];
#pragma unroll
                for (int e = 0; e < 4; e++)  // bias + s_lo + 256 s_hi, formed modulo 2^32 (the value fits int32)
                    v[e] = (int)((uint32_t)acc0[i][4 * g4 + e] + ((uint32_t)acc1[i][4 * g4 + e] << 8));
                if (all_fp) {
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = rq8_fp(v[e], ms, hsb);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = rq8((uint32_t)v[e], q, sat);
                }
                const uint32_t packed = pack4(y);
                *reinterpret_cast<uint32_t*>(sO + c * SOP + m0) = packed;
            }
    }
    __syncthreads();
    const bool full = ox0 + BM <= p.OW && (p.OW & 15) == 0 && ((uintptr_t)out & 15) == 0;
    for (int idx = tid; idx < BN * BM / 16; idx += 512) {
        const int c = idx >> 3, m = (idx & 7) * 16, n = n0 + c;
        if (n >= p.CO) continue;
        const v2i lo = *reinterpret_cast<const v2i*>(sO + c * SOP + m);
        const v2i hi = *reinterpret_cast<const v2i*>(sO + c * SOP + m + 8);
        int8_t* dst = out + ((size_t)n * p.OH + oy) * p.OW + ox0 + m;
        if (full) {
            *reinterpret_cast<v4i*>(dst) = v4i{lo.x, lo.y, hi.x, hi.y};
        } else {
            const v4i v{lo.x, lo.y, hi.x, hi.y};
            const int8_t* bb = reinterpret_cast<const int8_t*>(&v);
            for (int t = 0; t < 16 && ox0 + m + t < p.OW; t++) dst[t] = bb[t];
        }
    }
}

template <int KTILES, int DPR>
static hipError_t launch_conv_t(dim3 grid, size_t lds, hipStream_t s, const uint8_t* img, const int8_t* lut,
                                const PatchPlan& p, const int8_t* wlo, const int8_t* whi, const int32_t* bias,
                                const int32_t* mant, const int32_t* shift, int8_t* out) {
    conv_patch_kernel<KTILES, DPR><<<grid, dim3(512), lds, s>>>(img, lut, p, wlo, whi, bias, mant, shift, out);
    return hipGetLastError();
}

template <int KTILES>
static hipError_t launch_conv_k(int dpr, dim3 grid, size_t lds, hipStream_t s, const uint8_t* img, const int8_t* lut,
                                const PatchPlan& p, const int8_t* wlo, const int8_t* whi, const int32_t* bias,
                                const int32_t* mant, const int32_t* shift, int8_t* out) {
    switch (dpr) {
        case 1: return launch_conv_t<KTILES, 1>(grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
        case 2: return launch_conv_t<KTILES, 2>(grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
        case 3: return launch_conv_t<KTILES, 3>(grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
        default: return launch_conv_t<KTILES, 4>(grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
    }
}

// Patch-embed weights -> two int8 digit planes. One thread per fragment lane (column 32 nb + (l & 31), k = 32 kb +
// 16 (l >> 5) .. + 15 of the padded order (ic, ky, kx < kwp)): code = lo + 256 hi with hi = floor((code + 128) / 256)
// in [-8, 8] and lo in [-128, 127]; pad taps, padding rows and padding k are code 0.
__global__ void conv_pack_kernel(const int32_t* __restrict__ codes, int co, int kh, int kw, int kwp, int kk, int kp,
                                 int8_t* __restrict__ lo, int8_t* __restrict__ hi) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int KB = kp / 32, total = (co + 31) / 32 * KB * 64;
    if (idx >= total) return;
    const int frag = idx >> 6, l = idx & 63, nb = frag / KB, kb = frag - nb * KB;
    const int n = nb * 32 + (l & 31), c0 = kb * 32 + 16 * (l >> 5);
    const int rowk = kk / kwp * kw;  // codes per output channel: ci * kh * kw
    uint32_t lw[4] = {0, 0, 0, 0}, hw[4] = {0, 0, 0, 0};
    for (int t = 0; t < 16; t++) {
        const int c = c0 + t, run = c / kwp, tx = c - run * kwp;
        const int32_t v = n < co && c < kk && tx < kw ? codes[(size_t)n * rowk + run * kw + tx] : 0;
        const int32_t h = (v + 128) >> 8;  // arithmetic: floor
        lw[t >> 2] |= ((uint32_t)(v - 256 * h) & 255u) << (8 * (t & 3));
        hw[t >> 2] |= ((uint32_t)h & 255u) << (8 * (t & 3));
    }
    *reinterpret_cast<v4i*>(lo + (size_t)idx * 16) = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
    *reinterpret_cast<v4i*>(hi + (size_t)idx * 16) = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
}

hipError_t launch_conv_pack(const int32_t* codes, int co, int ci, int kh, int kw, int8_t* lo, int8_t* hi,
                            hipStream_t s) {
    const int kwp = conv_patch_kwp(kw);
    if (co < 1 || ci < 1 || ci > 4 || kh < 1 || kh > 256 || kwp == 0) return hipErrorInvalidValue;
    const int kk = ci * kh * kwp, kp = (kk + 63) / 64 * 64;
    const int64_t total = (int64_t)(co + 31) / 32 * (kp / 32) * 64;
    if (total > INT32_MAX) return hipErrorInvalidValue;
    conv_pack_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s>>>(codes, co, kh, kw, kwp, kk, kp, lo,
                                                                                 hi);
    return hipGetLastError();
}

// The smallest x >= lo with x % mod == want % mod.
static int64_t round_to_residue(int64_t lo, int64_t mod, int64_t want) {
    return lo + (((want - lo) % mod) + mod) % mod;
}

hipError_t launch_conv_patch(const uint8_t* img, const int8_t* lut, int CI, int H, int W, int KH, int KW, int S, int P,
                             const int8_t* wlo, const int8_t* whi, int CO, const int32_t* bias, const int32_t* mant,
                             const int32_t* shift, int8_t* out, hipStream_t s) {
    const int kwp = conv_patch_kwp(KW);
    if (CI < 1 || CI > 4 || KH < 1 || kwp == 0 || S < 1 || S > 256 || P < 0 || H + 2 * P < KH ||
        W + 2 * P < KW || CO < 1)
        return hipErrorInvalidValue;
    const int64_t KK = (int64_t)CI * KH * kwp;
    if (KK > 256) return hipErrorInvalidValue;
    const int KP = (int)((KK + 63) / 64 * 64), DPR = kwp / 4;
    PatchPlan p;
    p.CI = CI, p.H = H, p.W = W, p.KH = KH, p.S = S, p.P = P, p.CO = CO;
    p.OH = (H + 2 * P - KH) / S + 1, p.OW = (W + 2 * P - KW) / S + 1;
    p.segs = (p.OW + CONV_BM - 1) / CONV_BM;
    if ((int64_t)p.OH * p.segs > INT32_MAX || (int64_t)CI * H * W > INT32_MAX) return hipErrorInvalidValue;
    p.NR = CI * KH;
    p.RMAX = (KP + kwp - 1) / kwp;
    p.LPDU = S * (CONV_BM - 1) / 4 + DPR;
    p.NQ = (p.LPDU + 3) / 4;
    const int g = S % 4 == 0 ? 4 : S % 2 == 0 ? 2 : 1;
    p.NC = 4 / g, p.GSH = g == 4 ? 2 : g == 2 ? 1 : 0;
    // Bank spreading: the two lane halves of an A read are 4 / DPR rows apart and should land 32 banks apart; the
    // copies of consecutive positions (stride not a multiple of 4) 32 / NC banks apart.
    int64_t lpd = 4 * p.NQ;  // the items write whole quads
    if (DPR == 1) lpd = round_to_residue(lpd, 16, 8);
    else if (DPR == 2) lpd = round_to_residue(lpd, 32, 16);
    else if (DPR == 4) lpd = round_to_residue(lpd, 64, 32);
    int64_t csd = (int64_t)p.RMAX * lpd;
    if (p.NC > 1) csd = round_to_residue(csd, 64, 32 / p.NC);
    if (4 * csd * p.NC > CONV_STAGE_MAX) return hipErrorInvalidValue;
    p.LPB = (int)(4 * lpd), p.CSB = (int)(4 * csd);
    p.m_nq = (uint32_t)(0xFFFFFFFFull / (uint32_t)p.NQ + 1);
    p.m_kh = (uint32_t)(0xFFFFFFFFull / (uint32_t)KH + 1);
    const size_t lds = (size_t)CONV_BN * CONV_SOP + 32 * CONV_BN + (size_t)p.CSB * p.NC;  // + 1 KiB static
    dim3 grid((unsigned)(p.OH * p.segs), (unsigned)((CO + CONV_BN - 1) / CONV_BN));
    switch (KP / 64) {
        case 1: return launch_conv_k<1>(DPR, grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
        case 2: return launch_conv_k<2>(DPR, grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
        case 3: return launch_conv_k<3>(DPR, grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
        default: return launch_conv_k<4>(DPR, grid, lds, s, img, lut, p, wlo, whi, bias, mant, shift, out);
    }
}

}  // namespace kt
