// Internal launch interface between the host library (kt_hip.cpp) and the gfx950 kernels (kt_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kt_hip.h"

namespace kt {

hipError_t launch_pack_planes(const int32_t* codes, int64_t rows, int64_t k, int p, int wrong_carry, int8_t* out,
                              hipStream_t s);
hipError_t launch_w12_pack(const int32_t* codes, int64_t n, int64_t k, int64_t ilv, int8_t* lo, uint8_t* nib,
                           hipStream_t s);
struct QlState;
struct QlSeg;
// ql: one state, or (seg non-null) seg->n states, one per output segment (each CTA's columns in one segment).
hipError_t launch_plane_gemm(int px, int pw, const int8_t* xa, const int8_t* wb, int64_t* y, int M, int N, int kp,
                             int k0, int k1, int accumulate, int drop_top, hipStream_t s,
                             const int64_t* ql_bias = nullptr, QlState* ql = nullptr, int splits = 1,
                             unsigned* tile_cnt = nullptr, const QlSeg* seg = nullptr);
// The output columns each CTA of launch_plane_gemm covers (segment boundaries must be multiples of it).
int plane_gemm_cta_cols(int px, int pw, int M, int N);
// How many runs of k the digit-plane GEMM of [k0, k1) splits into (1 unless its tiles leave CUs idle); a split
// launch needs y zeroed, one zeroed counter per tile (the grid's tiles: at most 128) and accumulate = 0.
int plane_gemm_splits(int px, int pw, int M, int N, int k0, int k1);
hipError_t launch_w12b_pack(const int32_t* codes, int64_t n, int64_t k, int8_t* lo, int8_t* hi, hipStream_t s);
hipError_t launch_stream_read(const uint8_t* src, uint32_t bytes, uint32_t* out, hipStream_t s);
hipError_t launch_w12b_linear(const int8_t* x, const int8_t* lo, const int8_t* hi, int M, int N, int kp,
                              const int32_t* mant, const int32_t* shift, int out_kind, void* y, hipStream_t s);
hipError_t launch_w12_linear(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int N, int kp,
                             const int32_t* mant, const int32_t* shift, const int8_t* lut, int out_kind, void* y,
                             hipStream_t s);
hipError_t launch_moe_route(const int32_t* logits, int T, int E, int top_k, const int16_t* sig, int32_t* sel,
                            int32_t* cw, hipStream_t s);
hipError_t launch_moe_bucket(const int32_t* sel, int T, int E, int top_k, int32_t* list, int32_t* pos,
                             int32_t* count, hipStream_t s);
hipError_t launch_w12_grouped(const int8_t* x, size_t x_bytes, const int32_t* list, int list_stride,
                              const int32_t* count, int groups, int64_t max_rows, const int8_t* wlo,
                              const uint8_t* wnib, size_t glo, int N, int kp, const int32_t* mant,
                              const int32_t* shift, int epi, const int16_t* silu, int h_shift, int8_t* y,
                              int ystride, int32_t* off_out, hipStream_t s);
hipError_t launch_moe_combine(const int8_t* d, const int32_t* off, const int32_t* sel, const int32_t* cw,
                              const int32_t* pos, int T, int H, int E, int top_k, int out_shift, int8_t* out,
                              hipStream_t s);
// The tap-padded width of a patch-embed kernel row (the weights' k order is (ic, ky, kx < kwp)); 0 if kw > 16.
inline int conv_patch_kwp(int64_t kw) { return kw >= 1 && kw <= 16 ? (int)((kw + 3) & ~3) : 0; }
// Patch-embed weights: co x (ci * kh * kw) codes -> two int8 digit planes (lo, hi; code = lo + 256 hi), each
// co rounded up to 32 by k = ci * kh * kwp rounded up to 64 bytes, in the W12 fragment tiling.
hipError_t launch_conv_pack(const int32_t* codes, int co, int ci, int kh, int kw, int8_t* lo, int8_t* hi,
                            hipStream_t s);
hipError_t launch_conv_patch(const uint8_t* img, const int8_t* lut, int CI, int H, int W, int KH, int KW, int S, int P,
                             const int8_t* wlo, const int8_t* whi, int CO, const int32_t* bias, const int32_t* mant,
                             const int32_t* shift, int8_t* out, hipStream_t s);
hipError_t launch_dec_embed(const int32_t* tokens, int T, const int16_t* emb, int d, int32_t* r, hipStream_t s);
hipError_t launch_dec_rmsnorm(const int32_t* r, int T, int d, int8_t* q, int qs, hipStream_t s);
hipError_t launch_dec_rope_kv(int8_t* qkv, int T, int nqkv, const int32_t* pos, int nh, int nkv, int hd,
                              const int16_t* cosT, const int16_t* sinT, int8_t* kc, int8_t* vc, hipStream_t s);
hipError_t launch_dec_attention(const int8_t* qkv, int T, int nqkv, const int32_t* pos, const int8_t* kc,
                                const int8_t* vc, int nh, int nkv, const int32_t* exp_tab, int8_t* o, int max_pos,
                                hipStream_t s);
hipError_t launch_dec_argmax(const int32_t* logits, int n, int32_t* token, int32_t* record, int32_t* step,
                             hipStream_t s);
hipError_t launch_dec_advance(int32_t* pos, int by, hipStream_t s);
hipError_t launch_dec_attention_step(const int8_t* qkv, const int32_t* pos, int8_t* kc, int8_t* vc, int nh, int nkv,
                                     const int16_t* cosT, const int16_t* sinT, const int32_t* exp_tab, int8_t* o,
                                     int max_pos, hipStream_t s);
hipError_t launch_dec_attention_o_step(const int8_t* qkv, const int32_t* pos, int8_t* kc, int8_t* vc, int nh,
                                       int nkv, const int16_t* cosT, const int16_t* sinT, const int32_t* exp_tab,
                                       int max_pos, const int8_t* wo_lo, const uint8_t* wo_nib, int d, int32_t* acc,
                                       hipStream_t s);
hipError_t launch_w12_swiglu_norm_o(const int32_t* r, int d, const int8_t* lo, const uint8_t* nib, int F,
                                    const int32_t* mant, const int32_t* shift, const int16_t* silu, int h_shift,
                                    int8_t* y, const int32_t* oacc, const int32_t* omant, const int32_t* oshift,
                                    hipStream_t s);
hipError_t launch_w12_linear_add_o(const int8_t* x, const int8_t* lo, const uint8_t* nib, int N, int kp,
                                   const int32_t* mant, const int32_t* shift, int32_t* y, int32_t* oacc,
                                   const int32_t* omant, const int32_t* oshift, hipStream_t s);
hipError_t launch_dec_argmax_part(const int32_t* logits, int n, uint64_t* part, int nparts, int32_t* record,
                                  const int32_t* step, int32_t* pos, int advance, hipStream_t s);
hipError_t launch_dec_embed_argmax(const uint64_t* part, int nparts, const int16_t* emb, int d, int32_t* r,
                                   int32_t* token, int32_t* step, hipStream_t s);
hipError_t launch_w12_swiglu(const int8_t* x, const int8_t* lo, const uint8_t* nib, int M, int F, int kp,
                             const int32_t* mant, const int32_t* shift, const int16_t* silu, int h_shift, int8_t* y,
                             int ystride, hipStream_t s);
size_t ql_workspace_bytes(int64_t rows, int64_t in, int64_t out, size_t off[KT_QL_WS_PARTS]);
// The one-row product alone (kt_hip_quant_linear_multi_sums): no bias, the sums and states left in the workspace.
bool ql_sums_ok(int64_t in, int64_t out, int pw, int64_t flush_k);
hipError_t launch_quant_linear_sums(const int32_t* x, int64_t in, const kt_hip_qscale* xs, const int8_t* wb, int pw,
                                    int nseg, const int64_t* seg_out, const int64_t* w_mant, const int32_t* w_shift,
                                    int64_t flush_k, void* ws, hipStream_t s);
// Several QuantLinear calls on one x (seg_out[g] output columns each, weights side by side in wb): one x pass, one
// digit GEMM, each call's own requantization into y[g] with record os[g].
hipError_t launch_quant_linear_multi(const int32_t* x, int64_t rows, int64_t in, const kt_hip_qscale* xs,
                                     const int8_t* wb, int pw, int nseg, const int64_t* seg_out,
                                     const int64_t* w_mant, const int32_t* w_shift, const int64_t* bias,
                                     const int* has_bias, const int64_t* b_mant, const int32_t* b_shift,
                                     int64_t flush_k, void* ws, int32_t* const* y, kt_hip_qscale* os,
                                     hipStream_t s);
hipError_t launch_quant_linear(const int32_t* x, int64_t rows, int64_t in, const kt_hip_qscale* xs,
                               const int8_t* wb, int pw, int64_t out, int64_t w_mant, int32_t w_shift,
                               const int64_t* bias, int64_t b_mant, int32_t b_shift, int64_t flush_k, void* ws,
                               int32_t* y, kt_hip_qscale* os, hipStream_t s);
// A Conv2d lowered onto QuantLinear: the image x [ci][h][w], kernel kh x kw, stride, zero padding, output oh x ow.
struct ConvGeom {
    int32_t ci, h, w, kh, kw, stride, pad, oh, ow;
};
// Conv2d::forward_int (conv.rs:68-130) as QuantLinear over the im2col rows (oh * ow rows of ci * kh * kw columns;
// the workspace is ql_workspace_bytes of that shape) with the output stored [co][oh][ow].
hipError_t launch_ref_conv2d(const int32_t* x, const ConvGeom& g, const kt_hip_qscale* xs, const int8_t* wb, int pw,
                             int64_t co, int64_t w_mant, int32_t w_shift, const int64_t* bias, int64_t b_mant,
                             int32_t b_shift, int64_t flush_k, void* ws, int32_t* y, kt_hip_qscale* os,
                             hipStream_t s);
// The device address of device `dev`'s QuantLinear scratch array (KT_QL_SCRATCH_BYTES), looked up once per device;
// `dev` must be the current device.
hipError_t ql_scratch(int dev, void** ptr, hipStream_t s);
hipError_t launch_w12_linear_norm(const int32_t* r, int M, int d, const int8_t* lo, const uint8_t* nib, int N,
                                  const int32_t* mant, const int32_t* shift, int out_kind, void* y, hipStream_t s);
hipError_t launch_w12_swiglu_norm(const int32_t* r, int M, int d, const int8_t* lo, const uint8_t* nib, int F,
                                  const int32_t* mant, const int32_t* shift, const int16_t* silu, int h_shift,
                                  int8_t* y, int ystride, hipStream_t s);
struct RdAttn;
size_t rd_attention_lds(int max_seq, int nh, int hd, int hb);
hipError_t launch_rd_embed(const int32_t* emb, int64_t e_mant, int32_t e_shift, const int32_t* token, int vocab,
                           int dim, int32_t* y, kt_hip_qscale* ys, hipStream_t s);
hipError_t launch_rd_rmsnorm(const int32_t* x, int rows, int dim, const kt_hip_qscale* xs, const int32_t* g,
                             int64_t g_mant, int32_t g_shift, int64_t e_mant, int32_t e_shift, int32_t* y,
                             kt_hip_qscale* ys, hipStream_t s);
hipError_t launch_rd_add(const int32_t* a, const kt_hip_qscale* as, const int32_t* b, const kt_hip_qscale* bs, int n,
                         int32_t* y, kt_hip_qscale* ys, hipStream_t s);
hipError_t launch_rd_swiglu(const int32_t* g, const kt_hip_qscale* gs, const int32_t* u, const kt_hip_qscale* us,
                            int rows, int n, const int64_t* codes, const kt_hip_codelut* lut, int32_t* h,
                            kt_hip_qscale* hs, hipStream_t s);
hipError_t launch_rd_gelu(const int32_t* x, const kt_hip_qscale* xs, int64_t n, const int64_t* codes,
                          const kt_hip_codelut* lut, int32_t* y, kt_hip_qscale* ys, hipStream_t s);
size_t rq_workspace_bytes(int64_t rows, int64_t in, int64_t out, int64_t groups, size_t off[5]);
hipError_t launch_quant_linear_rows(const int32_t* x, const int32_t* xidx, int64_t x_rows, int64_t rows, int64_t in,
                                    const kt_hip_qscale* xs, int xs_step, int groups, const int64_t* off_dev,
                                    const int8_t* wb, size_t wgroup, int pw, int64_t out, const int64_t* wm_dev,
                                    const int32_t* wsh_dev, int64_t flush_k, void* ws, int32_t* y, kt_hip_qscale* ys,
                                    hipStream_t s);
hipError_t launch_rm_bucket(const int32_t* sel, int P, int top_k, int E, int64_t* off, int32_t* xidx, int32_t* pos,
                            hipStream_t s);
hipError_t launch_rm_route(const int32_t* logits, int T, int E, int top_k, const kt_hip_qscale* ls, int sigmoid,
                           int norm_topk, const int64_t* codes, const kt_hip_codelut* lut, const int64_t* bias,
                           int32_t* sel, int64_t* ec, int64_t* sumc, hipStream_t s);
hipError_t launch_rm_combine(const int32_t* y, const kt_hip_qscale* ys, int y_rows, int dim, const int32_t* pos,
                             const int64_t* ec, const int64_t* sumc, int T, int top_k, int32_t* out,
                             kt_hip_qscale* os, hipStream_t s);
size_t rm_merge_workspace_bytes(int64_t T);
hipError_t launch_rm_merge_rows(const int32_t* rows, const kt_hip_qscale* rs, int T, int dim, void* ws, int32_t* out,
                                kt_hip_qscale* os, hipStream_t s);
hipError_t launch_rd_attention_step(const RdAttn& a, hipStream_t s);
hipError_t launch_rd_argmax(const int32_t* logits, int n, const kt_hip_qscale* ls, int32_t* token, int32_t* record,
                            kt_hip_sscale* rscale, int32_t* step, hipStream_t s);
hipError_t launch_mfma_probe(const int8_t* a, const int8_t* b, int32_t* c32, int32_t* c16, hipStream_t s);

}  // namespace kt
