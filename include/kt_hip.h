/*
 * kt_hip.h -- C ABI of the MI355X (gfx950) exact-integer linear backend for tritify.
 *
 * This is the drop-in boundary for tritify's hot path, the LinearBackend seam
 * (crates/01-engine/kt-core/src/backend.rs:46-58): Y[r,o] = sum_k X[r,k] * W[o,k] with i32 codes in and exact
 * i64 sums out. It replaces the reference's CUDA digit backend (crates/02-runtime/kt-cuda) at the same two levels:
 *
 *   - the device layer, which replaces the kt_cuda_* C functions of crates/02-runtime/kt-cuda/src/digit_gemm.cu:86-147
 *     (bound in Rust at crates/02-runtime/kt-cuda/src/device.rs:9-38);
 *   - the backend layer, which replaces TcLinear<DeviceExec> (crates/02-runtime/kt-cuda/src/backend.rs:77-192 and
 *     kt_cuda::open / open_planted, crates/02-runtime/kt-cuda/src/lib.rs:252-279): bounds, packing, resident
 *     weights keyed by WeightId under an LRU byte budget, and the LinearBackend calls themselves.
 *
 * A third group serves the 12-bit-weight workloads (int8 activations x 12-bit codes, per-channel requant) with
 * operands resident in device memory.
 *
 * Conventions (as kt_cuda's): every function returning int returns a hipError_t code, 0 = success; an error never
 * leaves a partial result that looks valid. All pointers are plain host or device pointers; sizes are element counts
 * unless named _bytes. Device-layer calls take the device index and make it current. Stream arguments are
 * hipStream_t values passed as void* (NULL = the device's null stream).
 */
#ifndef KT_HIP_H
#define KT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Output kinds of the 12-bit-weight path. */
#define KT_OUT_I64 0 /* the exact accumulators */
#define KT_OUT_I32 1 /* per-channel requant, saturated to i32 */
#define KT_OUT_I8 2  /* per-channel requant, clamped to [-127, 127] */
#define KT_OUT_I32_ADD 3 /* per-channel requant saturated to i32, added (saturating) to the i32 already in y */

/* Planted defects (firing controls). Only the test build, libkt_hip_planted.so, accepts them; the product library
 * returns hipErrorNotSupported from kt_hip_open_planted. Mirrors kt_cuda::Plant
 * (crates/02-runtime/kt-cuda/src/backend.rs:31-40). */
#define KT_PLANT_DROP_TOP 1       /* the recombination skips the top plane pair (DropPlane22) */
#define KT_PLANT_WRONG_CARRY 2    /* the activation split drops the carry of a rebalanced digit (WrongCarry) */
#define KT_PLANT_NO_FLUSH 3       /* the int32 accumulators are never flushed into i64 (NoFlush) */
#define KT_PLANT_CACHE_BY_SHAPE 4 /* resident weights keyed by shape only (CacheByShape) */

/* ---------------------------------------------------------------------------------------------------------------
 * Device layer. Replaces kt_cuda_device_count / _device_info / _alloc / _free / _upload / _error_string
 * (digit_gemm.cu:88-119,145; device.rs:10-21,37).
 * ------------------------------------------------------------------------------------------------------------- */
int kt_hip_device_count(int* n);
int kt_hip_device_info(int dev, char* name, int len, int* major, int* minor, size_t* free_bytes);
int kt_hip_alloc(int dev, size_t bytes, void** p);
int kt_hip_free(int dev, void* p);
int kt_hip_upload(int dev, void* dst, const void* src, size_t bytes);
int kt_hip_download(int dev, void* dst, const void* src, size_t bytes);
const char* kt_hip_error_string(int e);

/* Digit planes: `codes_dev` (rows x k i32, device) -> `planes` balanced base-256 int8 planes, layout
 * [planes][rows][kp] with kp = kt_hip_kp(k) and zero padding. Replaces the host-side digits::pack
 * (crates/02-runtime/kt-cuda/src/digits.rs:83-101), which this backend runs on the device. */
int64_t kt_hip_kp(int64_t k);
int kt_hip_planes_for(const int32_t* codes, size_t n); /* 1, 3 or 5: the plane count the backend uses */
int kt_hip_pack_planes(int dev, const int32_t* codes_dev, int64_t rows, int64_t k, int planes, int8_t* planes_dev,
                       void* stream);

/* The digit-plane product on device buffers. Replaces kt_cuda_digit_gemm (digit_gemm.cu:123-143; device.rs:23-36),
 * minus its host copies: xa_dev holds px planes of rows x k, wb_dev pw planes of out x k (px, pw in {1, 3, 5}),
 * y_dev receives rows x out i64. `flush_k` (a multiple of 256, or <= 0 for the backend's bound) is the k-chunk after
 * which int32 sums are added into i64; drop_top is the planted DropPlane22 and must be 0 outside tests. */
int64_t kt_hip_flush_k(int px, int pw);
int kt_hip_digit_gemm(int dev, const int8_t* xa_dev, int px, const int8_t* wb_dev, int pw, int64_t* y_dev,
                      int64_t rows, int64_t out, int64_t k, int64_t flush_k, int drop_top, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * QuantLinear::forward_int on the device (crates/01-engine/kt-core/src/layers.rs:275-328, helpers 23-39): the
 * reference's dynamic per-tensor quantization before and after the seam, with no host round trip.
 * ------------------------------------------------------------------------------------------------------------- */
/* A tensor's Scale (kt-int Scale { mant, shift }, real = code * mant / 2^shift) as a device record, plus the two
 * maxima of the call that produced it (0 where not reached). The output record of one layer is the input record of
 * the next. */
typedef struct {
    int64_t mant;
    int32_t shift;
    int32_t pad;
    int64_t xmax;
    int64_t ymax;
} kt_hip_qscale;
/* workspace parts: x planes, i64 accumulators, partial maxima (of |x|, or for one row of the product per 8 output
 * columns), split-k tile counters, state */
#define KT_QL_WS_PARTS 5
#define KT_QL_PARTS 1024 /* partial maxima per reduction */
/* Workspace bytes of kt_hip_quant_linear for rows x in_f -> out_f (parts at *off, 256-byte aligned). */
size_t kt_hip_quant_linear_workspace(int64_t rows, int64_t in_f, int64_t out_f, size_t off[KT_QL_WS_PARTS]);
/* y_dev (rows x out_f i32 codes) and os_dev (their Scale) = QuantLinear::forward_int of x_dev (rows x in_f i32
 * codes at the scale in xs_dev, device) against weights held as pw in {1, 3, 5} digit planes (kt_hip_pack_planes of
 * the out_f x in_f codes) at scale (w_mant, w_shift), with optional bias codes bias_dev (out_f i64, device; NULL =
 * none) at scale (b_mant, b_shift):
 *   xmax = max |x|; xmax == 0 -> y = bias codes at the bias scale, or zeros at Scale::ZERO;
 *   qx = quant_to(x, xmax) = round_half_away(x * WLEVELS / xmax); c = from_ratio(xmax, WLEVELS) * xs * ws;
 *   c == 0 -> zeros; acc = qx . w^T (exact, i64) + (bs * c^-1).apply(bias); ymax = max |acc|; ymax == 0 -> zeros;
 *   y = requant_dyn(acc, 2^28, ymax), os = from_ratio(ymax, 2^28) * c.
 * Every pass runs on `stream` with no host synchronization (capturable in a HIP graph). ws_dev is the caller's
 * workspace of kt_hip_quant_linear_workspace bytes; calls that share one workspace must not overlap. Requires
 * rows, in_f, out_f >= 1, rows * kp and rows * out_f below 2^31, mantissas >= 0. */
int kt_hip_quant_linear(int dev, const int32_t* x_dev, int64_t rows, int64_t in_f, const kt_hip_qscale* xs_dev,
                        const int8_t* w_planes_dev, int pw, int64_t out_f, int64_t w_mant, int32_t w_shift,
                        const int64_t* bias_dev, int64_t b_mant, int32_t b_shift, void* ws_dev, size_t ws_bytes,
                        int32_t* y_dev, kt_hip_qscale* os_dev, void* stream);
/* Several QuantLinear::forward_int calls on the same x (the reference's projections of one tensor, layers.rs:275-328
 * called once each: q / k / v, gate / up), their outputs computed together: one quantization of x, one digit GEMM over
 * the weights side by side, each call's own bias, output maximum, requant_dyn and record. nseg calls of seg_out[g]
 * output columns; w_planes_dev: the pw digit planes of the calls' weight codes stacked by rows (kt_hip_pack_planes of
 * the (sum seg_out) x in_f matrix); w_mant / w_shift, has_bias / b_mant / b_shift: host arrays, one entry per call;
 * bias_dev: NULL or the stacked bias codes (zeros where a call has none); y_devs: a host array of nseg device
 * pointers (rows x seg_out[g] codes each); os_dev: nseg records. Each call's codes and record equal
 * kt_hip_quant_linear's. Every boundary between calls must be a multiple of kt_hip_quant_linear_multi_align(rows,
 * sum seg_out, pw) (else hipErrorInvalidValue: make the calls one at a time). ws_dev: kt_hip_quant_linear_workspace
 * of (rows, in_f, sum seg_out) bytes. No counterpart in the reference's API: it replaces nseg calls. */
#define KT_QL_MAX_SEGMENTS 4
int kt_hip_quant_linear_multi(int dev, const int32_t* x_dev, int64_t rows, int64_t in_f, const kt_hip_qscale* xs_dev,
                              int nseg, const int64_t* seg_out, const int8_t* w_planes_dev, int pw,
                              const int64_t* w_mant, const int32_t* w_shift, const int64_t* bias_dev,
                              const int* has_bias, const int64_t* b_mant, const int32_t* b_shift, void* ws_dev,
                              size_t ws_bytes, int32_t* const* y_devs, kt_hip_qscale* os_dev, void* stream);
int64_t kt_hip_quant_linear_multi_align(int64_t rows, int64_t out_f, int pw);
/* The decode row's QuantLinear calls up to their exact sums: kt_hip_quant_linear_multi at rows = 1 with no bias and
 * no codes out -- the quantization of x and the digit product, one launch -- leaving each call's i64 sums and state
 * (max |x|, c = from_ratio(xmax, WLEVELS) * xs * ws, the mode) in ws_dev for the op that reads the output next,
 * which applies requant_dyn (layers.rs:33-39, 321-327) itself and forms the record (the kt_hip_ref_*_sums entry
 * points): one launch fewer per projection, the same integers as kt_hip_quant_linear_multi followed by the plain
 * entry point. ws_dev (kt_hip_quant_linear_workspace(1, in_f, sum seg_out) bytes) must not be reused before that op
 * has run. Requires kt_hip_quant_linear_sums_ok(in_f, sum seg_out, pw) (the one-launch product takes the shape) and
 * every boundary between calls a multiple of 8. No counterpart in the reference's API: it splits QuantLinear's
 * forward_int at its requant. */
int kt_hip_quant_linear_sums_ok(int64_t in_f, int64_t out_f, int pw);
int kt_hip_quant_linear_multi_sums(int dev, const int32_t* x_dev, int64_t in_f, const kt_hip_qscale* xs_dev,
                                   int nseg, const int64_t* seg_out, const int8_t* w_planes_dev, int pw,
                                   const int64_t* w_mant, const int32_t* w_shift, void* ws_dev, size_t ws_bytes,
                                   void* stream);
/* One call's output of a kt_hip_quant_linear_multi_sums launch, as the op that reads it takes it: that launch's
 * workspace and shape (in_f, out_f = sum seg_out), the call's index seg and its columns [col0, col0 + n), and where
 * the reader writes the output's record (kt_hip_quant_linear's os_dev for that call), or NULL for none. */
typedef struct {
    const void* ws;
    int64_t in_f, out_f, col0, n;
    int32_t seg;
    int32_t pad;
    kt_hip_qscale* rec;
} kt_hip_ql_sums;
/* kt_hip_quant_linear with no workspace argument and no allocation of any kind: the workspace lives in a
 * library-owned device array of KT_QL_SCRATCH_BYTES on each GPU (held until the process ends), so the call can run
 * where hipMalloc cannot (code under HIP graph capture, tight serving loops, hosts that forbid allocation). No
 * counterpart in the reference; it is for those callers that cannot allocate. Same integers, arguments and
 * requirements as kt_hip_quant_linear, plus kt_hip_quant_linear_workspace(rows, in_f, out_f) <=
 * KT_QL_SCRATCH_BYTES (else hipErrorInvalidValue before any device work). Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams, two threads) race and must be ordered by the caller. The first
 * call on a GPU looks up its array's address (a runtime call outside any stream), so it must run eagerly: a first
 * call whose stream is being captured returns hipErrorStreamCaptureUnsupported and does nothing; every later call,
 * any shape, may be captured. */
#define KT_QL_SCRATCH_BYTES ((size_t)32 << 20)
int kt_hip_quant_linear_noalloc(int dev, const int32_t* x_dev, int64_t rows, int64_t in_f,
                                const kt_hip_qscale* xs_dev, const int8_t* w_planes_dev, int pw, int64_t out_f,
                                int64_t w_mant, int32_t w_shift, const int64_t* bias_dev, int64_t b_mant,
                                int32_t b_shift, int32_t* y_dev, kt_hip_qscale* os_dev, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * The reference decoder's layers at the reference's own integer semantics (crates/01-engine/kt-core/src/
 * {layers,attention,model,generate}.rs), device-resident: activations are i32 codes at the 2^28 level with one
 * kt-int Scale per tensor (a kt_hip_qscale record, the 32-byte device record of kt_hip_quant_linear), 12-trit
 * weight codes, per-tensor dynamic requant after every op. With kt_hip_quant_linear for every projection they run
 * DecoderModel::decode_step (model.rs:290-294, 338-353) with no host round trip. Each call is one launch on
 * `stream`; output records may not alias input records of the same call except where noted.
 * ------------------------------------------------------------------------------------------------------------- */
/* A signed Scale: sign * mant * 2^-shift (sign +1 or -1). The RoPE tables' entries (attention.rs:58-60) and the KV
 * cache's per-step scales (sign +1). */
typedef struct {
    int64_t mant;
    int32_t shift;
    int32_t sign;
} kt_hip_sscale;
/* A CodeLut's run-time constants (kt-int/src/lib.rs:346-396): the index factor inv_step as a Scale, lo_index,
 * the entry count n, the code scale, the identity right tail. Its n codes (i64) live in device memory. */
typedef struct {
    int64_t inv_mant;
    int32_t inv_shift;
    int32_t n;
    int64_t lo_index;
    int64_t code_mant;
    int32_t code_shift;
    int32_t right_identity;
} kt_hip_codelut;
#define KT_LUT_EXP 0  /* exp(x): the softmax table of Attention::new and MoeMlp::new */
#define KT_LUT_SILU 1 /* x / (1 + exp(-x)): SwiGluMlp::new's SiLU */
#define KT_LUT_SIGMOID 2 /* 1 / (1 + exp(-x)): SigmoidScore::new's router score (router.rs:38-49) */
#define KT_LUT_GELU 3    /* 0.5 x (1 + erf(x / sqrt 2)), erf by A&S 7.1.26: build_gelu_lut (kt-model-vision/src/
                            nonlin.rs:7-26) */
#define KT_REF_MAX_HEADS 64
#define KT_REF_ATTN_LDS 65536 /* the attention step's LDS: at least 40 B per cached position + 12 B per q value */
#define KT_REF_ATTN_MAX_SEQ 65536 /* the longest cache the attention step takes (with a workspace) */

/* Offline tables (host only, no GPU; f64 with the C library's exp/pow/cos/sin, as the reference's f64 methods use
 * its platform's): Scale::from_f64 (lib.rs:215-222); CodeLut::build (lib.rs:359-379) of `kind` over [lo, hi] at
 * 2^idx_bits entries and 2^code_bits code scale (codes may be NULL: constants only); the RoPE tables of
 * Attention::new / rope_tables (attention.rs:64-90): entry p * rot_dim/2 + j is the signed Scale of
 * cos / sin(p * theta^(-2j/rot_dim)). */
void kt_hip_ref_scale_from_f64(double x, int64_t* mant, int32_t* shift);
int kt_hip_ref_codelut(int kind, double lo, double hi, int idx_bits, int code_bits, int right_identity,
                       int64_t* codes, kt_hip_codelut* lut);
int kt_hip_ref_rope_tables(int64_t max_seq, int64_t rot_dim, double theta, kt_hip_sscale* cos_tab,
                           kt_hip_sscale* sin_tab);
/* IntTensor::from_reals (crates/01-engine/kt-core/src/tensor.rs:106-117), the model's entry quantization (SAM's
 * pixels, kt-model-vision/src/plugin.rs:38): codes round(v * levels / max |v|) (half away from zero) at
 * Scale::from_f64(max / levels); all zeros give zeros at Scale::ZERO. Host only; non-finite values are an error
 * (1 <= levels <= 2^30). */
int kt_hip_ref_from_reals(const double* real, int64_t n, int64_t levels, int32_t* codes, int64_t* mant,
                          int32_t* shift);

/* Embedding::lookup (layers.rs:1127-1140): y (dim codes) and ys = the row of the token at token_dev[0] of the
 * vocab x dim code table at Scale (e_mant, e_shift); a token outside [0, vocab) gives zeros at Scale::ZERO. */
int kt_hip_ref_embed(int dev, const int32_t* emb_dev, int64_t e_mant, int32_t e_shift, const int32_t* token_dev,
                     int64_t vocab, int64_t dim, int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream);
/* Embedding::lookup_seq (layers.rs:1138-1145): y (T x dim codes) = the rows of the T tokens at tokens_dev, at the
 * table's Scale; a token outside [0, vocab) gives a zero row (the reference panics). */
int kt_hip_ref_embed_seq(int dev, const int32_t* emb_dev, int64_t e_mant, int32_t e_shift, const int32_t* tokens_dev,
                         int64_t T, int64_t vocab, int64_t dim, int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream);
/* RmsNorm::forward_int, add and SwiGluMlp's activation (as kt_hip_ref_rmsnorm / _add / _swiglu with rows = 1: the
 * same integers) over whole-sequence tensors on many CTAs, for the batched forward's T-row tensors: one CTA forms the
 * tensor's Scales (and RMSNorm's row factors, any number of rows) into the workspace, a grid pass takes the largest
 * magnitude, a grid pass requantizes. The workspace holds kt_hip_ref_seq_workspace(rows) bytes (rows = 1 for add
 * and SwiGLU); add's y_dev / ys_dev may alias a / as or b / bs. */
size_t kt_hip_ref_seq_workspace(int64_t rows);
int kt_hip_ref_rmsnorm_seq(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t rows, int64_t dim,
                           const int32_t* g_dev, int64_t g_mant, int32_t g_shift, int64_t eps_mant, int32_t eps_shift,
                           void* ws_dev, size_t ws_bytes, int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream);
int kt_hip_ref_add_seq(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev, const int32_t* b_dev,
                       const kt_hip_qscale* bs_dev, int64_t n, void* ws_dev, size_t ws_bytes, int32_t* y_dev,
                       kt_hip_qscale* ys_dev, void* stream);
int kt_hip_ref_swiglu_seq(int dev, const int32_t* g_dev, const kt_hip_qscale* gs_dev, const int32_t* u_dev,
                          const kt_hip_qscale* us_dev, int64_t n, const int64_t* silu_codes_dev,
                          const kt_hip_codelut* silu, void* ws_dev, size_t ws_bytes, int32_t* h_dev,
                          kt_hip_qscale* hs_dev, void* stream);
/* Attention::forward_int between its projections over a whole sequence (attention.rs:467-598), the prefill of
 * DecoderModel's batched forward: q (T x nh hd), k and v (T x nkv hd) codes at one Scale each; row i rotated at
 * position i (the RoPE tables of kt_hip_ref_rope_tables, T <= max_seq); per head and row the causal integer-code
 * softmax at the one score scale q.scale * k.scale * (isq_mant, isq_shift) with the exp CodeLut; per (row, head)
 * the scale v.scale / sumc; all brought to their largest (the engine's fold over the [row][head] order) and
 * requantized: o_dev (T x nh hd) and os_dev. hd <= 256, T <= 8192; the workspace holds
 * kt_hip_ref_attention_prefill_workspace bytes (0: out of range). */
size_t kt_hip_ref_attention_prefill_workspace(int64_t T, int64_t nh, int64_t nkv, int64_t hd);
int kt_hip_ref_attention_prefill(int dev, const int32_t* q_dev, const kt_hip_qscale* qs_dev, const int32_t* k_dev,
                                 const kt_hip_qscale* ks_dev, const int32_t* v_dev, const kt_hip_qscale* vs_dev,
                                 int64_t T, int64_t nh, int64_t nkv, int64_t hd, int64_t max_seq,
                                 const kt_hip_sscale* cos_dev, const kt_hip_sscale* sin_dev, int64_t isq_mant,
                                 int32_t isq_shift, const int64_t* exp_codes_dev, const kt_hip_codelut* exp_lut,
                                 void* ws_dev, size_t ws_bytes, int32_t* o_dev, kt_hip_qscale* os_dev, void* stream);
/* RmsNorm::forward_int (layers.rs:392-434) of rows (<= 1024) x dim codes at xs: gamma codes g_dev at (g_mant,
 * g_shift), eps as the Scale (eps_mant, eps_shift). */
int kt_hip_ref_rmsnorm(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t rows, int64_t dim,
                       const int32_t* g_dev, int64_t g_mant, int32_t g_shift, int64_t eps_mant, int32_t eps_shift,
                       int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream);
/* add (layers.rs:121-136), the residual add of n codes: y_dev may alias a_dev or b_dev, ys_dev as_dev or bs_dev. */
int kt_hip_ref_add(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev, const int32_t* b_dev,
                   const kt_hip_qscale* bs_dev, int64_t n, int32_t* y_dev, kt_hip_qscale* ys_dev, void* stream);
/* add (layers.rs:121-136) and then RmsNorm::forward_int (layers.rs:392-434) of the sum, for one row of n <= 4096
 * codes: DecoderModel::decode_step's residual add followed by the next norm (model.rs:338-353), as one launch. y / ys
 * are kt_hip_ref_add's outputs (y_dev may alias a_dev or b_dev, ys_dev as_dev or bs_dev), h / hs kt_hip_ref_rmsnorm's
 * of y with gamma g at (g_mant, g_shift) and eps (eps_mant, eps_shift): the same integers as the two calls in
 * sequence. h_dev must not alias a_dev, b_dev or y_dev, nor hs_dev ys_dev. */
int kt_hip_ref_add_rmsnorm(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev, const int32_t* b_dev,
                           const kt_hip_qscale* bs_dev, int64_t n, int32_t* y_dev, kt_hip_qscale* ys_dev,
                           const int32_t* g_dev, int64_t g_mant, int32_t g_shift, int64_t eps_mant, int32_t eps_shift,
                           int32_t* h_dev, kt_hip_qscale* hs_dev, void* stream);
/* kt_hip_ref_add_rmsnorm with b the output of a kt_hip_quant_linear_multi_sums call (b->n == n): its requant_dyn
 * and record formed in the same launch, then the add and the norm -- the same integers as that QuantLinear call
 * (kt_hip_quant_linear_multi) followed by kt_hip_ref_add_rmsnorm. y_dev may alias a_dev. */
int kt_hip_ref_add_rmsnorm_sums(int dev, const int32_t* a_dev, const kt_hip_qscale* as_dev, const kt_hip_ql_sums* b,
                                int64_t n, int32_t* y_dev, kt_hip_qscale* ys_dev, const int32_t* g_dev,
                                int64_t g_mant, int32_t g_shift, int64_t eps_mant, int32_t eps_shift, int32_t* h_dev,
                                kt_hip_qscale* hs_dev, void* stream);
/* SwiGluMlp::forward_int's activation (layers.rs:615-637): h = requant_dyn(silu_code(g) * u), the SiLU CodeLut
 * (right_identity set) with its codes at silu_codes_dev, for `rows` tensors of n values each, row r with its own
 * records gs_dev[r], us_dev[r], hs_dev[r] (rows = 1: one tensor; rows > 1: the per-token expert calls of a MoE). */
int kt_hip_ref_swiglu(int dev, const int32_t* g_dev, const kt_hip_qscale* gs_dev, const int32_t* u_dev,
                      const kt_hip_qscale* us_dev, int64_t rows, int64_t n, const int64_t* silu_codes_dev,
                      const kt_hip_codelut* silu, int32_t* h_dev, kt_hip_qscale* hs_dev, void* stream);
/* kt_hip_ref_swiglu of one tensor (rows = 1, n <= 8192) with g and u the outputs of kt_hip_quant_linear_multi_sums
 * calls (g->n == u->n == n; the gate / up pair of one launch): their requant_dyn and records formed in the same
 * launch -- the same integers as the QuantLinear calls followed by kt_hip_ref_swiglu. */
int kt_hip_ref_swiglu_sums(int dev, const kt_hip_ql_sums* g, const kt_hip_ql_sums* u, int64_t n,
                           const int64_t* silu_codes_dev, const kt_hip_codelut* silu, int32_t* h_dev,
                           kt_hip_qscale* hs_dev, void* stream);
/* apply_gelu (crates/03-models/kt-model-vision/src/nonlin.rs:30-45) of n codes at xs_dev through the GELU CodeLut
 * (KT_LUT_GELU over [-10, 10], 2^16 entries, 2^20 code scale, right_identity set; its codes at gelu_codes_dev): y_dev
 * (may alias x_dev) at the table's code scale, written to ys_dev (which may not alias xs_dev). */
int kt_hip_ref_gelu(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t n,
                    const int64_t* gelu_codes_dev, const kt_hip_codelut* gelu, int32_t* y_dev, kt_hip_qscale* ys_dev,
                    void* stream);
/* Conv2d::forward_int (crates/01-engine/kt-core/src/conv.rs:68-130), SAM's PatchEmbed (kt-model-vision/src/
 * hiera.rs:187-190): the image x_dev [ci][h][w] of i32 codes at xs_dev, quant_to by its whole-image max, the
 * convolution against co x (ci kh kw) weight codes in the reference's [co][ci][kh][kw] order held as digit planes
 * (kt_hip_pack_planes of that co x ci*kh*kw matrix, pw planes) at Scale (w_mant, w_shift), the optional i64 bias
 * codes at (b_mant, b_shift) brought into the product's units, requant_dyn by the whole output's max. y_dev
 * [co][oh][ow], oh = (h + 2 pad - kh) / stride + 1 (ow alike), and its record in os_dev; an all-zero image gives
 * zeros at Scale::ZERO. The workspace holds kt_hip_ref_conv2d_workspace bytes (0: a shape out of range). */
size_t kt_hip_ref_conv2d_workspace(int64_t ci, int64_t h, int64_t w, int64_t co, int64_t kh, int64_t kw,
                                   int64_t stride, int64_t pad);
int kt_hip_ref_conv2d(int dev, const int32_t* x_dev, const kt_hip_qscale* xs_dev, int64_t ci, int64_t h, int64_t w,
                      const int8_t* w_planes_dev, int pw, int64_t co, int64_t kh, int64_t kw, int64_t stride,
                      int64_t pad, int64_t w_mant, int32_t w_shift, const int64_t* bias_dev, int64_t b_mant,
                      int32_t b_shift, void* ws_dev, size_t ws_bytes, int32_t* y_dev, kt_hip_qscale* os_dev,
                      void* stream);
/* Attention::decode_step between its projections (attention.rs:358-458) at the position pos_dev[0]: RoPE of the q
 * (nh x hd) and k (nkv x hd) codes by the tables cos_dev / sin_dev (max_seq x hd/2), the rotated k and the v codes
 * appended at row pos of kc_dev / vc_dev (max_seq x nkv hd) with their scales at kscale_dev / vscale_dev[pos], the
 * integer-code softmax over rows 0..pos at a common score scale (1/sqrt(hd) as (isq_mant, isq_shift); the exp
 * CodeLut), and the heads brought to one scale: o_dev (nh hd codes) and os_dev, the o projection's input. Rows
 * 0..pos-1 are those of earlier calls. A position outside [0, max_seq) gives zeros. nh <= KT_REF_MAX_HEADS, nh a
 * multiple of nkv, hd even; without a workspace LDS (KT_REF_ATTN_LDS) bounds max_seq (about 1,369 positions at
 * nh = 14, hd = 64): kt_hip_ref_attention_step_ws takes longer caches. */
int kt_hip_ref_attention_step(int dev, const int32_t* q_dev, const kt_hip_qscale* qs_dev, const int32_t* k_dev,
                              const kt_hip_qscale* ks_dev, const int32_t* v_dev, const kt_hip_qscale* vs_dev,
                              const int32_t* pos_dev, int64_t nh, int64_t nkv, int64_t hd, int64_t max_seq,
                              int32_t* kc_dev, int32_t* vc_dev, kt_hip_sscale* kscale_dev, kt_hip_sscale* vscale_dev,
                              const kt_hip_sscale* cos_dev, const kt_hip_sscale* sin_dev, int64_t isq_mant,
                              int32_t isq_shift, const int64_t* exp_codes_dev, const kt_hip_codelut* exp_lut,
                              int32_t* o_dev, kt_hip_qscale* os_dev, void* stream);
/* kt_hip_ref_attention_step with a workspace: several CTAs per q head (the cache reads and the per-step Scale work of
 * the head in each, P.V split between them: up to 128 CTAs in all; the parts added and the heads brought to one scale
 * by a second launch), for caches of any length up to
 * KT_REF_ATTN_MAX_SEQ (the reference's MAX_SEQ_CAP = 4096, crates/03-models/kt-model-decoder/src/lib.rs:46, and
 * beyond). ws_dev: a caller buffer of at least kt_hip_ref_attention_step_workspace(max_seq, nh, hd) bytes,
 * 16-byte aligned (per head: its output parts and scale, and 40 B per cached position and CTA). With ws_dev null this is
 * kt_hip_ref_attention_step (one CTA, max_seq bounded by its LDS). The same integers either way. Calls that share
 * ws_dev must be ordered. */
size_t kt_hip_ref_attention_step_workspace(int64_t max_seq, int64_t nh, int64_t hd);
int kt_hip_ref_attention_step_ws(int dev, const int32_t* q_dev, const kt_hip_qscale* qs_dev, const int32_t* k_dev,
                                 const kt_hip_qscale* ks_dev, const int32_t* v_dev, const kt_hip_qscale* vs_dev,
                                 const int32_t* pos_dev, int64_t nh, int64_t nkv, int64_t hd, int64_t max_seq,
                                 int32_t* kc_dev, int32_t* vc_dev, kt_hip_sscale* kscale_dev,
                                 kt_hip_sscale* vscale_dev, const kt_hip_sscale* cos_dev, const kt_hip_sscale* sin_dev,
                                 int64_t isq_mant, int32_t isq_shift, const int64_t* exp_codes_dev,
                                 const kt_hip_codelut* exp_lut, int32_t* o_dev, kt_hip_qscale* os_dev, void* ws_dev,
                                 size_t ws_bytes, void* stream);
/* kt_hip_ref_attention_step_ws (a workspace required) with q, k and v the outputs of kt_hip_quant_linear_multi_sums
 * calls (q->n == nh hd, k->n == v->n == nkv hd; the q / k / v trio of one launch): every CTA forms the three
 * outputs' maxima, Scales and the codes it reads itself (the first CTA writes the records) -- the same integers as
 * the QuantLinear calls followed by kt_hip_ref_attention_step_ws. */
int kt_hip_ref_attention_step_sums(int dev, const kt_hip_ql_sums* q, const kt_hip_ql_sums* k, const kt_hip_ql_sums* v,
                                   const int32_t* pos_dev, int64_t nh, int64_t nkv, int64_t hd, int64_t max_seq,
                                   int32_t* kc_dev, int32_t* vc_dev, kt_hip_sscale* kscale_dev,
                                   kt_hip_sscale* vscale_dev, const kt_hip_sscale* cos_dev,
                                   const kt_hip_sscale* sin_dev, int64_t isq_mant, int32_t isq_shift,
                                   const int64_t* exp_codes_dev, const kt_hip_codelut* exp_lut, int32_t* o_dev,
                                   kt_hip_qscale* os_dev, void* ws_dev, size_t ws_bytes, void* stream);
/* argmax_codes (generate.rs:48-56): token_dev[0] = the first index of the largest of n codes. With record_dev
 * non-null the codes are copied to record_dev + step * n and (mant, shift) of ls_dev to rscale_dev[step], step =
 * step_dev[0], which then advances (the per-step logits hash_step covers, generate.rs:58-64). record_dev holds
 * record_rows rows of n codes and rscale_dev record_rows entries: a step outside [0, record_rows) writes neither and
 * leaves step_dev unchanged (the token is still chosen), so replays of a captured step past the last row are
 * harmless. record_rows is ignored without a record. */
int kt_hip_ref_argmax(int dev, const int32_t* logits_dev, int64_t n, const kt_hip_qscale* ls_dev, int32_t* token_dev,
                      int32_t* record_dev, kt_hip_sscale* rscale_dev, int32_t* step_dev, int64_t record_rows,
                      void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * The reference's MoeMlp at its own semantics (crates/01-engine/kt-core/src/layers.rs:652-1020, router.rs:29-79):
 * every router and expert call is a QuantLinear of one token row; the rows are grouped by their weights only at the
 * product, which is exact.
 * ------------------------------------------------------------------------------------------------------------- */
#define KT_REF_MOE_MAX_E 4096 /* experts a route call takes (their codes live in LDS) */
#define KT_REF_MOE_MAX_K 32    /* top-k a route or combine call takes */
/* QuantLinear::forward_int (layers.rs:275-328) applied to each of `rows` rows on its own, as the reference's per-token
 * calls run it: output row r is forward_int of input row xidx_dev[r] of x_dev (x_rows x in_f; xidx_dev NULL: row
 * r; an index outside [0, x_rows) reads as zeros) at the scale record xs_dev[xs_step * r] (xs_step 0: one record
 * for every row, 1: one per row), quantized by its own max |x|, requantized by its own max |acc|, against the weights
 * of the group g holding r (rows off[g] .. off[g + 1] - 1, off_dev the groups + 1 offsets on the device, off[0] = 0,
 * off[groups] = rows): pw digit planes of out_f x in_f codes at w_planes_dev + g * w_group_bytes, in the tiled
 * layout of kt_hip_pack_planes_tiled (w_group_bytes at least kt_hip_pack_planes_tiled_bytes), Scale
 * (w_mant_dev[g], w_shift_dev[g]). No bias. y_dev: rows x out_f codes, ys_dev: rows
 * records. ws_dev: the caller's workspace of kt_hip_quant_linear_rows_workspace bytes. The group sizes are read on
 * the device (no host round trip): off_host, the same offsets on the host, is optional and only checked (an invalid
 * copy is an error); offsets on the device that are not monotone or leave [0, rows] are clamped into a valid split
 * rather than read out of bounds. Layers at model size bucket their rows with kt_hip_ref_moe_bucket. */
size_t kt_hip_quant_linear_rows_workspace(int64_t rows, int64_t in_f, int64_t out_f, int64_t groups);
/* The weight layout of kt_hip_quant_linear_rows: the pw balanced base-256 digit planes of rows x k codes (the digits
 * of kt_hip_pack_planes) stored by tile -- for each block of 128 rows, k in steps of 64 bytes, each step the planes'
 * 128 x 64-byte blocks with the 16-byte chunks of row r permuted by (r / 4) % 4 (the order the product's LDS reads
 * want) -- so that one output block's run of k is contiguous memory. Rows past `rows` and k past `k` are zero.
 * kt_hip_pack_planes_tiled_bytes: the size (0 for an invalid shape). */
size_t kt_hip_pack_planes_tiled_bytes(int64_t rows, int64_t k, int planes);
int kt_hip_pack_planes_tiled(int dev, const int32_t* codes_dev, int64_t rows, int64_t k, int planes,
                             int8_t* planes_dev, void* stream);
int kt_hip_quant_linear_rows(int dev, const int32_t* x_dev, const int32_t* xidx_dev, int64_t x_rows, int64_t rows,
                             int64_t in_f, const kt_hip_qscale* xs_dev, int xs_step, int64_t groups,
                             const int64_t* off_host, const int64_t* off_dev, const int8_t* w_planes_dev,
                             size_t w_group_bytes, int pw, int64_t out_f, const int64_t* w_mant_dev,
                             const int32_t* w_shift_dev, void* ws_dev, size_t ws_bytes, int32_t* y_dev,
                             kt_hip_qscale* ys_dev, void* stream);
/* MoeMlp::route / route_sigmoid (layers.rs:826-870; router.rs:61-71) of `tokens` rows of router logits (experts
 * codes each, row t at the record ls_dev[t]): softmax (sigmoid 0): the numerators exp(l - lmax) from the exp CodeLut
 * (codes_dev, lut; 0 below the table), top-k by logit code; sigmoid (sigmoid 1): the sigma codes from its CodeLut,
 * top-k by code + bias_dev[e] (the coded selection bias, round(b * 2^20)). Ties go to the lower index. sel_dev /
 * ec_dev: tokens x top_k experts and numerators in rank order; sumc_dev: the normalizer (norm_topk: the top-k sum;
 * else softmax: the sum over every expert, sigmoid: 2^20). */
int kt_hip_ref_moe_route(int dev, const int32_t* logits_dev, int64_t tokens, int64_t experts, int top_k,
                         const kt_hip_qscale* ls_dev, int sigmoid, int norm_topk, const int64_t* codes_dev,
                         const kt_hip_codelut* lut, const int64_t* bias_dev, int32_t* sel_dev, int64_t* ec_dev,
                         int64_t* sumc_dev, void* stream);
/* MoeMlp's bucket (layers.rs:928-937, forward_one_int's expert calls for every token) on the device: the tokens x
 * top_k pairs of sel_dev (expert ids, as kt_hip_ref_moe_route writes them) grouped by expert for
 * kt_hip_quant_linear_rows -- off_dev (experts + 1 offsets), xidx_dev (row -> token), pos_dev (pair t * top_k + i ->
 * row, for kt_hip_ref_moe_combine). The order of the rows inside a group is not fixed (each row is computed on its
 * own, so no result depends on it). A pair whose id is outside [0, experts) gets pos -1 and no row; the rows left
 * over read as zeros (xidx -1). */
int kt_hip_ref_moe_bucket(int dev, const int32_t* sel_dev, int64_t tokens, int top_k, int64_t experts,
                          int64_t* off_dev, int32_t* xidx_dev, int32_t* pos_dev, void* stream);
/* MoeMlp::combine (layers.rs:893-923) for each token: the top_k expert outputs at rows pos_dev[t * top_k + i] of
 * y_dev (y_rows rows of dim codes, records ys_dev; a row index outside them contributes nothing) brought to their
 * largest scale, summed with the numerators ec_dev, requantized, 1/sumc folded into the scale; zeros at Scale::ZERO
 * when sumc <= 0. out_dev: tokens x dim codes, os_dev: tokens records. */
int kt_hip_ref_moe_combine(int dev, const int32_t* y_dev, const kt_hip_qscale* ys_dev, int64_t y_rows, int64_t dim,
                           const int32_t* pos_dev, const int64_t* ec_dev, const int64_t* sumc_dev, int64_t tokens,
                           int top_k, int32_t* out_dev, kt_hip_qscale* os_dev, void* stream);
/* merge_rows (layers.rs:873-891): tokens rows of dim codes, row t at the record rs_dev[t], brought to the largest row
 * scale (of equal values the latest row's) and requantized as one tensor: out_dev and os_dev. */
size_t kt_hip_ref_merge_rows_workspace(int64_t tokens);
int kt_hip_ref_merge_rows(int dev, const int32_t* rows_dev, const kt_hip_qscale* rs_dev, int64_t tokens, int64_t dim,
                          void* ws_dev, size_t ws_bytes, int32_t* out_dev, kt_hip_qscale* os_dev, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Backend layer: one LinearBackend on one device (kt_cuda::open, lib.rs:252; TcLinear, backend.rs:77-192).
 * ------------------------------------------------------------------------------------------------------------- */
typedef struct kt_hip_backend kt_hip_backend;

/* Open device `dev` with a resident-weight budget in bytes (0 = 4/5 of the device memory free at open,
 * kt-cuda/src/device.rs:147-149). A budget of 1 evicts on every call. */
int kt_hip_open(int dev, uint64_t budget_bytes, kt_hip_backend** out);
/* The backend with one planted defect (kt_cuda::open_planted, lib.rs:270). Test build only. */
int kt_hip_open_planted(int dev, int plant, kt_hip_backend** out);
void kt_hip_close(kt_hip_backend* b);

/* LinearBackend::name (backend.rs:47-48): "hip:<device name>", "hip:<device name> [budget N B]" or
 * "planted-hip-<Plant>". Writes a NUL-terminated string of at most len bytes. */
int kt_hip_name(const kt_hip_backend* b, char* buf, int len);

/* LinearBackend::linear (backend.rs:49-52): x is rows x k, w is out x k, both row-major i32; y (rows x out i64,
 * caller-owned) receives Y[r,o] = sum_i x[r*k+i] * w[o*k+i], the integers Portable returns (wrapping i64 as the
 * reference's release build does). Every i32 code is in this backend's domain. */
int kt_hip_linear(kt_hip_backend* b, const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k,
                  int64_t* y);
/* LinearBackend::linear_weights (backend.rs:54-58): the same, told the weights' identity so they stay resident
 * between calls. The codes behind an id must never change (backend.rs:37). */
int kt_hip_linear_weights(kt_hip_backend* b, const int32_t* x, uint64_t weight_id, const int32_t* w, size_t rows,
                          size_t out, size_t k, int64_t* y);
/* WeightId::fresh (backend.rs:29-35): a process-local id, never reused. */
uint64_t kt_hip_weight_id_fresh(void);
/* TcLinear::resident_bytes (backend.rs:118-121). */
uint64_t kt_hip_resident_bytes(const kt_hip_backend* b);
/* kt_cuda::fallbacks (backend.rs:42-48): calls handed to a CPU path. This backend computes every i32 code and
 * every k on the device, so it never falls back and this stays 0. */
uint64_t kt_hip_fallbacks(void);

/* ---------------------------------------------------------------------------------------------------------------
 * The cross-backend gates (crates/02-runtime/kt-runtime/src/gate.rs:1-140; runtime_probe, examples/runtime_probe.rs:
 * 19-89): run the linear accumulate through every backend on one fixed corpus and require identical bytes. A gate
 * backend is a name and a linear_weights function with its context: this library's backend (kt_hip_gate_backend),
 * the engine's Portable (kt_hip_gate_portable, the gates' reference: the i64 dot of kt-core/src/backend.rs:66-160
 * on the CPU; no HIP call ever hands work to it), a planted build's backend, or a caller's own.
 * ------------------------------------------------------------------------------------------------------------- */
#define KT_GATE_NAME_LEN 96
#define KT_GATE_EINVAL 1     /* hipErrorInvalidValue */
#define KT_GATE_DIVERGED (-1) /* a gate found a backend whose bytes differ */
typedef struct {
    const char* label;
    uint64_t id; /* the weights' WeightId */
    size_t rows, out, k;
    const int32_t* x; /* rows x k */
    const int32_t* w; /* out x k */
} kt_gate_case;
typedef int (*kt_gate_linear_fn)(void* ctx, const int32_t* x, uint64_t weight_id, const int32_t* w, size_t rows,
                                 size_t out, size_t k, int64_t* y);
typedef struct {
    char name[KT_GATE_NAME_LEN];
    kt_gate_linear_fn linear_weights;
    void* ctx;
} kt_gate_backend;
/* GateReport (gate.rs:71-79): the backend's name, SHA-256 (hex) over every accumulator of every case in order
 * (little-endian i64), the cases whose accumulators differ from the first backend's (bit c for case c), and the
 * first error a call returned (its case counts as diverged). */
typedef struct {
    char backend[KT_GATE_NAME_LEN];
    char hash[65];
    uint64_t diverged;
    int error;
} kt_gate_report;
/* corpus() (gate.rs:26-58): the fixed corpus, library-owned and the same bytes on every machine; returns the count. */
size_t kt_hip_gate_corpus(const kt_gate_case** cases);
/* The bound cases, outside the corpus: flush_case() (gate.rs:60-69), the reference digit backend's smallest k beyond
 * one int32 flush, then this backend's own bound for 1-plane and 3-plane codes (one 256-deep chunk past
 * kt_hip_flush_k, every digit -128). Each answer is +-k * code^2. Returns the count. */
size_t kt_hip_gate_bound_cases(const kt_gate_case** cases);
int kt_hip_gate_portable(kt_gate_backend* out);
int kt_hip_gate_backend(kt_hip_backend* b, kt_gate_backend* out);
/* Portable::linear (backend.rs:143-160) on the host: the gates' reference. */
int kt_hip_portable_linear(const int32_t* x, const int32_t* w, size_t rows, size_t out, size_t k, int64_t* y);
/* equality_gate (gate.rs:81-106): every backend over the cases (at most 64), the first as the reference; one report
 * each. Returns 0 if all are byte-identical, KT_GATE_DIVERGED if any differs. */
int kt_hip_equality_gate(const kt_gate_backend* backends, size_t n, const kt_gate_case* cases, size_t ncases,
                         kt_gate_report* reports);
/* residency_gate (gate.rs:108-140): the cases twice over (the second pass reuses every resident weight), then two
 * weight matrices of one shape interleaved four times, each answer against Portable. 0 if it holds, else
 * KT_GATE_DIVERGED with msg naming the first case that differs. */
int kt_hip_residency_gate(const kt_gate_backend* b, const kt_gate_case* cases, size_t ncases, char* msg, size_t len);

/* ---------------------------------------------------------------------------------------------------------------
 * 12-bit-weight path (benchmark workloads), device-resident operands. No counterpart in the reference: there the
 * weights are 12-trit codes on the digit path above. W12 digits: lo = (v & 255) - 128 (int8), hi = (v + 2048) >> 8
 * (4 bits), v = lo + 256 hi - 1920, stored fragment-tiled in blocks of 32 rows x 32 k (64 lanes x 16 lo bytes and
 * 64 lanes x 8 nib bytes per block, in MFMA operand order). Activations are int8, m x kp, zero padded in k.
 * ------------------------------------------------------------------------------------------------------------- */
/* Bytes of the W12 planes of an n x k matrix: lo = round_up(n, 32) * kp, nib = lo / 2. */
void kt_hip_w12_bytes(int64_t n, int64_t k, size_t* lo_bytes, size_t* nib_bytes);
/* Pack n x k codes in [-2048, 2047] (device) into W12 planes (device). Codes outside the range give wrong planes:
 * use kt_hip_w12_upload to have them checked. */
int kt_hip_w12_pack(int dev, const int32_t* codes_dev, int64_t n, int64_t k, int8_t* lo_dev, uint8_t* nib_dev,
                    void* stream);
/* Check host codes (hipErrorInvalidValue if any is outside [-2048, 2047]), upload and pack them. */
int kt_hip_w12_upload(int dev, const int32_t* codes, int64_t n, int64_t k, int8_t* lo_dev, uint8_t* nib_dev);
/* Y = X W^T for int8 activations x_dev (m x kp, zero padded in k) against W12 weights (n x k), recombined exactly
 * in i64, then written per out_kind: KT_OUT_I64 the accumulators; KT_OUT_I32 / KT_OUT_I8 the per-output-channel
 * requant of crates/00-kernels/kt-int/src/lib.rs:78-86, round(acc * mant[o] / 2^shift[o]) half away from zero,
 * clamped to [-2^31, 2^31 - 1] / [-127, 127]. That value is exact for every int32 mant and shift (kt-int
 * wraps a product beyond i64 where this clamps; they agree wherever the value fits i64). mant_dev and shift_dev
 * (n x i32, device) may be NULL for KT_OUT_I64. m <= KT_W12_SKINNY_MAX_M runs the skinny kernel (one CTA per 16
 * output columns, k <= KT_W12_SKINNY_MAX_K), larger m the MFMA GEMM (k <= KT_W12_GEMM_MAX_K); longer k is
 * hipErrorInvalidValue. Asynchronous on `stream`. */
#define KT_W12_SKINNY_MAX_M 128
#define KT_W12_GEMM_MAX_K 131008 /* 131008 * 128 * 128 < 2^31: the GEMM's int32 plane accumulators cannot wrap */
#define KT_W12_SKINNY_MAX_K 262144 /* >= 4 waves each sum <= k / 4 per int32 accumulator: 65536 * 128 * 128 = 2^30 */
int kt_hip_w12_linear(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                      int64_t n, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev, int out_kind,
                      void* y_dev, void* stream);

/* The same 12-bit weights as two balanced int8 digit planes (W12B), for the MFMA-bound products whose m gives every CU
 * a 256 x 128 tile (config 2 at m = 2048): hi = (v + 128) >> 8 in [-8, 8], lo = v - 256 hi in [-128, 127], so
 * v = lo + 256 hi with no offset term and the product needs no row sums of x and no nibble unpacking. Each plane is
 * fragment-tiled as the W12 lo plane (kt_hip_w12b_bytes: round_up(n, 32) * kp bytes each, 2 bytes per weight
 * together). kt_hip_w12b_linear: the same integers and out_kind semantics as kt_hip_w12_linear for every m and n
 * (always the DMA-fed 256 x 128 GEMM), k <= KT_W12_GEMM_MAX_K, m * kp and round_up(n, 32) * kp below 2^32. No
 * counterpart in the reference. */
void kt_hip_w12b_bytes(int64_t n, int64_t k, size_t* plane_bytes);
int kt_hip_w12b_pack(int dev, const int32_t* codes_dev, int64_t n, int64_t k, int8_t* lo_dev, int8_t* hi_dev,
                     void* stream);
int kt_hip_w12b_linear(int dev, const int8_t* x_dev, const int8_t* lo_dev, const int8_t* hi_dev, int64_t m,
                       int64_t n, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev, int out_kind,
                       void* y_dev, void* stream);

/* A pure read of bytes_n bytes (a multiple of 16, below 2^31) of src_dev with the W12 GEMV's load form (16-byte buffer
 * loads, 4 per thread in flight, KT_STREAM_READ_CTAS CTAs over contiguous chunks); out_dev (KT_STREAM_READ_CTAS
 * uint32, device) receives each chunk's XOR of 32-bit words. A measurement aid with no counterpart in the reference:
 * the time memory takes to deliver a weight matrix's bytes to this load form with no compute, beside the GEMVs that
 * stream the same bytes. */
#define KT_STREAM_READ_CTAS 256
int kt_hip_stream_read(int dev, const uint8_t* src_dev, int64_t bytes_n, uint32_t* out_dev, void* stream);

/* As kt_hip_w12_linear with out_kind KT_OUT_I8, then each int8 output q replaced by lut_dev[q + 127] (255 int8
 * entries, device): an activation-code table applied in the epilogue (the GELU of config 5's FeedForward,
 * crates/03-models/kt-model-vision/src/hiera.rs:336-340 with nonlin.rs:30-47, as an int8 code table).
 * 1 <= k <= 8128. */
int kt_hip_w12_linear_lut(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                          int64_t n, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev,
                          const int8_t* lut_dev, int8_t* y_dev, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * MoE layer of config 4 (GLM-4.5-Air shape), device-resident operands. Replaces the reference's per-token MoE path:
 * MoeMlp::route / topk (crates/01-engine/kt-core/src/layers.rs:800-851), the expert calls of
 * forward_int_with_experts (layers.rs:954-986) and MoeMlp::combine (layers.rs:893-923), with the shared expert of
 * layers.rs:757-780. Integer semantics (this build's int8 definition of that layer):
 *   route:   the top_k experts of token t by router code r[t, e] (descending, ties to the lower index), weight
 *            cw = sig[clamp(round_half_away(r / 16), -127, 127) + 127] (sig: 255 int16 sigmoid codes);
 *   expert:  gq, uq = int8 per-channel requant of the gate and up rows of x . WGU^T; h = clamp(requant(
 *            silu[gq + 127] * uq, 1, h_shift), +-127) (silu: 255 int16 codes); d = int8 per-channel requant of
 *            h . WD^T;
 *   combine: out = clamp(requant(sum_i cw_i d_i + 4096 d_shared, 1, out_shift), +-127).
 * Experts are groups 0..E-1, the shared expert is group E. Expert g's gate/up weights are the W12 planes of its
 * 2F x H matrix (rows 0..F-1 gate, F..2F-1 up) packed by kt_hip_w12_pack_gate_up, at gu_lo + g * gu_lo_bytes
 * (kt_hip_w12_bytes(2F, H)) and gu_nib + g * gu_lo_bytes / 2, scales (2F per group, natural order) at
 * gu_mant/gu_shift + g * 2F; its down weights are H x F planes at d_lo + g * d_lo_bytes (kt_hip_w12_bytes(H, F)),
 * scales at d_mant/d_shift + g * H. H and F are multiples of 64, at most 8128; 1 <= top_k <= min(E, 32); E + 1 <=
 * KT_MAX_GROUPS.
 * ------------------------------------------------------------------------------------------------------------- */
#define KT_MAX_GROUPS 1024
#define KT_EPI_I8 0     /* grouped GEMM epilogue: per-channel int8 requant */
#define KT_EPI_SWIGLU 1 /* grouped GEMM epilogue: SwiGLU over an interleaved gate/up matrix */

/* Pack a SwiGLU gate/up matrix (2*ffn x k i32 codes in [-2048, 2047], device: gate rows then up rows) into W12
 * planes with 32-row gate/up interleave (packed row block 2j = gate rows 32j.., 2j+1 = up rows 32j..), the layout
 * the SwiGLU epilogue reads. ffn is a multiple of 32. */
int kt_hip_w12_pack_gate_up(int dev, const int32_t* codes_dev, int64_t ffn, int64_t k, int8_t* lo_dev,
                            uint8_t* nib_dev, void* stream);

/* MoeMlp::route (layers.rs:826-851, sigmoid score as GLM-4.5's router.rs:29-79): logits T x E int32 (device) ->
 * sel (T x top_k expert ids) and cw (T x top_k weights). E <= 1024. */
int kt_hip_moe_route(int dev, const int32_t* logits_dev, int64_t tokens, int64_t experts, int top_k,
                     const int16_t* sig_dev, int32_t* sel_dev, int32_t* cw_dev, void* stream);

/* Bucket the routed tokens by expert: list ((E + 1) x T) holds group g's tokens in increasing order at
 * g * T .. g * T + count[g] - 1 (group E: every token), pos (T x top_k) each choice's row within its group. */
int kt_hip_moe_bucket(int dev, const int32_t* sel_dev, int64_t tokens, int64_t experts, int top_k,
                      int32_t* list_dev, int32_t* pos_dev, int32_t* count_dev, void* stream);

/* The ragged grouped W12 GEMM (the experts of forward_int_with_experts, layers.rs:954-986, run as one launch).
 * groups <= KT_MAX_GROUPS; group g has count[g] rows (sum <= max_rows); its row j is x row list[g * list_stride + j]
 * (list_dev non-null) or x row off[g] + j (off = exclusive prefix of count); x is x_rows x kp(k) int8. Group g's
 * weights: n x k W12 planes at lo_dev + g * lo_bytes(n, k) and nib_dev + g * lo_bytes / 2, scales mant/shift +
 * g * n. Output row j of group g is y row off[g] + j (row stride y_stride bytes). epilogue KT_EPI_I8: the n columns'
 * per-channel int8 requant; KT_EPI_SWIGLU: weights packed by kt_hip_w12_pack_gate_up (n = 2F), output F columns of
 * clamp(requant(silu[gq + 127] * uq, 1, h_shift)). off_dev (optional, groups + 1 int32) receives off. k <= 8128. */
int kt_hip_w12_grouped_linear(int dev, const int8_t* x_dev, int64_t x_rows, const int32_t* list_dev,
                              int64_t list_stride, const int32_t* count_dev, int64_t groups, int64_t max_rows,
                              const int8_t* lo_dev, const uint8_t* nib_dev, int64_t n, int64_t k,
                              const int32_t* mant_dev, const int32_t* shift_dev, int epilogue,
                              const int16_t* silu_dev, int h_shift, int8_t* y_dev, int64_t y_stride,
                              int32_t* off_dev, void* stream);

/* The SwiGLU MLP's gate/up product for a dense batch (SwiGluMlp::forward_int, crates/01-engine/kt-core/src/
 * layers.rs:609-640, with this build's int8 epilogue): x (m x kp(k) int8) against a gate/up matrix packed by
 * kt_hip_w12_pack_gate_up (2 ffn x k), y (m rows of stride y_stride int8) = clamp(requant(silu[gq + 127] * uq, 1,
 * h_shift)) with gq, uq the per-channel int8 requant of the gate and up rows (scales in natural order, 2 ffn).
 * m <= KT_W12_SKINNY_MAX_M runs the bandwidth-bound skinny kernel, longer batches the MFMA tile kernel.
 * ffn a multiple of 64, 1 <= k <= 8128. */
int kt_hip_w12_swiglu(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                      int64_t ffn, int64_t k, const int32_t* mant_dev, const int32_t* shift_dev,
                      const int16_t* silu_dev, int h_shift, int8_t* y_dev, int64_t y_stride, void* stream);

/* The decoder's one-token products with the RMSNorm before them fused in (RmsNorm then QuantLinear /
 * SwiGluMlp::forward_int, crates/01-engine/kt-core/src/model.rs:290-353, layers.rs:609-640): r_dev holds m
 * (1..KT_NORM_MAX_M) rows of the int32 residual, d values each; every CTA normalizes them into LDS with the rule of
 * kt_hip_dec_rmsnorm (rms = isqrt(floor(sum r^2 / d)), q = clamp(round_half_away(32 r / rms), +-127), 0 when
 * rms = 0) and then runs the product of kt_hip_w12_linear (out_kind KT_OUT_I64, KT_OUT_I32 or KT_OUT_I8) or of
 * kt_hip_w12_swiglu on those rows: the same integers as kt_hip_dec_rmsnorm followed by that call, one launch
 * instead of two. y_dev must not alias r_dev. d <= KT_NORM_MAX_D and m * kp(d) <= KT_NORM_LDS_BYTES. */
#define KT_NORM_MAX_M 16
#define KT_NORM_MAX_D 2048
#define KT_NORM_LDS_BYTES 65536
int kt_hip_w12_linear_norm(int dev, const int32_t* r_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                           int64_t n, int64_t d, const int32_t* mant_dev, const int32_t* shift_dev, int out_kind,
                           void* y_dev, void* stream);
int kt_hip_w12_swiglu_norm(int dev, const int32_t* r_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t m,
                           int64_t ffn, int64_t d, const int32_t* mant_dev, const int32_t* shift_dev,
                           const int16_t* silu_dev, int h_shift, int8_t* y_dev, int64_t y_stride, void* stream);

/* MoeMlp::combine (layers.rs:893-923) plus the shared expert: out (T x H int8) from d (rows in bucket order, H
 * columns), off (groups + 1, from the grouped GEMM), sel, cw, pos. */
int kt_hip_moe_combine(int dev, const int8_t* d_dev, const int32_t* off_dev, const int32_t* sel_dev,
                       const int32_t* cw_dev, const int32_t* pos_dev, int64_t tokens, int64_t hidden,
                       int64_t experts, int top_k, int out_shift, int8_t* out_dev, void* stream);

/* The workspace of kt_hip_moe_forward: total bytes and the byte offsets of its parts, in this order: sel, cw, pos
 * (T x top_k int32 each), list ((E + 1) x T int32), count (E + 1 int32), off (E + 2 int32), h (P x F int8) and
 * d (P x H int8), P = T * (top_k + 1). Every part is 256-byte aligned. */
#define KT_MOE_WS_PARTS 8
int kt_hip_moe_workspace(int64_t tokens, int64_t hidden, int64_t ffn, int64_t experts, int top_k, size_t* total,
                         size_t* offsets);

/* The whole layer (MoeMlp::forward_int_with_experts with the local experts, layers.rs:954-986): route, bucket,
 * gate/up grouped GEMM with the SwiGLU epilogue, down grouped GEMM, combine -- five launches on `stream`, no host
 * synchronization. x is T x H int8 (H a multiple of 64), logits T x E int32, out T x H int8; workspace as
 * kt_hip_moe_workspace describes (its intermediates stay readable after the call). */
int kt_hip_moe_forward(int dev, const int8_t* x_dev, const int32_t* logits_dev, int64_t tokens, int64_t hidden,
                       int64_t ffn, int64_t experts, int top_k, const int8_t* gu_lo_dev, const uint8_t* gu_nib_dev,
                       const int32_t* gu_mant_dev, const int32_t* gu_shift_dev, const int8_t* d_lo_dev,
                       const uint8_t* d_nib_dev, const int32_t* d_mant_dev, const int32_t* d_shift_dev,
                       const int16_t* silu_dev, const int16_t* sig_dev, int h_shift, int out_shift,
                       void* workspace_dev, int8_t* out_dev, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * SAM 2.1 image path of config 5, device-resident operands.
 * ------------------------------------------------------------------------------------------------------------- */
/* The patch-embed convolution (Conv2d::forward_int, crates/01-engine/kt-core/src/conv.rs:68-130, as PatchEmbed
 * uses it, crates/03-models/kt-model-vision/src/hiera.rs:165-190) as an im2col-fused W12 GEMM. img_dev holds the
 * u8 pixels [ci][h][w]; each pixel p of channel c enters as the int8 code lut_dev[c * 256 + p] (the entry
 * quantization of the normalized image, plugin.rs:38); taps outside the image contribute nothing. The weights are
 * the co x (ci * kh * kw) code matrix, k ordered (ic, ky, kx) as the reference's accumulation, packed by
 * kt_hip_sam_patch_pack / kt_hip_sam_patch_upload. out_dev [co][oh][ow] int8 receives
 * clamp(requant(acc + bias[c], mant[c], shift[c]), +-127) (bias_dev may be NULL; |bias| < 2^30).
 * oh = (h + 2 pad - kh) / stride + 1, likewise ow. Limits: ci <= 4, kw <= 16, ci * kh * kwp <= 256 (kwp = kw
 * rounded up to 4), and the staged image rows of 128 output positions fit 40.5 KiB: nc * rows * (stride * 127 / 4
 * + kwp / 4) dwords plus bank padding, nc = 4 / gcd(stride, 4), rows = ci * kh * kwp rounded up to 64, divided by
 * kwp (7 x 7 stride 4 over 3 channels: 13.5 KiB). Asynchronous on `stream`. */
int kt_hip_sam_patch_embed(int dev, const uint8_t* img_dev, const int8_t* lut_dev, int64_t ci, int64_t h, int64_t w,
                           const int8_t* lo_dev, const int8_t* hi_dev, int64_t co, int64_t kh, int64_t kw,
                           int64_t stride, int64_t pad, const int32_t* bias_dev, const int32_t* mant_dev,
                           const int32_t* shift_dev, int8_t* out_dev, void* stream);
/* Bytes of each of the two patch-embed weight planes for co x (ci * kh * kw) codes: co rounded up to 32 times
 * ci * kh * kwp rounded up to 64; both 0 when the shape has no layout (kw > 16, ci > 4). */
void kt_hip_sam_patch_bytes(int64_t co, int64_t ci, int64_t kh, int64_t kw, size_t* lo_bytes, size_t* hi_bytes);
/* Pack co x (ci * kh * kw) codes in [-2048, 2047] (device, the reference's [c_out][c_in][kh][kw] order) into the
 * patch-embed planes (device): int8 digits with code = lo + 256 hi (hi in [-8, 8]), each kernel row's taps padded
 * to kwp with zero codes, in the W12 fragment tiling. Codes outside the range give wrong planes. */
int kt_hip_sam_patch_pack(int dev, const int32_t* codes_dev, int64_t co, int64_t ci, int64_t kh, int64_t kw,
                          int8_t* lo_dev, int8_t* hi_dev, void* stream);
/* Check host codes (hipErrorInvalidValue if any is outside [-2048, 2047]), upload and pack them. */
int kt_hip_sam_patch_upload(int dev, const int32_t* codes, int64_t co, int64_t ci, int64_t kh, int64_t kw,
                            int8_t* lo_dev, int8_t* hi_dev);

/* ---------------------------------------------------------------------------------------------------------------
 * Decoder of config 3 (Qwen2.5-0.5B shape): the operations between the W12 GEMMs, device-resident operands. They
 * replace the reference decoder's host-side steps (DecoderModel::embed_int / blocks_int / head_int / decode_step,
 * crates/01-engine/kt-core/src/model.rs:168-188, 290-353; RmsNorm and Attention, attention.rs:347-480;
 * generate_greedy_by, generate.rs:82-111) with this build's int8 rules. Positions are read from pos_dev (the
 * position of row 0 of the call) so a captured decode step replays at every position; kt_hip_dec_advance moves it.
 * The q/k/v projection output is one row of nqkv = (nh + 2 nkv) hd int8 values per token: q heads, k heads, v heads.
 * ------------------------------------------------------------------------------------------------------------- */
/* r[t] = emb[tokens[t]] (int16 codes, the tied embedding) into the int32 residual rows (t < T, d wide). */
int kt_hip_dec_embed(int dev, const int32_t* tokens_dev, int64_t tokens, const int16_t* emb_dev, int64_t d,
                     int32_t* r_dev, void* stream);
/* RmsNorm to int8: rms = isqrt(floor(sum_i r_i^2 / d)), q_i = clamp(round_half_away(32 r_i / rms), +-127), 0 when
 * rms is 0. q rows have stride q_stride (>= d). */
int kt_hip_dec_rmsnorm(int dev, const int32_t* r_dev, int64_t tokens, int64_t d, int8_t* q_dev, int64_t q_stride,
                       void* stream);
/* Rotate-half RoPE of the q and k heads of each row in place at position p = pos + t (pairs i, i + hd/2:
 * a' = clamp(sr(a C - b S, 14)), b' = clamp(sr(b C + a S, 14)), sr = round-half-away shift, C/S = cos/sin tables
 * [max_pos][hd/2] int16 at 2^14), then the rotated k and the v heads into the layer's caches [max_pos][nkv][hd]. */
int kt_hip_dec_rope_kv(int dev, int8_t* qkv_dev, int64_t tokens, int64_t nqkv, const int32_t* pos_dev, int64_t nh,
                       int64_t nkv, int64_t hd, const int16_t* cos_dev, const int16_t* sin_dev, int8_t* kcache_dev,
                       int8_t* vcache_dev, void* stream);
/* Causal GQA attention with an integer softmax: head h of row t (kv head g = h / (nh / nkv)) attends positions
 * j <= p: s_j = q . k_j, m = max s_j, e_j = exp_tab[(m - s_j + 64) >> 7] (0 past its 1024 entries),
 * o = clamp(round_half_away(sum_j e_j v_j / sum_j e_j)). o is tokens x nh hd int8. hd = 64, max_pos <= 16384. */
int kt_hip_dec_attention(int dev, const int8_t* qkv_dev, int64_t tokens, int64_t nqkv, const int32_t* pos_dev,
                         const int8_t* kcache_dev, const int8_t* vcache_dev, int64_t nh, int64_t nkv, int64_t hd,
                         const int32_t* exp_tab_dev, int8_t* o_dev, int64_t max_pos, void* stream);
/* argmax_codes (generate.rs:48-56): token_dev[0] = the first index of the maximum of n int32 logits. With
 * record_dev non-null the logits are also copied to record_dev + step_dev[0] * n and step_dev[0] advances by one
 * (the per-step logits the generation hash covers). */
int kt_hip_dec_argmax(int dev, const int32_t* logits_dev, int64_t n, int32_t* token_dev, int32_t* record_dev,
                      int32_t* step_dev, void* stream);
/* pos_dev[0] += by. */
int kt_hip_dec_advance(int dev, int32_t* pos_dev, int64_t by, void* stream);
/* One decode step's attention (one row at p = pos) with its RoPE and KV append fused: the same integers as
 * kt_hip_dec_rope_kv followed by kt_hip_dec_attention with tokens = 1 (qkv_dev is read, not rotated in place). */
int kt_hip_dec_attention_step(int dev, const int8_t* qkv_dev, const int32_t* pos_dev, int8_t* kcache_dev,
                              int8_t* vcache_dev, int64_t nh, int64_t nkv, int64_t hd, const int16_t* cos_dev,
                              const int16_t* sin_dev, const int32_t* exp_tab_dev, int8_t* o_dev, int64_t max_pos,
                              void* stream);
/* The decode step's attention output projection spread over the calls around it (no separate counterpart in the
 * reference: its decode step runs attention and then the o QuantLinear, decoder.rs), three calls that together give
 * the integers of kt_hip_dec_attention_step, kt_hip_w12_linear (KT_OUT_I32_ADD, the o projection into the
 * residual r), kt_hip_w12_swiglu_norm (m = 1) and kt_hip_w12_linear (KT_OUT_I32_ADD, the down projection into r),
 * with one launch fewer:
 * 1. kt_hip_dec_attention_o_step: the attention step, then each head's CTA adds its 64 outputs' products with W_o
 *    (wo_lo_dev / wo_nib_dev: the d x (nh * hd) W12 planes, kt_hip_w12_bytes layout) into oacc_dev (d int32, the
 *    W12 dot sums before requantization), which must be zero on entry.
 * 2. kt_hip_w12_swiglu_norm_o: kt_hip_w12_swiglu_norm of the one residual row r + requant_o(oacc) (saturating;
 *    omant_dev / oshift_dev: the o projection's per-channel scales); r is not written.
 * 3. kt_hip_w12_linear_add_o: r[n] = sat(sat(r[n] + requant_o(oacc[n])) + requant(x . W[n])) for the one row x
 *    (the down projection), and oacc[n] = 0 again.
 * The three calls share oacc_dev and must not overlap other calls that use it. d <= 1024, nh * hd <= 8128,
 * k <= 8128. */
int kt_hip_dec_attention_o_step(int dev, const int8_t* qkv_dev, const int32_t* pos_dev, int8_t* kcache_dev,
                                int8_t* vcache_dev, int64_t nh, int64_t nkv, int64_t hd, const int16_t* cos_dev,
                                const int16_t* sin_dev, const int32_t* exp_tab_dev, int64_t max_pos,
                                const int8_t* wo_lo_dev, const uint8_t* wo_nib_dev, int64_t d, int32_t* oacc_dev,
                                void* stream);
int kt_hip_w12_swiglu_norm_o(int dev, const int32_t* r_dev, const int8_t* lo_dev, const uint8_t* nib_dev,
                             int64_t ffn, int64_t d, const int32_t* mant_dev, const int32_t* shift_dev,
                             const int16_t* silu_dev, int h_shift, int8_t* y_dev, const int32_t* oacc_dev,
                             const int32_t* omant_dev, const int32_t* oshift_dev, void* stream);
int kt_hip_w12_linear_add_o(int dev, const int8_t* x_dev, const int8_t* lo_dev, const uint8_t* nib_dev, int64_t n,
                            int64_t k, const int32_t* mant_dev, const int32_t* shift_dev, int32_t* y_dev,
                            int32_t* oacc_dev, const int32_t* omant_dev, const int32_t* oshift_dev, void* stream);
/* The greedy argmax in two stages for a replayable decode step. Stage 1: nparts CTAs reduce the n logits to nparts
 * keys (part_dev, uint64 each; the largest key is the first maximum), copy the logits to record_dev + step * n
 * (record_dev optional) and advance pos_dev by `advance` (pos_dev optional). Stage 2, fused with the next step's
 * embedding: token = the best key's index (written to token_dev when non-null), r_dev = emb[token], step += 1
 * (step_dev optional). */
int kt_hip_dec_argmax_part(int dev, const int32_t* logits_dev, int64_t n, uint64_t* part_dev, int64_t nparts,
                           int32_t* record_dev, const int32_t* step_dev, int32_t* pos_dev, int64_t advance,
                           void* stream);
int kt_hip_dec_embed_argmax(int dev, const uint64_t* part_dev, int64_t nparts, const int16_t* emb_dev, int64_t d,
                            int32_t* r_dev, int32_t* token_dev, int32_t* step_dev, void* stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Synthetic workload generators (host only, no GPU): the benchmark configs' integer samplers on the reference LCG
 * (apps/kt-demo/src/main.rs:19-22), multithreaded over the host cores. No counterpart in the reference.
 * ------------------------------------------------------------------------------------------------------------- */
/* n codes uniform in [-2048, 2047]: ((s >> 33) % 4096) - 2048 on the stream seeded seed ^ 0x9E3779B97F4A7C15. */
void kt_hip_gen_w12(uint64_t seed, size_t n, int32_t* out);
/* n values round_half_away(N(0, sigma)), clipped to +-clip when clip > 0: an Irwin-Hall sum of 12 draws
 * u = (s >> 33) & 0xFFFF on the stream seed ^ 0xD1B54A32D192ED03, t = 2 sum - 12 * 65535,
 * v = sign(t) * ((|t| sigma + 2^16) >> 17). */
void kt_hip_gen_gauss(uint64_t seed, int64_t sigma, int64_t clip, size_t n, int32_t* out);
/* n values uniform in [lo, hi]: ((s >> 33) % (hi - lo + 1)) + lo on the stream seed ^ 0x9E3779B97F4A7C15. */
void kt_hip_gen_uniform(uint64_t seed, int64_t lo, int64_t hi, size_t n, int32_t* out);
/* Per output channel of an n x k code matrix: to_i32(Scale::from_ratio(target, 4 * sigma * isqrt(sum_k w^2)))
 * (crates/00-kernels/kt-int/src/lib.rs:191-212), mapping 4 standard deviations of the accumulator (inputs of
 * standard deviation sigma) to target (127 for int8 outputs). */
void kt_hip_channel_scales(const int32_t* w, size_t n, size_t k, int64_t sigma, int64_t target, int32_t* mant,
                           int32_t* shift);
/* rows x cols 12-bit codes of a Gaussian matrix quantized per row: v = round(N(0, 2^20)) on kt_hip_gen_gauss's
 * stream, code = round_half_away(2047 v / max_row |v|). */
void kt_hip_gen_quant_rows(uint64_t seed, size_t rows, size_t cols, int32_t* out);

/* Test hook: one 32x32x32 and one 16x16x64 int8 MFMA on 64 lanes x 16 bytes of a_dev / b_dev; the raw accumulator
 * registers go to c32_dev (64 x 16 i32) and c16_dev (64 x 4 i32). */
int kt_hip_probe_mfma(int dev, const int8_t* a_dev, const int8_t* b_dev, int32_t* c32_dev, int32_t* c16_dev,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KT_HIP_H */
