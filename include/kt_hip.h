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
 * 12-bit-weight path (BASELINE workloads), device-resident operands. No counterpart in the reference: there the
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

/* Test hook: one 32x32x32 and one 16x16x64 int8 MFMA on 64 lanes x 16 bytes of a_dev / b_dev; the raw accumulator
 * registers go to c32_dev (64 x 16 i32) and c16_dev (64 x 4 i32). */
int kt_hip_probe_mfma(int dev, const int8_t* a_dev, const int8_t* b_dev, int32_t* c32_dev, int32_t* c16_dev,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KT_HIP_H */
