/*
 * zg_hip.h — C ABI of the MI355X (gfx950) backend for zerogravity's Qwen3.5
 * GGUF decode/prefill path.
 *
 * Boundary A (per-region operator API).  Each zg_<region> entry point is the
 * device implementation of one optional method of the reference trait
 *   pub trait MatVecKernel: Send + Sync            core/src/accelerator.rs:682-731
 * and takes the same fields as the region struct it names, flattened into
 * (pointer, length) pairs of caller-owned host memory.  Outcomes map 1:1 to
 * the reference's three-way result (core/src/accelerator.rs:671-681):
 *   ZG_COMPLETED (0)   device work finished and read back (RegionExecution::Completed)
 *   ZG_UNSUPPORTED (1) region not offered; the caller may run its CPU path
 *                      (RegionExecution::Unsupported)
 *   < 0                error; the caller must abort the proposal, no fallback (Err)
 * A nonfinite device result is reported as ZG_E_STATE, never as Completed
 * (validate_completed, core/src/accelerator.rs:734-744).
 *
 * Device API (boundary for the whole-program path).  zg_weight_* and
 * zg_gemv_device operate on device-resident buffers and a caller stream; they
 * are what a RegionExecutionProvider (core/src/provider.rs:10-42) would build
 * its resident program on.
 *
 * Thread safety: every entry point taking a zg_ctx serialises on that ctx
 * (the reference trait is Send + Sync, accelerator.rs:682).
 * No torch types appear in this ABI; streams are hipStream_t passed as void*.
 */
#ifndef ZG_HIP_H
#define ZG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Outcomes.  Negative codes mirror Error::{Malformed, Unsupported, Resource,
 * Limit, State} of core/src/lib.rs:95-102 plus a device-runtime failure. */
enum {
    ZG_COMPLETED = 0,
    ZG_UNSUPPORTED = 1,
    ZG_E_MALFORMED = -1,
    ZG_E_UNSUPPORTED = -2,
    ZG_E_RESOURCE = -3,
    ZG_E_LIMIT = -4,
    ZG_E_STATE = -5,
    ZG_E_DEVICE = -6
};

/* ggml tensor type codes, core/src/encoding.rs:77-91 */
enum { ZG_F32 = 0, ZG_F16 = 1, ZG_Q8_0 = 8, ZG_Q4_K = 12, ZG_BF16 = 30 };

typedef struct zg_ctx zg_ctx;
typedef struct zg_weight zg_weight;

/* ---------------------------------------------------------------- context */

/* Create a context bound to one HIP device with its own default-priority
 * stream.  Returns ZG_COMPLETED or ZG_E_DEVICE. */
int zg_ctx_create(int device, zg_ctx** out);
void zg_ctx_destroy(zg_ctx* ctx);
/* Message for the last failing call on this ctx ("" if none).  Valid until
 * the next call on the ctx. */
const char* zg_last_error(const zg_ctx* ctx);
/* Version string of this library. */
const char* zg_version(void);

/* ---------------------------------------------------------------- weights */

/* Register (or find) the device copy of an immutable GGUF matrix.  The key is
 * (source_id, name, ggml_type, columns, rows), as the reference requires of
 * every resident cache (core/src/accelerator.rs:22-68); source_id 0 is the
 * reserved unbound identity and is refused (ZG_E_MALFORMED).  `bytes` holds
 * rows * row_bytes(columns) of GGUF blocks; a nonfinite block scale is
 * ZG_E_MALFORMED (artifacts/src/codecs/q8.rs:6-15, q4.rs:39-70).  Idempotent
 * per key: a repeated call returns the cached handle.  Replaces the per-call
 * upload implied by MatVecRegion::packed_weights (accelerator.rs:61-75). */
int zg_weight_register(zg_ctx* ctx, uint64_t source_id, const char* name, int ggml_type,
                       size_t columns, size_t rows, const void* bytes, size_t len,
                       zg_weight** out);
/* Drop every resident weight registered under source_id (model close). */
int zg_source_release(zg_ctx* ctx, uint64_t source_id);
/* Device bytes held by a registered weight (payload + headers). */
size_t zg_weight_device_bytes(const zg_weight* w);

/* Exact dequantization of a registered weight into caller host memory,
 * out[rows * columns] f32, bit-identical to the reference codecs
 * (artifacts/src/codecs/mod.rs:36-88). */
int zg_weight_dequantize(zg_ctx* ctx, const zg_weight* w, float* out, size_t out_len);

/* ------------------------------------------------------- boundary A regions */

/* MatVecRegion (core/src/accelerator.rs:61-75) -> MatVecKernel::try_execute
 * (:683).  Q8_0 runs against the dynamic Q8_0 activation coding
 * (cpu/src/source/quantization.rs:37-61,171-196); Q4_K against the f32
 * activation (dot_row, cpu/src/source.rs:431-459; the reference CPU itself
 * refuses Q4_K at source.rs:265-270); F32 as an f32 dot.  For a bound
 * source_id the device weight is cached under its key; source_id 0 uploads
 * for this call only.  out[rows]. */
int zg_matvec(zg_ctx* ctx, uint64_t source_id, const char* tensor_name, int ggml_type,
              size_t columns, size_t rows, const void* packed_weights, size_t packed_len,
              const float* activation, size_t activation_len, float* out, size_t out_len);

/* EmbeddingRegion (accelerator.rs:417-453) -> try_embedding: dequantize row
 * `token` of a [vocabulary, width] GGUF matrix. out[width]. */
int zg_embedding(zg_ctx* ctx, uint64_t source_id, const char* tensor_name, int ggml_type,
                 const void* packed_weights, size_t packed_len, uint32_t token, size_t width,
                 size_t vocabulary, float* out, size_t out_len);

/* RmsNormRegion (accelerator.rs:77-88) -> try_rms_norm; semantics of
 * source_rms_normalize (model-qwen35/src/lib.rs:263-284). out[n]. */
int zg_rms_norm(zg_ctx* ctx, const float* input, const float* weights, size_t n, float eps,
                float* out);

/* GroupedRmsNormRegion (accelerator.rs:90-104) -> try_grouped_rms_norm;
 * source_grouped_rms_normalize (lib.rs:289-306). out[group_width*groups]. */
int zg_grouped_rms_norm(zg_ctx* ctx, const float* input, const float* weights, size_t group_width,
                        size_t groups, float eps, float* out);

/* SiluRegion (accelerator.rs:509-530) -> try_silu; source_silu (lib.rs:310-321)
 * with the GGML polynomial exp (cpu/src/ops.rs:317-355).  multiplier may be
 * NULL. out[n]. */
int zg_silu(zg_ctx* ctx, const float* input, const float* multiplier, size_t n, float* out);

/* BinaryRegion (accelerator.rs:383-416) -> try_binary; source_binary
 * (lib.rs:1258-1271).  kind 0 = Add, 1 = SigmoidGate. out[n]. */
int zg_binary(zg_ctx* ctx, int kind, const float* left, const float* right, size_t n, float* out);

/* ------------------------------------------------------------- device API */

/* y[M][rows] = W . rmsnorm(x)[M][columns] on device memory, the fused
 * dequant-GEMV/skinny-GEMM of the decode path.  x is bf16 (x_dtype ZG_BF16)
 * or f32 (ZG_F32), row-major [M][columns]; gamma (device, [columns]) applies
 * the RMSNorm prologue of lib.rs:263-284 when non-NULL; y is f32.  Runs on
 * `stream` (hipStream_t) or the ctx stream when NULL; asynchronous.  M <= 64.
 * No counterpart in the reference beyond MatVecKernel::try_execute; this is
 * the resident form the whole-program provider uses. */
int zg_gemv_device(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows,
                   const float* gamma, float eps, float* y, void* stream);

/* Only the GEMV kernel of zg_gemv_device, on activations already prepared by
 * zg_act_prepare_device (for timing the kernel alone).  For Q8_0 pass the
 * codes/scales, for Q4_K and F32 the f32 activation. */
int zg_act_prepare_device(zg_ctx* ctx, const void* x, int x_dtype, size_t m_rows, size_t columns,
                          const float* gamma, float eps, float* xf, int8_t* codes, float* scales,
                          void* stream);
int zg_gemv_prepared_device(zg_ctx* ctx, const zg_weight* w, size_t m_rows, const float* xf,
                            const int8_t* codes, const float* scales, float* y, void* stream);

#ifdef __cplusplus
}
#endif
#endif
