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
 * (the reference trait is Send + Sync, accelerator.rs:682), and failure
 * text is kept per calling thread (zg_last_error).
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
enum { ZG_F32 = 0, ZG_F16 = 1, ZG_Q4_1 = 3, ZG_Q8_0 = 8, ZG_Q4_K = 12, ZG_Q6_K = 14, ZG_BF16 = 30 };

typedef struct zg_ctx zg_ctx;
typedef struct zg_weight zg_weight;

/* ---------------------------------------------------------------- context */

/* Create a context bound to one HIP device with its own default-priority
 * stream.  Returns ZG_COMPLETED or ZG_E_DEVICE. */
int zg_ctx_create(int device, zg_ctx** out);
void zg_ctx_destroy(zg_ctx* ctx);
/* Message of the calling thread's last failing call on this ctx ("" if
 * none).  Valid until that thread's next failing call on the ctx. */
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
/* Release the handles registered under source_id (model close).  A weight
 * that a loaded model (zg_model_load) still uses stays resident until the
 * last such model is destroyed; models take their own references, so
 * destroying one model never frees a weight another model or a registered
 * handle uses. */
int zg_source_release(zg_ctx* ctx, uint64_t source_id);
/* Device bytes held by a registered weight (payload + headers). */
size_t zg_weight_device_bytes(const zg_weight* w);

/* Exact dequantization of a registered weight into caller host memory,
 * out[rows * columns] f32, bit-identical to the reference codecs
 * (artifacts/src/codecs/mod.rs:36-88). */
int zg_weight_dequantize(zg_ctx* ctx, const zg_weight* w, float* out, size_t out_len);

/* ------------------------------------------------------- boundary A regions */

/* greedy_finite (core/src/numerics.rs:124-140) on the device: for each of
 * `rows` rows of n logits (host, row-major), the index of the first maximum
 * (ties, +0 vs -0 included, keep the lower index).  A nonfinite logit is
 * ZG_E_STATE; n == 0 is ZG_E_LIMIT.  out[rows].  The decode step's greedy
 * readout runs the same kernels. */
int zg_greedy(zg_ctx* ctx, const float* logits, size_t rows, size_t n, uint32_t* out);

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

/* GdnConvRegion (accelerator.rs:106-117) -> try_gdn_conv; gdn_conv_step
 * (cpu/src/ops/gdn.rs:7-44): raw_out[channels] and history_out[channels*3]
 * (oldest -> newest per channel); weights [channels][4]. */
int zg_gdn_conv(zg_ctx* ctx, const float* activation, const float* weights, const float* history,
                size_t channels, float* raw_out, float* history_out);

/* GdnCoefficientRegion (accelerator.rs:135-189) -> try_gdn_coefficients;
 * source_gdn_coefficients (model-qwen35/src/lib.rs:339-362).  The caller
 * attaches the immutable `scale` to each head's coefficients. */
int zg_gdn_coefficients(zg_ctx* ctx, const float* alpha, const float* beta, const float* dt, const float* a,
                        size_t heads, float scale, float* gain_out, float* beta_out, float* softplus_out,
                        float* gate_raw_out);

/* GdnRecurrentRegion (accelerator.rs:592-633) -> try_gdn_recurrent;
 * source_gdn_recurrent_step per head (lib.rs:1446-1499).  q, k, v [heads][width];
 * coefficients [heads][3] = {gain, beta, scale}; state value-major
 * [heads][width][width].  Offered for width 128. */
int zg_gdn_recurrent(zg_ctx* ctx, size_t width, size_t heads, const float* q, const float* k, const float* v,
                     const float* coefficients, const float* state, float* output, float* state_out);

/* Chunked (WY/UT) GDN prefill over one chunk: replaces
 * numerics/torch_cpu/gdn/chunk/core.rs:69-274 (`core(ChunkInputs)`), with
 * its checks (:86-116).  rows 1..64; heads a multiple of 16, at most 48;
 * query/key/value [rows][heads][128] and beta [rows][heads] bf16-exact f32;
 * beta in [0, 1]; log_decay [rows][heads] finite and <= 0; previous_state
 * key-major [heads][128 key][128 value] or NULL for zero.  output_bf16
 * [rows][heads][128] is the core output rounded to bf16 (gdn.rs:69-76);
 * state_out key-major.  ZG_E_MALFORMED on a failed check. */
int zg_gdn_chunk(zg_ctx* ctx, size_t rows, size_t heads, const float* query, const float* key, const float* value,
                 const float* beta, const float* log_decay, const float* previous_state, float* output_bf16,
                 float* state_out);

/* One GDN layer's decode step for `rows` sequences on device buffers and the
 * caller's stream: the causal conv (cpu/src/ops/gdn.rs:7-44) over a 4-slot
 * ring per channel, SiLU, two-stage q/k L2 (forward.rs:564-576), gates
 * (lib.rs:339-362) and the recurrence (lib.rs:1446-1499), i.e. gdn_layer
 * (forward.rs:518-632) up to the gated norm.  Replaces the per-token
 * GdnConvRegion + GdnRecurrentRegion pair (accelerator.rs:592-633) for a
 * resident state.  proj [rows][proj_stride]: [qkv (3W) | z (W) | alpha (H) |
 * beta (H)], W = 128 heads; conv_w [3W][4] (the GGUF ssm_conv1d layout);
 * ring [rows][3W][4]: the token at position p lives in slot p % 4;
 * positions [rows]; dt, ssm_a [heads]; state [rows][heads][128 v][128 k];
 * core [rows][W] = o / sqrt(128). */
int zg_gdn_decode_device(zg_ctx* ctx, size_t rows, size_t heads, const float* proj, size_t proj_stride,
                         const float* conv_w, float* ring, const int32_t* positions, const float* dt,
                         const float* ssm_a, float eps, float* state, float* core, void* stream);

/* The batched-rows form of zg_gdn_decode_device (one workgroup per head and
 * row, the kernel the decode step uses above 4 rows): the same core and
 * state, plus ssm_out's activation -- the gated RMSNorm of each head's core
 * with gamma norm[128], times silu(z) (forward.rs:586-594) -- rounded to f16
 * into `tiles` in the batched projections' MFMA A-operand order, W =
 * heads*128, rows padded to 32 (zg_gdn_decode_tiles_bytes).  With rows < 256
 * and W a multiple of 1024 up to 6144 (the 16-row decode kernel's layout),
 * element (row m, channel k) is at f16 index ((((m/16)*(W/128) + k/128)*4 +
 * 2*((k/32)%2) + (k/8)%2)*64 + m%16 + 16*((k/16)%2 + 2*((k/64)%2)))*8 + k%8;
 * otherwise at ((((m/32)*(W/256) + k/256)*16 + (k%256)/16)*64 +
 * ((k%16)/8)*32 + m%32)*8 + k%8.  heads even. */
size_t zg_gdn_decode_tiles_bytes(size_t rows, size_t heads);
int zg_gdn_decode_gated_device(zg_ctx* ctx, size_t rows, size_t heads, const float* proj, size_t proj_stride,
                               const float* conv_w, float* ring, const int32_t* positions, const float* dt,
                               const float* ssm_a, const float* norm, float eps, float* state, float* core,
                               void* tiles, void* stream);

/* One attention layer's decode step for `rows` sequences on device buffers
 * and the caller's stream: attention_layer (forward.rs:634-755) between its
 * projections -- head RMSNorm of q and k (:680-695), RoPE on the first 64
 * dimensions from each row's position (lib.rs:1552-1577), K/V appended at
 * that position (host_math.rs:1055-1064, rounded to the cache type), scores
 * (lib.rs:1427-1441, x 1/16), softmax (lib.rs:1352-1387), values
 * (lib.rs:1276-1305) and the sigmoid gate (forward.rs:751).  Replaces the
 * per-token RoPE/QK/softmax/value regions for a resident KV cache.
 * head_dim 256, q_heads / kv_heads <= 4.  proj [rows][proj_stride] =
 * [q | gate] per query head (2 x 256 each), then k (kv_heads x 256), then v;
 * kcache, vcache [rows][max_ctx][kv_heads x 256] of kv_dtype (ZG_BF16 or
 * ZG_F32); positions [rows], each < max_ctx; workspace of
 * zg_attn_decode_workspace_bytes(rows, q_heads, max_ctx) bytes (scores and
 * softmax statistics); out [rows][q_heads x 256].  A degenerate softmax sum
 * raises the context's device flag.  Asynchronous. */
size_t zg_attn_decode_workspace_bytes(size_t rows, size_t q_heads, size_t max_ctx);
int zg_attn_decode_device(zg_ctx* ctx, size_t rows, size_t q_heads, size_t kv_heads, const float* proj,
                          size_t proj_stride, const float* q_norm, const float* k_norm, float eps, float theta_scale,
                          const int32_t* positions, void* kcache, void* vcache, size_t max_ctx, int kv_dtype,
                          void* workspace, float* out, void* stream);

/* The same attention layer in split-T form for 1..64 rows, as the decode
 * step of an all-Q4_K model runs it: each of ~128 or more workgroups scores one span
 * of a row's tokens and keeps the span's max, sum of exp and exp-weighted
 * values; a second launch combines the spans and applies the gate.  The
 * operations are the reference's regrouped (no counterpart in the reference:
 * it normalises with the global max and sums values in token order), so the
 * output agrees to f32 rounding rather than bit for bit; K/V are appended
 * exactly as above.  Same arguments, with a workspace of
 * zg_attn_decode_split_workspace_bytes(rows, q_heads, kv_heads, max_ctx)
 * bytes; ZG_E_LIMIT beyond 64 rows or beyond 262144 cached tokens. */
size_t zg_attn_decode_split_workspace_bytes(size_t rows, size_t q_heads, size_t kv_heads, size_t max_ctx);
int zg_attn_decode_split_device(zg_ctx* ctx, size_t rows, size_t q_heads, size_t kv_heads, const float* proj,
                                size_t proj_stride, const float* q_norm, const float* k_norm, float eps,
                                float theta_scale, const int32_t* positions, void* kcache, void* vcache,
                                size_t max_ctx, int kv_dtype, void* workspace, float* out, void* stream);

/* Multi-chunk prefill on device buffers and the caller's stream (the same
 * kernels as zg_gdn_chunk; no reference counterpart takes more than one
 * chunk per call, core.rs:89).  Chunks of 64 tokens in order; query, key,
 * value, output [tokens][heads][128] f32; beta, log_decay [tokens][heads];
 * state value-major [heads][128 value][128 key] (the decode recurrence's
 * layout, lib.rs:81-83), updated in place; output f32 before rounding.
 * Inputs are not inspected on the host.  zg_gdn_chunk_scratch_bytes is the
 * size of the context-owned record buffer a call of this size uses.
 * ZG_E_LIMIT when (tokens + 64) * heads * 512 bytes reaches 4 GiB. */
size_t zg_gdn_chunk_scratch_bytes(size_t tokens, size_t heads);
int zg_gdn_chunk_prefill_device(zg_ctx* ctx, size_t tokens, size_t heads, const float* query, const float* key,
                                const float* value, const float* beta, const float* log_decay, float* state,
                                float* output, void* stream);

/* RopeKvRegion (accelerator.rs:205-296) -> try_rope_kv; source_rope_kv
 * (lib.rs:1552-1577).  Returns the rotated query and key and the unchanged
 * value slab. */
int zg_rope_kv(zg_ctx* ctx, const float* query, const float* key, const float* value, size_t head_width,
               size_t query_heads, size_t kv_heads, size_t rotate, size_t position, float theta_scale,
               float* query_out, float* key_out, float* value_out);

/* AttentionQkRegion (accelerator.rs:302-362) -> try_attention_qk;
 * source_attention_qk (lib.rs:1427-1441).  keys [tokens][kv_heads*head_width];
 * dots and scores [query_heads][tokens]. Offered for head width 256. */
int zg_attention_qk(zg_ctx* ctx, const float* query, const float* keys, size_t tokens, size_t head_width,
                    size_t query_heads, size_t kv_heads, float scale, float* dots, float* scores);

/* AttentionSoftmaxRegion (accelerator.rs:368-453) -> try_attention_softmax;
 * source_attention_softmax (lib.rs:1352-1387). probabilities [heads][width]. */
int zg_attention_softmax(zg_ctx* ctx, const float* scores, size_t heads, size_t width, float* probabilities);

/* AttentionValueRegion (accelerator.rs:450-500) -> try_attention_value;
 * source_attention_value (lib.rs:1276-1305); the reference's +0 padding of
 * the FMA schedule has no arithmetic effect beyond the sign of an exact zero.
 * values [tokens][kv_heads*head_width]; out [query_heads][head_width]. */
int zg_attention_value(zg_ctx* ctx, const float* probabilities, const float* values, size_t tokens,
                       size_t head_width, size_t query_heads, size_t kv_heads, float* out);

/* --------------------------------------------- boundary B: whole program */

/* Replaces RegionExecutionProvider::prepare(ModelProgram) for the Qwen3.5
 * GGUF forward plan (core/src/provider.rs:10-42, engine/src/prepare.rs:11-26):
 * the model is loaded once from a tensor table (names and GGML shapes of
 * model-qwen35/src/source/binding.rs:43-91, checked as in
 * LoadedQwenModel::from_checked_source, lib.rs:386-507) and sessions run
 * forward::forward_token (forward.rs:451-755) on the device. */
typedef struct zg_model zg_model;
typedef struct zg_session zg_session;

typedef struct zg_tensor_desc {
    const char* name;  /* GGUF tensor name, e.g. "blk.0.attn_qkv.weight" */
    int ggml_type;     /* ZG_F32, ZG_Q8_0, ZG_Q4_K, ZG_Q4_1 or ZG_Q6_K */
    uint64_t shape0;   /* GGML ne0: inner (columns / vector length) */
    uint64_t shape1;   /* GGML ne1: rows (1 for vectors) */
    const void* data;  /* host bytes, only read during zg_model_load */
    uint64_t nbytes;
} zg_tensor_desc;

typedef struct zg_geometry { /* ModelGeometry, model-qwen35/src/config.rs:51-182 */
    uint32_t hidden, layers, ffn, vocab;
    uint32_t gdn_heads, gdn_dim;          /* linear_num_value_heads, head width (128) */
    uint32_t q_heads, kv_heads, head_dim; /* full attention (head_dim 256) */
    uint32_t full_attention_interval;     /* layer i is full attention iff (i+1) % interval == 0 */
    uint32_t max_context;
    float eps;                            /* 1e-6 (lib.rs:505) */
} zg_geometry;

/* Numerical profiles a ForwardPlan carries, in the order of
 * ProgramNumericalProfile (core/src/numerics.rs:30-40). */
enum {
    ZG_PROFILE_GGUF_SOURCE_V1 = 0,
    ZG_PROFILE_TORCH_CPU_BF16_AVX2_MIXED_SOURCE_V1 = 1,
    ZG_PROFILE_SOURCE_CUDA_SM86_BF16_V1 = 2,
    ZG_PROFILE_ANALYTIC_F32_TEXT_V1 = 3,
    ZG_PROFILE_DIRECT_GAMMA_BF16_TEXT_CANDIDATE_V1 = 4
};

/* Admission of a plan before any device work: whether its numerical profile
 * (ForwardPlan::numerical_profile, core/src/accelerator/program/
 * source_program.rs:1178) and tensor table are the schedule this backend
 * runs.  Only ZG_PROFILE_GGUF_SOURCE_V1 is, as LoadedQwenModel::
 * require_execution_profile admits only GgufSourceV1 (model-qwen35/src/
 * source/binding.rs:363-371); a provider prepares whatever plan it is given
 * (core/src/provider.rs:38-42), so the refusal is made here.  Host only: no
 * context, no device.  ZG_COMPLETED; ZG_E_UNSUPPORTED for another profile,
 * a geometry outside the schedule or a codec the role's kernels do not
 * take; ZG_E_MALFORMED for a missing tensor, a shape that differs from the
 * geometry or a wrong packed length.  The reason goes to msg (msg_len bytes,
 * NUL-terminated; may be NULL).  zg_model_load applies the same check. */
int zg_model_admit(int profile, const zg_geometry* geometry, const zg_tensor_desc* tensors, size_t n_tensors,
                   char* msg, size_t msg_len);
int zg_model_load(zg_ctx* ctx, uint64_t source_id, const zg_geometry* geometry, const zg_tensor_desc* tensors,
                  size_t n_tensors, zg_model** out);
void zg_model_destroy(zg_model* model);

/* A session holds max_batch independent rows (continuous batch), each with
 * its own position, GDN conv/recurrent state and KV cache (kv_dtype ZG_BF16
 * or ZG_F32) of max_context tokens.  QwenDenseCpu's per-session state
 * (lib.rs:76-150). */
int zg_session_create(zg_model* model, size_t max_batch, size_t max_context, int kv_dtype, zg_session** out);
void zg_session_destroy(zg_session* s);
/* All rows back to position 0 with zero state (QwenDenseCpu::reset). */
int zg_session_reset(zg_session* s);
int zg_session_position(const zg_session* s, size_t row);
/* Continuous-batch row management over the session's contiguous per-row
 * slots (the reference keeps private per-row state in cohorts,
 * resident_inference.rs:1101-1111, and shares prompt prefixes through
 * paged block tables, core/src/paged_state.rs:239-330).  reset_row retires
 * one row (state and KV zeroed, position 0).  copy_row gives row dst a copy
 * of row src's state, KV prefix and position: retiring row r of a batch of
 * n active rows is copy_row(r, n-1) + reset_row(n-1), which keeps the active
 * rows dense for zg_decode_step; copying a prefilled row forks its prompt.
 * ZG_E_LIMIT for a row outside the batch. */
int zg_session_reset_row(zg_session* s, size_t row);
int zg_session_copy_row(zg_session* s, size_t dst, size_t src);

/* Publication.  Every state-changing call is a transaction over rows
 * [0, rows) (or its one row): it either completes and publishes, or fails
 * and leaves every row's position, conv history, GDN state and KV prefix
 * bit-identical to before (QwenDenseCpu: next_logits works on a draft,
 * commit publishes it, prefill_transaction installs its state only if every
 * token succeeds; lib.rs:1057-1070, 1114-1187, 1211-1225).  A failure that
 * leaves the device state unknown (a HIP launch error, ZG_E_DEVICE) poisons
 * the session: every row is marked unknown, and the session refuses work
 * until each marked row has been reset (zg_session_reset_row), restored or
 * imported, or the whole session reset.
 *
 * One forward_token for rows [0, rows): tokens[rows] host ids, logits
 * [rows][vocab] and/or greedy [rows] (first maximum, numerics.rs:126-140)
 * written to host memory when non-NULL.  Each row advances one position
 * (QwenDenseCpu::forward = next_logits + commit, lib.rs:1227-1232).  A
 * nonfinite layer or logit is ZG_E_STATE and publishes nothing. */
int zg_decode_step(zg_session* s, size_t rows, const uint32_t* tokens, float* logits, uint32_t* greedy);
/* QwenDenseCpu::next_logits (lib.rs:1057-1070): the step's logits/greedy
 * on a draft; nothing is published until zg_session_commit.  Any other
 * state-changing call on the session drops the proposal. */
int zg_session_propose(zg_session* s, size_t rows, const uint32_t* tokens, float* logits, uint32_t* greedy);
/* QwenDenseCpu::commit (lib.rs:1211-1225): publish the pending proposal.
 * ZG_E_STATE when there is none (never made, already committed, or dropped). */
int zg_session_commit(zg_session* s);
/* n tokens per row (tokens[row*n + t]), logits of the last only
 * (QwenDenseCpu::prefill_transaction, lib.rs:1119-1187); atomic over the
 * call. */
int zg_prefill(zg_session* s, size_t rows, size_t n, const uint32_t* tokens, float* logits);
/* n tokens of one row at once (QwenDenseCpu::prefill_transaction,
 * lib.rs:1119-1187, computed layer by layer over the whole prompt: batched
 * MFMA projections, the chunked GDN prefill (gdn/chunk.rs), causal attention
 * appending to the KV cache).  Logits of the last token to host when
 * non-NULL.  Same functions as zg_prefill in another order of summation;
 * needs Q4_K projections (ZG_E_UNSUPPORTED otherwise).  Atomic: a failure
 * leaves the row's published state as it was, and the other rows' state and
 * positions untouched.  ZG_E_LIMIT when an operand of the prompt's
 * projections would reach 4 GiB (32-bit offsets: 32-row f16 activation
 * tiles of n x K, e.g. n >= 349,526 at K = 6144), or when the chunked GDN
 * prefill's output would (zg_gdn_chunk_prefill_device); split such a
 * prompt over several calls. */
int zg_prefill_batched(zg_session* s, size_t row, size_t n, const uint32_t* tokens, float* logits);
/* Device-side step: d_tokens/d_logits/d_greedy are device pointers, no host
 * synchronisation.  The step's last kernel publishes it only if the status
 * word is clear, so after a failure every later queued step is a no-op on
 * the published state until the failure is read: zg_session_check (or the
 * next host-synchronous call on the session) waits for the queued steps,
 * reports the failure and clears it.  One captured graph is kept per
 * (rows, d_tokens, d_logits, d_greedy); reuse the same buffers every step
 * (at most 16 graphs are cached, the least recently used is rebuilt). */
int zg_decode_step_device(zg_session* s, size_t rows, const uint32_t* d_tokens, float* d_logits, uint32_t* d_greedy,
                          void* stream);
int zg_session_check(zg_session* s, void* stream);

/* Device-side snapshot of one row's published state (conv history, GDN
 * state, KV prefix, position), the resident form of
 * ResidentSession::snapshot / restore (gpu/src/resident_inference.rs:2766,
 * 3258).  restore puts it into any row of any session of the same model
 * with the same KV cache type (a fork when the row differs); a snapshot of
 * another model is ZG_E_STATE ("foreign"), one longer than the session's
 * context ZG_E_LIMIT.  Snapshots own device memory until destroyed. */
typedef struct zg_snapshot zg_snapshot;
int zg_session_snapshot(zg_session* s, size_t row, zg_snapshot** out);
int zg_session_restore(zg_session* s, size_t row, const zg_snapshot* snap);
size_t zg_snapshot_bytes(const zg_snapshot* snap);
int zg_snapshot_position(const zg_snapshot* snap);
void zg_snapshot_destroy(zg_snapshot* snap);

/* State domains of one row in the reference order (lib.rs:112-150): per layer,
 * GDN conv history then recurrent state (value-major), or attention keys then
 * values (token-major, f32). */
size_t zg_state_floats(const zg_session* s, size_t row);
int zg_state_export(zg_session* s, size_t row, float* out, size_t n);
/* The row takes the image and position (published GDN half 0), or on a
 * refusal (length, nonfinite value) or an allocation failure nothing
 * changes; a device copy failing midway poisons the session. */
int zg_state_import(zg_session* s, size_t row, const float* in, size_t n, int position);
/* Seeded synthetic prefix for benchmarking: rows [0, rows) get `prefix`
 * random tokens of KV (N(0,1)), recurrent state N(0,0.02) and conv history
 * N(0,0.5), and position `prefix`.  No reference counterpart. */
int zg_session_fill_random(zg_session* s, size_t rows, size_t prefix, uint64_t seed);

/* ------------------------------------------------------------- device API */

/* y[M][rows] = W . rmsnorm(x)[M][columns] on device memory, the fused
 * dequant-GEMV/skinny-GEMM of the decode path.  x is bf16 (x_dtype ZG_BF16)
 * or f32 (ZG_F32), row-major [M][columns]; gamma (device, [columns]) applies
 * the RMSNorm prologue of lib.rs:263-284 when non-NULL; y is f32.  Runs on
 * `stream` (hipStream_t) or the ctx stream when NULL; asynchronous.  M <= 64
 * for bf16 activations, M <= 65536 for f32.  f32 activations run the decode
 * step's own kernels: the prologue inside the GEMV (Q8_0, Q4_1, Q6_K and F32
 * bit-identical to the CPU at any M; Q4_K for one row, on the int8 matrix
 * cores; Q8_0 and Q6_K beyond 4 rows code each activation row once and
 * stream the weights once per 16 rows), and for Q4_K with M >= 2 the activation rounded to f16 and an f16
 * MFMA GEMM (f32 accumulate; within 1e-3 relative of the CPU), LDS-staged
 * for prompt-sized M >= 1024.
 * No counterpart in the reference beyond MatVecKernel::try_execute; this is
 * the resident form the whole-program provider uses. */
int zg_gemv_device(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows,
                   const float* gamma, float eps, float* y, void* stream);

/* Prologue and epilogue forms of the decode step's projections. */
enum { ZG_PRO_RMS = 0, ZG_PRO_GATED = 1, ZG_PRO_SILU_MUL = 2, ZG_PRO_PLAIN = 3, ZG_PRO_GATED_PRE = 5 };
enum { ZG_EPI_STORE = 0, ZG_EPI_RESID = 1, ZG_EPI_GLU = 2 };

/* One projection of the resident decode step with the operations around it
 * fused, for 1..4 f32 activation rows x[m][0:K] (device memory, row stride
 * ldx; the caller's stream, asynchronous), on the kernels the step itself
 * launches for one row and for rows of the codecs other than Q4_K (a
 * step's 2-4 Q4_K rows take its batched f16 kernels instead):
 *   prologue ZG_PRO_RMS       RMSNorm(x, gamma, eps) (model-qwen35/src/lib.rs:263-284)
 *            ZG_PRO_GATED     grouped RMSNorm(x, gamma[group], eps) * silu(x2) (forward.rs:586-594)
 *            ZG_PRO_SILU_MUL  x2 * silu(x) (forward.rs:498)
 *            ZG_PRO_PLAIN     x
 *            ZG_PRO_GATED_PRE ZG_PRO_GATED with the product (x * gamma[i % group])
 *                             * silu(z) already formed by the producer in x2
 *                             (x the norm input); one row of a Q4_K weight
 *                             with K a multiple of 512, group 128 -- the
 *                             one-row step's ssm_out, after the GDN kernel
 *   epilogue ZG_EPI_STORE     y = W a
 *            ZG_EPI_RESID     y = y + W a, the residual add (forward.rs:489,501)
 *            ZG_EPI_GLU       w stacks [gate | up] (N even): y[0:N/2] = up * silu(gate)
 * For one row also: `embedding` (a Q4_K token_embd of width K) with `token`
 * (device, one id): the activation is that token's embedding row,
 * dequantised in the prologue and also stored at x (the step's residual
 * stream; ZG_PRO_RMS); `greedy_max`/`greedy_idx` (device,
 * zg_gemv_greedy_parts(w) entries; ZG_PRO_RMS with ZG_EPI_STORE): each
 * workgroup's largest output and its first index (greedy_finite,
 * core/src/numerics.rs:126-140, over the workgroup's outputs).  The
 * arithmetic is the decode step's (Q4_K within 1e-3 relative of the CPU,
 * the other codecs bit-identical).  ZG_UNSUPPORTED for a shape without
 * such a kernel.  No counterpart in the reference beyond the regions it
 * fuses; the form a whole-program provider composes its step from. */
int zg_gemv_device_fused(zg_ctx* ctx, const zg_weight* w, size_t m_rows, int prologue, int epilogue, float* x,
                         size_t ldx, const float* x2, size_t ldx2, const float* gamma, float eps, size_t group,
                         float* y, size_t ldy, const zg_weight* embedding, const uint32_t* token, float* greedy_max,
                         int32_t* greedy_idx, void* stream);
/* Workgroup partials zg_gemv_device_fused leaves for greedy readout of one
 * row through w (0: w takes another kernel and offers none). */
size_t zg_gemv_greedy_parts(const zg_weight* w);

/* zg_gemv_device without any allocation: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and bit-identical results, with the activation scratch
 * in a static per-device array of 4 MiB (held until the process ends)
 * instead of a context buffer.  Limits: m_rows 1..64 and the prepared
 * activation within 4 MiB (ZG_E_LIMIT otherwise); Q4_K with f32 input, 2
 * or more rows and a shape the 16-row kernel does not take needs the
 * weight's batched tile layout, which one zg_gemv_device call of that shape
 * builds (ZG_E_STATE otherwise).
 * Every call on a device shares that device's array, which keeps the last
 * call's contents.  Calls are ordered on it: each waits on an event the
 * previous call on that device (any stream, thread or context) recorded
 * after its kernels.  A call made while its stream is captured into a graph
 * is ordered only by the graph's own stream order: replaying that graph
 * while other calls use the array on the same GPU races. */
int zg_gemv_device_noalloc(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows,
                           const float* gamma, float eps, float* y, void* stream);

/* The two halves of zg_gemv_device, for callers that prepare one activation
 * and reuse it (and for timing the GEMV kernel alone).  The prepared buffer
 * is device memory of zg_act_prepared_bytes(w, m_rows) bytes holding the
 * activation in the format w's codec consumes:
 *   Q8_0: int8 codes [M][columns], then f32 scales [M][columns/32]: the
 *         dynamic Q8_0 coding of cpu/src/source/quantization.rs:37-61;
 *   Q4_K: int16 fixed-point group-pair records [M][columns/64][64], then f32
 *         {scale_lo, scale_hi, sum_lo, sum_hi} [M][columns/64];
 *   F32 : f32 [M][columns];
 * each part starting on a 256-byte boundary. */
size_t zg_act_prepared_bytes(const zg_weight* w, size_t m_rows);
int zg_act_prepare_device(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows,
                          const float* gamma, float eps, void* prepared, size_t prepared_len, void* stream);
int zg_gemv_prepared_device(zg_ctx* ctx, const zg_weight* w, size_t m_rows, const void* prepared, float* y,
                            void* stream);

#ifdef __cplusplus
}
#endif
#endif
