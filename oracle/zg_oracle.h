/*
 * zg_oracle — CPU restatement of zerogravity's GGUF Qwen3.5 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the timed
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library (libzg_hip.so) never
 * links, loads or falls back to it.
 *
 * Every function restates one reference function (file:line relative to the
 * zerogravity repository root).  Build flags: -O2 -ffp-contract=off, with an
 * explicit fmaf() exactly where the Rust source calls mul_add, f64 exactly
 * where it widens, and glibc expf/logf/powf/sinf/cosf where it calls the
 * platform f32::{exp,ln,powf,sin_cos}.
 *
 * Pinning (what checks each function; see tests/test_oracle_kat.py):
 *   codecs ................. reference KATs codecs/mod.rs:95-166,243-261,
 *                            codecs/exact_tests.rs:5-140, cpu/src/source.rs:605-619
 *   q8 activation coding ... quantization.rs:318-365,402-433 KATs
 *   q8_0 row dot ........... quantization.rs:436-494 (-1016.0) + exact integer
 *                            brute force on random rows (f64 closed form)
 *   q4_k row dot ........... source.rs:641-679 + f64 closed form over decoded rows
 *   rms / grouped rms ...... ops.rs:157-159, lib.rs:1911-1941, lib.rs:1944-1976
 *   ggml exp / silu ........ ops.rs:358-377 (|err| <= 1e-5 vs exact SiLU)
 *   binary ................. lib.rs:1701-1736 signed-zero table
 *   gdn conv ............... cpu/src/ops/gdn.rs:51-84 exact bits
 *   gdn recurrence ......... lib.rs:1998-2055 f64 oracle, 32768 tokens, 1e-5
 *   rope ................... lib.rs:1864-1908, 2151-2172 (f64, 2e-6)
 *   softmax ................ lib.rs:1803-1862 (padded 8-lane equivalence)
 *   attention value ........ lib.rs:1738-1799 signed-zero padding table
 *   attention qk ........... core/src/accelerator.rs:1012-1054 (score = dot*scale)
 *   greedy ................. core/src/numerics.rs:146-162
 *   gdn recurrence (real) .. the reference's pinned_cached_head0.f32le.bin vector
 *                            (recurrent_tests.rs:14-76), at tolerance
 *   forward_token .......... composition of the above in forward.rs:451-755 order;
 *                            no reference-held end-to-end vector exists (all such
 *                            reference tests need private checkpoints).  Pinned by an
 *                            independent float64 numpy forward written from
 *                            forward.rs and the closed-form GDN update
 *                            (tests/test_forward_independent.py), which a planted
 *                            [q|gate] swap is shown to fail.
 *
 * Transcendentals: ZGO_LIBM_GLIBC (default) calls glibc expf/logf/sinf/cosf,
 * as Rust's f32::{exp, ln, sin_cos} do on Linux; ZGO_LIBM_CORRECT rounds the
 * double result once (the correctly rounded value the HIP kernels compute),
 * selected only by the bit-exact device regression tests.
 */
#ifndef ZG_ORACLE_H
#define ZG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ZGO_LIBM_GLIBC = 0, ZGO_LIBM_CORRECT = 1 };
/* Select the transcendental mode (returns the previous one). */
int zgo_set_libm_mode(int mode);
int zgo_libm_mode(void);

/* ggml type codes, core/src/encoding.rs:77-91 */
enum { ZGO_F32 = 0, ZGO_F16 = 1, ZGO_Q4_0 = 2, ZGO_Q4_1 = 3, ZGO_Q8_0 = 8,
       ZGO_Q4_K = 12, ZGO_Q6_K = 14, ZGO_BF16 = 30 };

/* status codes */
enum { ZGO_OK = 0, ZGO_E_MALFORMED = -1, ZGO_E_UNSUPPORTED = -2, ZGO_E_STATE = -3,
       ZGO_E_LIMIT = -4 };

float    zgo_f16_to_f32(uint16_t bits);
uint16_t zgo_f32_to_f16_rne(float value);
int      zgo_block_geometry(int ggml_type, uint64_t* elements, uint64_t* bytes);
int      zgo_dequantize(int ggml_type, const uint8_t* data, size_t nbytes, size_t elements,
                        float* out);

int   zgo_q8_activation(const float* x, size_t n, int8_t* qs, float* d, float* s);
float zgo_dot_q8_0_row(const uint8_t* row, const int8_t* qs, const float* d, size_t nblocks);
float zgo_dot_q4k_row(const uint8_t* row, const float* x, size_t nblocks);
float zgo_dot_f32_row(const uint8_t* row, const float* x, size_t n);
int   zgo_q8k_activation(const float* x, size_t n, int8_t* qs, float* d, int32_t* bsums);
float zgo_dot_q4_0_row(const uint8_t* row, const int8_t* qs, const float* d, size_t nblocks);
float zgo_dot_q4_0_repacked_row(const uint8_t* row, const int8_t* qs, const float* d, size_t nblocks);
float zgo_dot_q4_1_row(const uint8_t* row, const int8_t* qs, const float* d, const float* s, size_t nblocks);
float zgo_dot_q6k_row(const uint8_t* row, const int8_t* qs, const float* d, const int32_t* bsums, size_t nblocks);
int   zgo_matvec(int ggml_type, const uint8_t* w, size_t wbytes, size_t rows, size_t cols,
                 const float* x, float* y, int threads);

int zgo_rms_norm(const float* x, const float* w, size_t n, float eps, float* out);
int zgo_grouped_rms_norm(const float* x, const float* w, size_t width, size_t groups,
                         float eps, float* out);

float zgo_ggml_exp(float x);
float zgo_ggml_silu(float x);
int   zgo_silu(const float* x, const float* mult, size_t n, float* out);
float zgo_sigmoid(float x);
float zgo_softplus(float x);
int   zgo_binary(int kind, const float* a, const float* b, size_t n, float* out);

int   zgo_gdn_conv_step(const float* act, const float* w, float* history, float* raw,
                        size_t channels);
int   zgo_gdn_coefficients(const float* alpha, const float* beta, const float* dt,
                           const float* a, size_t heads, float scale, float* gain,
                           float* beta_out, float* softplus_out, float* gate_raw_out);
float zgo_source_dot_f32(const float* a, const float* b, size_t n);
int   zgo_gdn_recurrent_step(float* state, const float* q, const float* k, const float* v,
                             float gain, float beta, float scale, float* out, size_t d);

int zgo_rope_kv(float* q, float* k, size_t head_width, size_t q_heads, size_t kv_heads,
                size_t rotate, size_t position, float theta_scale);
int zgo_attention_qk(const float* q, const float* keys, size_t tokens, size_t head_width,
                     size_t q_heads, size_t kv_heads, float scale, float* dots, float* scores);
int zgo_attention_softmax(const float* scores, size_t heads, size_t width, float* exps,
                          float* probs, double* sums);
int zgo_attention_value(const float* probs, const float* values, size_t tokens,
                        size_t head_width, size_t q_heads, size_t kv_heads, size_t padded,
                        float* out);
int zgo_greedy(const float* logits, size_t n, uint32_t* out);

/* Chunked (WY/UT) GDN prefill restated from the Torch-profile chunk reference,
 * numerics/torch_cpu/gdn/chunk/core.rs:152-363.  q, k, v: [tokens][heads][d];
 * beta, log_decay: [tokens][heads]; state in/out value-major [h][v][k] (the
 * decode recurrence's layout, lib.rs:81-83), key-major [k][v] inside. */
int zgo_gdn_chunk_prefill(const float* q, const float* k, const float* v, const float* beta,
                          const float* log_decay, size_t tokens, size_t heads, size_t d,
                          size_t chunk, float* state, float* out);

/* ---- whole model (forward.rs:451-755 schedule) ---- */
typedef struct zgo_tensor {
    const char*    name;
    int            ggml_type;
    uint64_t       shape0;  /* GGML ne0 (inner, K) */
    uint64_t       shape1;  /* GGML ne1 (rows, N); 1 for vectors */
    const uint8_t* data;
    uint64_t       nbytes;
} zgo_tensor;

typedef struct zgo_geometry {
    uint32_t hidden, layers, ffn, vocab;
    uint32_t gdn_heads, gdn_dim;          /* linear_num_value_heads, head width */
    uint32_t q_heads, kv_heads, head_dim; /* full attention */
    uint32_t full_attention_interval;
    uint32_t max_context;
    float    eps;
} zgo_geometry;

typedef struct zgo_model   zgo_model;
typedef struct zgo_session zgo_session;

zgo_model*   zgo_model_create(const zgo_geometry* g, const zgo_tensor* tensors, size_t n,
                              int threads);
void         zgo_model_destroy(zgo_model* m);
const char*  zgo_model_error(const zgo_model* m);
zgo_session* zgo_session_create(zgo_model* m);
/* Test hook (no reference counterpart): store appended K/V rounded to bf16,
 * as a device session with a bf16 KV cache does. */
void         zgo_session_set_kv_bf16(zgo_session* s, int on);
void         zgo_session_destroy(zgo_session* s);
int          zgo_session_position(const zgo_session* s);
/* One forward_token: logits (vocab floats) written when logits != NULL. */
int zgo_forward_token(zgo_session* s, uint32_t token, float* logits);
/* Domain export in the reference order (lib.rs:112-150): per layer conv then
 * recurrent (value-major) for GDN layers, KV keys then values for attention. */
size_t zgo_state_floats(const zgo_session* s);
int    zgo_state_export(const zgo_session* s, float* out, size_t n);
int    zgo_state_import(zgo_session* s, const float* in, size_t n, int position);

#ifdef __cplusplus
}
#endif
#endif
