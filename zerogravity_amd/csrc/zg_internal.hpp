// Host-side interface between the C ABI (zg_api.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace zg {

enum GgmlType { kF32 = 0, kF16 = 1, kQ4_1 = 3, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kBF16 = 30 };

// A registered weight matrix in its device layout.  The GGUF block stream is
// split once at registration into a streaming payload and a small per-block
// header array so every wavefront load is a coalesced 16-byte load:
//   Q8_0: qs  = int8 [N][K]            hdr = f16 scale [N][K/32]
//   Q4_K: qs  = nibbles in 16-row tiles (q4k_chunk_offset)
//         hdr = 16-byte block headers in 16-row tiles (q4k_hdr_index):
//         d, dmin and the 12 scale/min bytes repacked (q4k_dev_scale_min)
//   F32 : qs  = float [N][K]           hdr = null
//   Q4_1: qs  = nibble words in 8-row tiles (q41_word_index)
//         hdr = uint32 d | m << 16 [N][K/32 rounded to 8 blocks]
//   Q6_K: qs  = bit planes A and B in 8-row tiles (q6k_a_index, q6k_b_index)
//         hdr = int8 local scales [N][K/256][16], then f32 d [N][K/256]
// Algorithmic bytes are unchanged: 1.0625 B/elem (Q8_0), 0.5625 (Q4_K; plus
// the zero rows that complete the last 16-row tile).
struct DeviceWeight {
    int type = -1;
    size_t K = 0, N = 0;
    void* qs = nullptr;
    void* hdr = nullptr;
    size_t qs_bytes = 0, hdr_bytes = 0;
    // Q4_K only, built on demand for the batched-row MFMA path: payload and
    // headers in the MFMA operand order of 32-row tiles (ensure_mfma_tiles).
    void* qs_t = nullptr;
    void* hdr_t = nullptr;
};

size_t gguf_row_bytes(int type, size_t K);

// Split a GGUF tensor (already on the device) into the layout above.  Any
// nonfinite block scale sets *d_bad to 1 (the reference codecs refuse it).
hipError_t repack_weight(const uint8_t* d_gguf, DeviceWeight& w, int* d_bad, hipStream_t s);

// Exact dequantization of rows [row0, row0+rows) of a registered weight into
// f32 [rows][K].
hipError_t dequantize_rows(const DeviceWeight& w, size_t row0, size_t rows, float* out, hipStream_t s);

// Activation rows from which batched_gemv runs the register-blocked prompt
// GEMM (zg_gemm.hip) instead of the decode-shaped MFMA kernel.
constexpr int kGemmRows = 256;

// f16 activation tiles of the batched GEMMs, element (m, k) for K columns.
// 32-row layout (the prompt GEMM and the 32-row decode kernel): lane l of a
// v_mfma_f32_32x32x16_f16 A operand loads 16 contiguous bytes.
__host__ __device__ inline size_t xh32_index(size_t m, size_t k, size_t K) {
    return ((((m >> 5) * (K >> 8) + (k >> 8)) * 16 + ((k & 255) >> 4)) * 64 + ((k & 15) >> 3) * 32 + (m & 31)) * 8 +
           (k & 7);
}
// 16-row layout (the decode kernel on Q4_K 16-row tiles): per 16 rows mb and
// 128-column unit u, four 1 KB v_mfma_f32_16x16x32_f16 A operands i; lane
// (m % 16) + 16 (h + 2 cp) of operand i = 2 nib + sub holds the 8 columns
// whose weights the same lane of the weight operand dequantises from the
// Q4_K tile layout: run 2u + cp of the row, bytes 16 h + 8 sub .. + 7, low
// (nib 0) or high (nib 1) nibbles, i.e. k = 128 u + 64 cp + 32 nib + 16 h +
// 8 sub + e.
__host__ __device__ inline size_t xh16_index(size_t m, size_t k, size_t K) {
    const size_t u = k >> 7, cp = (k >> 6) & 1, nib = (k >> 5) & 1, h = (k >> 4) & 1, sub = (k >> 3) & 1;
    return ((((m >> 4) * (K >> 7) + u) * 4 + 2 * nib + sub) * 64 + (m & 15) + 16 * (h + 2 * cp)) * 8 + (k & 7);
}
// Decode-sized batches (M < kGemmRows) whose K is a multiple of 1024 up to
// 6144 run the 16-row kernel, so their activations use the 16-row layout;
// every producer of batched activation tiles picks the layout with this.
__host__ __device__ inline bool xh16_layout(size_t M, size_t K) {
    return M < (size_t)kGemmRows && K % 1024 == 0 && K <= 6144;
}
__host__ __device__ inline size_t xh_tile_index(size_t m, size_t k, size_t K, size_t M) {
    return xh16_layout(M, K) ? xh16_index(m, k, K) : xh32_index(m, k, K);
}

// Activation preparation for M rows of width K: optional RMSNorm with gamma
// (f64 sum of f32 squares, f32 mean, 1/sqrtf, (x*inv)*gamma), then any of:
// f32 output (xf); the dynamic Q8_0 coding (aq codes, ad f16-rounded
// scales); the Q4_K int16 group-pair records (x4, m4).  x is bf16 when
// x_bf16 != 0, else f32.
hipError_t act_prep(const void* x, int x_bf16, size_t M, size_t K, const float* gamma, float eps,
                    float* xf, int8_t* aq, float* ad, int16_t* x4, float* m4, hipStream_t s);

// The activation format a weight type consumes, in one device buffer:
//   Q8_0: int8 codes [M][K], then f32 scales [M][K/32]
//   Q4_K: int16 records [M][K/64][64], then f32 {xs_lo, xs_hi, sum_lo, sum_hi} [M][K/64]
//   F32 : f32 [M][K]
// (each part 256-byte aligned).
size_t prepared_bytes(int type, size_t M, size_t K);
hipError_t act_prepare_for(int type, const void* x, int x_bf16, size_t M, size_t K, const float* gamma, float eps,
                           void* prepared, hipStream_t s);

// y[M][N] = W x for a registered weight over a prepared activation.
// Returns hipErrorInvalidValue for unsupported geometry.
hipError_t gemv(const DeviceWeight& w, size_t M, const void* prepared, float* y, hipStream_t s);
bool gemv_supported(int type, size_t K, size_t M);

// Pointwise / normalisation kernels (zg_elementwise.hip).
hipError_t rms_groups(const float* x, const float* w, size_t width, size_t groups, float eps, float* out,
                      hipStream_t s);
hipError_t silu(const float* x, const float* m, size_t n, float* out, hipStream_t s);
hipError_t binary(int kind, const float* a, const float* b, size_t n, float* out, hipStream_t s);

// Gated DeltaNet decode (zg_gdn.hip).  Strides are in floats per row.
hipError_t gdn_conv(const float* x, const float* w, float* hist, float* out, size_t C, size_t rows, int apply_silu,
                    size_t x_stride, size_t hist_stride, size_t out_stride, hipStream_t s);
hipError_t gdn_coefficients(const float* alpha, const float* beta, const float* dt, const float* a, size_t H,
                            float* gain, float* beta_out, float* sp, float* gr, hipStream_t s);
// fused: q/k L2 + coefficients from raw alpha/beta projections (model path);
// otherwise alpha/beta carry gain/beta and scale_h (nullable) the per-head scale.
hipError_t gdn_recurrent(bool fused, const float* q, const float* k, const float* v, size_t src_stride,
                         const float* alpha, const float* beta, size_t coef_stride, const float* dt, const float* a,
                         float eps, float scale, const float* scale_h, float* state, float* out, size_t out_stride,
                         size_t H, size_t D, size_t rows, hipStream_t s);

// GQA decode attention (zg_attn.hip), d = 256, <= 8 query heads, <= 4 per kv
// head.  Scores/probs are compact per row: [h][ntok[b]] at b*score_stride.
struct AttnArgs {
    int B = 0, nq = 0, nkv = 0, d = 0, rotate = 64, tmax = 0;
    int kv_bf16 = 0, do_prep = 0, prep_only = 0, norm = 1;
    const float* qproj = nullptr;  // [B][nq*2d] (q | gate per head)
    size_t q_stride = 0;
    const float *kproj = nullptr, *vproj = nullptr;
    size_t kv_stride = 0;
    const float *qnorm = nullptr, *knorm = nullptr;
    const int* pos = nullptr;   // [B] position written by this step
    const int* ntok = nullptr;  // [B] valid tokens
    float theta_scale = 0.0f, eps = 0.0f, scale = 0.0f;
    float* qr = nullptr;  // [B][nq*d] roped query
    size_t qr_stride = 0;
    void *kcache = nullptr, *vcache = nullptr;  // [B][tmax][nkv*d] KV
    size_t cache_row_stride = 0;                // elements per row
    float *kout = nullptr, *vout = nullptr;     // direct f32 k/v outputs (region path)
    float *dots = nullptr, *scores = nullptr, *exps = nullptr, *probs = nullptr;
    double* sums = nullptr;
    size_t score_stride = 0;
    const float* gate = nullptr;
    size_t gate_stride = 0;
    float* out = nullptr;
    size_t out_stride = 0;
};
hipError_t attention(const AttnArgs& a, hipStream_t s);            // prep (if do_prep) + all parts
hipError_t rope_prep(const AttnArgs& a, hipStream_t s);            // norm + RoPE + KV append only
hipError_t attention_parts(const AttnArgs& a, bool qk, bool softmax, bool pv, hipStream_t s);
hipError_t softmax_rows(const float* scores, size_t score_stride, const int* ntok, float* probs, size_t heads, size_t B,
                        hipStream_t s);

// Model-step helpers (zg_model.hip).  `status` is a device word: bit 0
// nonfinite residual, bit 1 out-of-vocabulary token, bit 2 nonfinite logits.
hipError_t embed(const DeviceWeight& w, const uint32_t* tokens, float* x, size_t B, int* status, hipStream_t s);
hipError_t fill_normal(void* p, size_t n, bool bf16, uint64_t seed, float sigma, hipStream_t s);
hipError_t convert_kv(const void* in, void* out, size_t n, bool to_f32, hipStream_t s);
hipError_t fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s);

// ---------------------------------------------------- fused decode step
// (zg_fused*.hip, zg_batched.hip, zg_gdn_decode.hip, zg_attn_decode.hip).  A GEMV launch with an activation prologue and an output
// epilogue:
//   PRO_RMS       x[m][0:K] -> (x*inv)*gamma            (RMSNorm, eps)
//   PRO_GATED     per group of `group` elements: ((x*inv)*gamma[i % group])
//                 * silu(x2)                            (gated RMSNorm)
//   PRO_SILU_MUL  x2 * silu(x)                          (x = gate, x2 = up)
//   PRO_PLAIN     x
//   PRO_GATED_PRE PRO_GATED with the product (x*gamma[i % group])*silu(z)
//                 already formed (GdnDecodeArgs::gated) in x2; x is the
//                 norm input (its per-group sums of squares).  One row on
//                 the matrix-core Q4_K GEMV only (gated_pre_supported).
//   EPI_STORE     y[m][n] = W a
//   EPI_RESID     y[m][n] += W a, nonfinite -> status bit 0
//   EPI_GLU       stacked [gate (N/2 rows) | up (N/2 rows)]:
//                 y[m][j] = up_j * silu(gate_j) for j < N/2 (the SwiGLU
//                 product the down projection takes, forward.rs ffn);
//                 batched rows write it in f16 MFMA tile order to xh_out
enum { PRO_RMS = 0, PRO_GATED = 1, PRO_SILU_MUL = 2, PRO_PLAIN = 3, PRO_EMBED_RMS = 4, PRO_GATED_PRE = 5 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_GLU = 2 };
struct FusedGemvArgs {
    const void* qs = nullptr;  // filled from the weight
    const void* hdr = nullptr;
    int N = 0, K = 0;
    int M = 0;  // activation rows
    int pro = PRO_PLAIN, epi = EPI_STORE;
    const float* x = nullptr;
    size_t ldx = 0;
    const float* x2 = nullptr;
    size_t ldx2 = 0;
    const float* gamma = nullptr;
    float eps = 0.0f;
    int group = 128;
    float* y = nullptr;
    size_t ldy = 0;
    int* status = nullptr;
    // batched rows only.  splits > 1 (EPI_RESID): the GEMM writes partial
    // tiles parts[split][Mpad][N] instead of adding into y; the following
    // PRO_RMS call over y passes them as rparts/rsplits and its activation
    // kernel first adds their fixed-order sum into its input rows (x, which
    // must then be writable: xw).
    float* parts = nullptr;
    int splits = 0;
    const float* rparts = nullptr;
    int rsplits = 0;
    // prompt-sized residual projections (optional): workspace of
    // prompt_parts_n floats for the prompt GEMM's own split over K (two or
    // four runs of S x M x N partial sums), summed into y by a second launch
    // in a fixed order; a split that would not fit is not taken
    float* prompt_parts = nullptr;
    size_t prompt_parts_n = 0;
    float* xw = nullptr;
    // batched rows, a residual projection without splits: with
    // rms_tiles_out it also leaves the next RMS projection's input -- f16
    // (x_new * rms_gamma) in MFMA A-tile order for K = N (xh_tile_index),
    // and per row and 32-column tile (16-column on the 16-row kernel) the
    // f64 sum of the f32 squares of x_new at rms_ss_out[m][N/32 or N/16].
    // That RMS projection passes the tiles as xh_in and the sums as
    // rms_ss_in (rms_ss_n per row) and scales each row's outputs by 1/rms
    // (RMSNorm's factor moved past the dot).
    _Float16* rms_tiles_out = nullptr;
    const float* rms_gamma = nullptr;
    double* rms_ss_out = nullptr;
    const double* rms_ss_in = nullptr;
    int rms_ss_n = 0;
    const int* staged = nullptr;  // Q6_K beyond 4 rows: the rows coded once (q6k_rows_gemv)
    void* xh_out = nullptr;      // EPI_GLU, batched: f16 tiled product
    const void* xh_in = nullptr;  // batched: f16 tiled activation ready (no activation kernel)
    int xh_rows = 0;              // activation kernel: f16 row-major [M][K] instead of MFMA tiles
    // one activation row, EPI_STORE, matrix-core GEMV: each workgroup also
    // leaves its outputs' greedy partial (largest value, first index; a
    // nonfinite output sets status bit 2) at amax/aidx[blockIdx.x]
    float* amax = nullptr;
    int* aidx = nullptr;
    // one activation row, PRO_RMS, matrix-core GEMV: the activation is the
    // Q4_K embedding row (emb_qs/emb_hdr, emb_rows rows of width K) of the
    // token at *tok, dequantised in the prologue (embed_q4k_kernel's
    // arithmetic; a token past emb_rows sets status bit 1 and reads zeros),
    // and workgroup 0 also stores it at x_out (the residual stream)
    const uint32_t* tok = nullptr;
    const void* emb_qs = nullptr;
    const void* emb_hdr = nullptr;
    int emb_rows = 0;
    float* x_out = nullptr;
    // one activation row, EPI_STORE, matrix-core GEMV, the GDN input
    // projection: outputs gate_row + h (h < gate_heads, alpha) are stored as
    // the gain gdn_gain(alpha, gate_dt[h], gate_a[h]) and outputs gate_row +
    // gate_heads + h (beta) as source_sigmoid(beta), the GDN gates formed by
    // the same functions the GDN kernel would apply (GdnDecodeArgs::
    // gates_formed); the workgroups holding those rows run first
    const float* gate_dt = nullptr;
    const float* gate_a = nullptr;
    int gate_row = 0, gate_heads = 0;
};
// EPI_GLU offered for these shapes (fused path: K <= 2048 so a row group
// holds a gate and an up row; batched path: N/2 a multiple of 32).
bool fused_glu_supported(int type, size_t K, size_t N);
bool batched_glu_supported(int type, size_t K, size_t N);
// K splits for a residual batched GEMM of this shape (1: none).
int batched_splits(size_t N, size_t K);
// Whether batched_gemv runs M rows of this shape on the 16-row Q4_K kernel
// (no split-K; xh16_layout(M, K) holds, and a residual projection with
// rms_tiles_out leaves rms_ss_out[m][N/16]).
bool batched16_supported(size_t M, size_t K, size_t N, int epi);
bool fused_gemv_supported(int type, size_t K, size_t N, int pro);
// Greedy partials the one-row matrix-core GEMV leaves for this weight with
// EPI_STORE (0 when the weight takes another kernel).
int gemv1_greedy_parts(const DeviceWeight& w, int pro);
// Whether a one-row PRO_RMS projection of w can take its activation from a
// Q4_K embedding (FusedGemvArgs::tok/emb_*) in its prologue.
bool gemv1_embed_supported(const DeviceWeight& w, const DeviceWeight& emb);
// Whether a one-row projection of w can take PRO_GATED_PRE (group 128).
bool gated_pre_supported(const DeviceWeight& w);
hipError_t fused_gemv(const DeviceWeight& w, const FusedGemvArgs& a, hipStream_t s);
// Batched rows (M > 4, Q4_K; decode batches and prompts): the prologue
// values rounded to f16 into `scratch` (batched_scratch_bytes), then an f16
// MFMA GEMM with the epilogue (LDS-staged from 1024 rows).
size_t batched_scratch_bytes(size_t M, size_t K);
// Builds w.qs_t / w.hdr_t (Q4_K) if absent: allocates, so call it outside
// graph capture.  batched_gemv refuses a Q4_K weight without them.
hipError_t ensure_mfma_tiles(DeviceWeight& w, hipStream_t s);
hipError_t batched_gemv(const DeviceWeight& w, const FusedGemvArgs& a, void* scratch, hipStream_t s);
// Q8_0 beyond 4 rows (zg_q8rows.hip): every activation row coded once into
// `scratch` in act_prepare_for's layout (prepared_bytes(kQ8_0, M, K), within
// batched_scratch_bytes), then the weights streamed once per 16 rows;
// bit-identical to the fused kernels.  Prologues RMS, GATED, SILU_MUL,
// PLAIN; epilogues STORE and RESID.  batched_gemv routes Q8_0 here.
bool q8_rows_supported(size_t K, size_t N, int pro);
hipError_t q8_rows_gemv(const DeviceWeight& w, const FusedGemvArgs& a, void* scratch, hipStream_t s);
// Q6_K beyond 4 rows: each row coded once to Q8_K into `scratch` (within
// batched_scratch_bytes), then the fused Q6_K kernel on up to 16 staged rows
// per workgroup; bit-identical to the 1-4 row kernel.  batched_gemv routes
// Q6_K here.
bool q6k_rows_supported(size_t K, size_t N, int pro);
hipError_t q6k_rows_gemv(const DeviceWeight& w, const FusedGemvArgs& a, void* scratch, hipStream_t s);
// The same GEMV on an activation act_prepare_for already prepared.
hipError_t q8_rows_prepared(const DeviceWeight& w, size_t M, const void* prepared, float* y, hipStream_t s);
// The prompt-sized GEMM on f16 A tiles `xh` (act16_kernel's layout, or the
// previous gate/up GEMM's SwiGLU tiles): EPI_STORE / EPI_RESID into y, or
// EPI_GLU into xh_out (a product past the f16 range sets status bit 4).
bool prompt_gemm_supported(int type, size_t K, size_t N, int epi);
hipError_t prompt_gemm(const DeviceWeight& w, const FusedGemvArgs& a, const _Float16* xh, hipStream_t s);
uint64_t prompt_gemm_bytes(size_t M, size_t K, size_t N);

// GDN decode: conv (4-slot ring per channel) + SiLU + q/k L2 + gates +
// recurrence for B rows.  proj rows: [qkv (3W) | z (W) | alpha (H) | beta (H)].
struct GdnDecodeArgs {
    const float* proj = nullptr;
    size_t proj_stride = 0;
    const float* conv_w = nullptr;  // [3W][4]
    float* ring = nullptr;          // [B][3W][4]
    const int* pos = nullptr;       // [B] position of this step's token
    const float *dt = nullptr, *ssm_a = nullptr;
    float eps = 0.0f, scale = 0.0f;
    float* state = nullptr;  // row b at state + b*state_row: [H][128][128] value-major
    int* status = nullptr;   // bit 4: the f16 tiles' value past the f16 range
    float* core = nullptr;   // [B][W]
    int H = 0;
    // optional double-buffered rows (the session's uncommitted draft): row b
    // reads half cur[b] (at + cur[b]*state_half) and writes the other half;
    // without cur the state is updated in place.  state_row 0 = H*128*128.
    const int* cur = nullptr;
    size_t state_row = 0, state_half = 0;
    // batched rows (optional): the output projection's activation --
    // gated RMSNorm (ssm_norm [128], z = proj[3W:4W]) x silu(z) -- written as
    // f16 MFMA tiles for K = W (the layout act16_kernel writes), so that GEMM
    // needs no activation launch.  One workgroup then holds a whole head.
    void* xh = nullptr;
    const float* norm = nullptr;
    // one-workgroup-per-quarter rows (optional, with norm): [B][W] the gated
    // norm's product before its 1/rms, (core * norm[j % 128]) * silu(z),
    // for the output projection's PRO_GATED_PRE prologue
    float* gated = nullptr;
    // the projection already holds the gain at proj[4W + h] and beta at
    // proj[4W + H + h] (FusedGemvArgs::gate_dt) instead of alpha and the
    // beta projection
    int gates_formed = 0;
};
hipError_t gdn_decode(const GdnDecodeArgs& a, size_t B, hipStream_t s);

// Attention decode (d = 256): proj rows [q|gate per head (nq*2d) | k (nkv*d)
// | v (nkv*d)]; KV cache [B][max_ctx][nkv*d]; scores at
// b*score_stride + h*head_stride + t; out [B][nq*d] (gated).
struct AttnDecodeArgs {
    const float* proj = nullptr;
    size_t proj_stride = 0;
    const float *qnorm = nullptr, *knorm = nullptr;
    float eps = 0.0f, theta_scale = 0.0f, scale = 0.0f;
    const int* pos = nullptr;
    void *kcache = nullptr, *vcache = nullptr;
    size_t cache_row_stride = 0;
    int kv_bf16 = 0;
    float* scores = nullptr;
    size_t score_stride = 0, head_stride = 0;
    float* out = nullptr;
    size_t out_stride = 0;
    int* status = nullptr;  // bit 3: degenerate softmax sum; bit 4: a batched f16 operand past its range
    float* stats = nullptr;  // [B][nq][2] softmax {max, 1/sum}
    int nq = 0, nkv = 0, max_ctx = 0;
    // batched rows (optional): the gated output also written as f16 MFMA
    // tiles for K = nq*d (xh_tile_index), the output projection's activation
    void* xh = nullptr;
    // split form (optional): the RoPE table of rope_table, [max_ctx][32]
    // (cos, sin) pairs for this theta_scale
    const float* rope = nullptr;
};
hipError_t rope_table(float* tab, size_t n, float theta_scale, hipStream_t s);
hipError_t attn_decode(const AttnDecodeArgs& a, size_t B, hipStream_t s);
// Split-T form for 1..64 rows (attn_split_kernel + attn_combine_kernel):
// per-span partials in `part` (attn_split_part_bytes), then the combine
// into out (and the xh tiles when set); the same operations regrouped,
// within f32 rounding of the reference's order.
bool attn_split_supported(size_t B, int nq, int nkv, size_t max_ctx);
size_t attn_split_part_bytes(size_t B, int nq, int nkv, size_t max_ctx);
hipError_t attn_decode_split(const AttnDecodeArgs& a, size_t B, float* part, hipStream_t s);

// Chunked GDN prefill (zg_prefill.hip), d = 128, chunk 64: q, k, v
// [T][H][128], beta and log decay [T][H], state [H][128][128] updated in
// place (value-major [h][v][k], or [h][k][v] with key_major), out
// [T][H][128] (before the gated norm; bf16-rounded with round_bf16); scratch
// of gdn_chunk_scratch_bytes(T, H).
size_t gdn_chunk_scratch_bytes(size_t T, size_t H);
hipError_t gdn_chunk_prefill(const float* q, const float* k, const float* v, const float* beta, const float* logd,
                             size_t T, size_t H, float* state, float* out, float* scratch, bool key_major,
                             bool round_bf16, hipStream_t s);

// Batched prefill of one sequence (zg_prefill_model.hip).
// gdn_prefill_conv: conv inputs P[t][0:3W] (row stride ldp, then z, alpha,
// beta as in the decode projection) -> SiLU(conv) split into q, k, v [n][W],
// gates beta / log decay [n][H]; the row's ring [3W][4] then holds the last
// four prompt tokens.
hipError_t gdn_prefill_conv(const float* P, size_t ldp, size_t n, size_t W, size_t H, const float* conv_w,
                            float* ring, int pos0, const float* dt, const float* ssm_a, float* q, float* k, float* v,
                            float* beta, float* logd, hipStream_t s);
struct AttnPrefillArgs {
    const float* P = nullptr;  // [n][ldp]: q|gate per head, k, v (the decode projection layout)
    size_t ldp = 0, n = 0;
    int nq = 0, nkv = 0, pos0 = 0, kv_bf16 = 0;
    const float *qnorm = nullptr, *knorm = nullptr;
    float eps = 0.0f, theta_scale = 0.0f, scale = 0.0f;
    void *kcache = nullptr, *vcache = nullptr;  // this row's [max_ctx][nkv*256]
    float* Q = nullptr;                         // scratch [n][nq][256]
    float* out = nullptr;                       // [n][nq*256], gated
    int* status = nullptr;                      // bit 4: a K or V value past the f16 range
    // optional key-chunk partials, attn_prefill_part_bytes(n, nq) bytes: long
    // prompts split each query tile's keys over several workgroups
    float* part = nullptr;
    // optional RoPE table of rope_table covering positions pos0 .. pos0+n-1
    const float* rope = nullptr;
};
// q/k norm + RoPE + KV append for the n tokens, then causal attention.
hipError_t attn_prefill(const AttnPrefillArgs& a, hipStream_t s);
size_t attn_prefill_part_bytes(size_t n, int nq);

// Greedy ids of B logit rows (leading dimension ld) through partials
// [argmax_partials(B)] (core/src/numerics.rs:126-140: first maximum wins,
// a nonfinite logit sets status bit 2).  With `commit` non-null the last
// launch also publishes the step for rows [0, B) when the status word is
// clear: pos and ntok move on and cur flips (commit_step's rule).
size_t argmax_partials(size_t B);
struct StepCommit {
    int* pos = nullptr;
    int* ntok = nullptr;
    int* cur = nullptr;
};
hipError_t argmax_step(const float* logits, size_t V, size_t ld, size_t B, uint32_t* greedy, int* status, float* pmax,
                       int* pidx, const StepCommit* commit, hipStream_t s);
// The greedy id of one row from `parts` partials a GEMV left (gemv1
// amax/aidx), with the same commit rule as argmax_step.
hipError_t argmax_final(const float* pmax, const int* pidx, int parts, uint32_t* greedy, int* status,
                        const StepCommit* commit, hipStream_t s);
// Publish a decode step for rows [0, B) if *status == 0: positions advance
// and each row's GDN state half flips to the draft the step wrote.
hipError_t commit_step(const StepCommit& c, const int* status, size_t B, hipStream_t s);

}  // namespace zg
