// Boundary A: the GDN and attention operator regions of the reference's
// MatVecKernel (core/src/accelerator.rs:592-655, 682-731), each one call
// over caller-owned host buffers staged through the context's scratch.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "zg_context.hpp"

using namespace zgc;

extern "C" {


int zg_gdn_conv(zg_ctx* ctx, const float* activation, const float* weights, const float* history, size_t channels,
                float* raw_out, float* history_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!activation || !weights || !history || !raw_out || !history_out || channels == 0 ||
        !all_finite(activation, channels) || !all_finite(weights, channels * 4) || !all_finite(history, channels * 3))
        return fail(ctx, ZG_E_MALFORMED, "GDN causal convolution source geometry/nonfinite input");
    const size_t oa = 0, ow = align256(channels * 4), oh = ow + align256(channels * 16), oo = oh + align256(channels * 12);
    int rc = ensure(ctx, ctx->scratch, oo + align256(channels * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    ZG_HIP(hipMemcpyAsync(b + oa, activation, channels * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ow, weights, channels * 16, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oh, history, channels * 12, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::gdn_conv((const float*)(b + oa), (const float*)(b + ow), (float*)(b + oh), (float*)(b + oo), channels, 1,
                        0, 0, 0, 0, st));
    ZG_HIP(hipMemcpyAsync(raw_out, b + oo, channels * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(history_out, b + oh, channels * 12, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(raw_out, channels) || !all_finite(history_out, channels * 3))
        return fail(ctx, ZG_E_STATE, "physical GDN convolution returned incomplete/nonfinite source state");
    return ZG_COMPLETED;
}

int zg_gdn_coefficients(zg_ctx* ctx, const float* alpha, const float* beta, const float* dt, const float* a,
                        size_t heads, float scale, float* gain_out, float* beta_out, float* softplus_out,
                        float* gate_raw_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!alpha || !beta || !dt || !a || !gain_out || !beta_out || !softplus_out || !gate_raw_out || heads == 0 ||
        !all_finite(alpha, heads) || !all_finite(beta, heads) || !all_finite(dt, heads) || !all_finite(a, heads) ||
        !std::isfinite(scale) || scale <= 0.0f)
        return fail(ctx, ZG_E_MALFORMED, "invalid source GDN coefficient inputs");
    const size_t stride = align256(heads * 4);
    int rc = ensure(ctx, ctx->scratch, 8 * stride);
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const float* ins[4] = {alpha, beta, dt, a};
    for (int i = 0; i < 4; ++i) ZG_HIP(hipMemcpyAsync(b + i * stride, ins[i], heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::gdn_coefficients((const float*)b, (const float*)(b + stride), (const float*)(b + 2 * stride),
                                (const float*)(b + 3 * stride), heads, (float*)(b + 4 * stride), (float*)(b + 5 * stride),
                                (float*)(b + 6 * stride), (float*)(b + 7 * stride), st));
    float* outs[4] = {gain_out, beta_out, softplus_out, gate_raw_out};
    for (int i = 0; i < 4; ++i)
        ZG_HIP(hipMemcpyAsync(outs[i], b + (4 + i) * stride, heads * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    for (int i = 0; i < 4; ++i)
        if (!all_finite(outs[i], heads)) return fail(ctx, ZG_E_STATE, "incomplete/nonfinite source GDN coefficients");
    return ZG_COMPLETED;
}

int zg_gdn_recurrent(zg_ctx* ctx, size_t width, size_t heads, const float* q, const float* k, const float* v,
                     const float* coefficients, const float* state, float* output, float* state_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!q || !k || !v || !coefficients || !state || !output || !state_out || width == 0 || heads == 0)
        return fail(ctx, ZG_E_MALFORMED, "invalid source GDN recurrent geometry or FP32 inputs");
    const size_t n = heads * width, ns = n * width;
    if (!all_finite(q, n) || !all_finite(k, n) || !all_finite(v, n) || !all_finite(state, ns) ||
        !all_finite(coefficients, heads * 3))
        return fail(ctx, ZG_E_MALFORMED, "invalid source GDN recurrent geometry or FP32 inputs");
    if (width != 128) return fail(ctx, ZG_UNSUPPORTED, "GDN recurrence offered for head width 128");
    std::vector<float> gain(heads), beta(heads), scale(heads);
    for (size_t h = 0; h < heads; ++h) {
        gain[h] = coefficients[3 * h];
        beta[h] = coefficients[3 * h + 1];
        scale[h] = coefficients[3 * h + 2];
    }
    const size_t oq = 0, ok = align256(n * 4), ov = ok + align256(n * 4), oc = ov + align256(n * 4),
                 os = oc + 3 * align256(heads * 4), oo = os + align256(ns * 4);
    int rc = ensure(ctx, ctx->scratch, oo + align256(n * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    ZG_HIP(hipMemcpyAsync(b + oq, q, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ok, k, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ov, v, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oc, gain.data(), heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oc + align256(heads * 4), beta.data(), heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oc + 2 * align256(heads * 4), scale.data(), heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + os, state, ns * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::gdn_recurrent(false, (const float*)(b + oq), (const float*)(b + ok), (const float*)(b + ov), 0,
                             (const float*)(b + oc), (const float*)(b + oc + align256(heads * 4)), 0, nullptr, nullptr,
                             0.0f, 0.0f, (const float*)(b + oc + 2 * align256(heads * 4)), (float*)(b + os),
                             (float*)(b + oo), 0, heads, width, 1, st));
    ZG_HIP(hipMemcpyAsync(output, b + oo, n * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(state_out, b + os, ns * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(output, n) || !all_finite(state_out, ns))
        return fail(ctx, ZG_E_STATE, "incomplete/nonfinite GDN recurrent proposal");
    return ZG_COMPLETED;
}

// The chunk (WY/UT) GDN step of numerics/torch_cpu/gdn/chunk/core.rs:69-274
// over one chunk of rows <= 64, with core()'s input checks (:86-116):
// heads a multiple of 16 and at most 48, q/k/v bf16-exact and finite, beta in
// [0, 1], log decay finite and <= 0, prior state finite.  State key-major
// [heads][128][128]; outputs rounded to bf16 (gdn.rs:69-76).
int zg_gdn_chunk(zg_ctx* ctx, size_t rows, size_t heads, const float* query, const float* key, const float* value,
                 const float* beta, const float* log_decay, const float* previous_state, float* output_bf16,
                 float* state_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    const size_t W = 128;
    if (!query || !key || !value || !beta || !log_decay || !output_bf16 || !state_out || rows < 1 || rows > 64 ||
        heads == 0 || heads > 48 || heads % 16 != 0)
        return fail(ctx, ZG_E_MALFORMED, "source chunk grouped input/state geometry");
    const size_t n = rows * heads * W, nb = rows * heads, ns = heads * W * W;
    auto bf16_exact = [](const float* x, size_t m) {
        for (size_t i = 0; i < m; ++i) {
            uint32_t b;
            std::memcpy(&b, &x[i], 4);
            if (!std::isfinite(x[i]) || (b & 0xffffu) != 0) return false;
        }
        return true;
    };
    bool ok = bf16_exact(query, n) && bf16_exact(key, n) && bf16_exact(value, n) && bf16_exact(beta, nb);
    for (size_t i = 0; ok && i < nb; ++i) ok = beta[i] >= 0.0f && beta[i] <= 1.0f;
    for (size_t i = 0; ok && i < nb; ++i) ok = std::isfinite(log_decay[i]) && log_decay[i] <= 0.0f;
    if (ok && previous_state) ok = all_finite(previous_state, ns);
    // the f64 cumulative decay must stay finite once rounded to f32 (finite
    // inputs cannot publish an overflowing cumsum)
    for (size_t h = 0; ok && h < heads; ++h) {
        double running = 0.0;
        for (size_t t = 0; ok && t < rows; ++t) {
            running += (double)log_decay[t * heads + h];
            ok = std::isfinite((float)running);
        }
    }
    if (!ok) return fail(ctx, ZG_E_MALFORMED, "source chunk BF16/decay/state operands");
    const size_t oq = 0, ok_ = align256(n * 4), ov = ok_ + align256(n * 4), ob = ov + align256(n * 4),
                 ol = ob + align256(nb * 4), os = ol + align256(nb * 4), oo = os + align256(ns * 4),
                 osc = oo + align256(n * 4);
    int rc = ensure(ctx, ctx->scratch, osc + zg::gdn_chunk_scratch_bytes(rows, heads));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    ZG_HIP(hipMemcpyAsync(b + oq, query, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ok_, key, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ov, value, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ob, beta, nb * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ol, log_decay, nb * 4, hipMemcpyHostToDevice, st));
    if (previous_state)
        ZG_HIP(hipMemcpyAsync(b + os, previous_state, ns * 4, hipMemcpyHostToDevice, st));
    else
        ZG_HIP(hipMemsetAsync(b + os, 0, ns * 4, st));
    ZG_HIP(zg::gdn_chunk_prefill((const float*)(b + oq), (const float*)(b + ok_), (const float*)(b + ov),
                                 (const float*)(b + ob), (const float*)(b + ol), rows, heads, (float*)(b + os),
                                 (float*)(b + oo), (float*)(b + osc), true, true, st));
    ZG_HIP(hipMemcpyAsync(output_bf16, b + oo, n * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(state_out, b + os, ns * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(output_bf16, n) || !all_finite(state_out, ns))
        return fail(ctx, ZG_E_MALFORMED, "diagnostic GDN BF16 overflow");
    return ZG_COMPLETED;
}

size_t zg_gdn_chunk_scratch_bytes(size_t tokens, size_t heads) { return zg::gdn_chunk_scratch_bytes(tokens, heads); }

// Multi-chunk prefill over device buffers on the caller's stream: chunks of
// 64 tokens in order, state value-major [heads][128][128] in place, f32
// outputs.  The per-(chunk, head) records live in the context's buffer,
// grown (after a stream synchronisation) when a longer prompt arrives.
int zg_gdn_chunk_prefill_device(zg_ctx* ctx, size_t tokens, size_t heads, const float* query, const float* key,
                                const float* value, const float* beta, const float* log_decay, float* state,
                                float* output, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!query || !key || !value || !beta || !log_decay || !state || !output || tokens == 0 || heads == 0 ||
        tokens > (1u << 24) || heads > 4096)
        return fail(ctx, ZG_E_MALFORMED, "chunk prefill geometry");
    if ((tokens + 64) * heads * 128 * 4 >= ((size_t)1 << 32))
        return fail(ctx, ZG_E_LIMIT, "chunk output (with one chunk of padding) of 4 GiB or more");
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    const size_t need = zg::gdn_chunk_scratch_bytes(tokens, heads);
    if (ctx->chunkbuf.bytes < need) ZG_HIP(hipStreamSynchronize(st));
    int rc = ensure(ctx, ctx->chunkbuf, need);
    if (rc) return rc;
    ZG_HIP(zg::gdn_chunk_prefill(query, key, value, beta, log_decay, tokens, heads, state, output,
                                 (float*)ctx->chunkbuf.ptr, false, false, st));
    return ZG_COMPLETED;
}

// One GDN layer's token step for `rows` sequences on device buffers (the
// resident decode step's kernel; forward.rs:518-632 up to the gated norm).
int zg_gdn_decode_device(zg_ctx* ctx, size_t rows, size_t heads, const float* proj, size_t proj_stride,
                         const float* conv_w, float* ring, const int32_t* positions, const float* dt,
                         const float* ssm_a, float eps, float* state, float* core, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!proj || !conv_w || !ring || !positions || !dt || !ssm_a || !state || !core || rows == 0 || heads == 0 ||
        rows > 65535 || heads > 1024 || proj_stride < heads * 128 * 4 + 2 * heads || !(eps > 0.0f))
        return fail(ctx, ZG_E_MALFORMED, "GDN decode geometry");
    zg::GdnDecodeArgs d;
    d.proj = proj;
    d.proj_stride = proj_stride;
    d.conv_w = conv_w;
    d.ring = ring;
    d.pos = positions;
    d.dt = dt;
    d.ssm_a = ssm_a;
    d.eps = eps;
    d.scale = 1.0f / sqrtf(128.0f);
    d.state = state;
    d.core = core;
    d.H = (int)heads;
    ZG_HIP(zg::gdn_decode(d, rows, stream ? (hipStream_t)stream : ctx->stream));
    return ZG_COMPLETED;
}

// The batched rows' form of the same step: one workgroup per (head, row)
// that also applies the gated RMSNorm (forward.rs:586-594) to the head's
// output and writes ssm_out's activation in f16, in the MFMA A-operand tile
// order the batched projections read (zg_gdn_decode_tiles_bytes).
size_t zg_gdn_decode_tiles_bytes(size_t rows, size_t heads) { return (rows + 31) / 32 * 32 * heads * 128 * 2; }

int zg_gdn_decode_gated_device(zg_ctx* ctx, size_t rows, size_t heads, const float* proj, size_t proj_stride,
                               const float* conv_w, float* ring, const int32_t* positions, const float* dt,
                               const float* ssm_a, const float* norm, float eps, float* state, float* core,
                               void* tiles, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!proj || !conv_w || !ring || !positions || !dt || !ssm_a || !norm || !state || !core || !tiles || rows == 0 ||
        heads == 0 || rows > 65535 || heads > 1024 || heads % 2 || proj_stride < heads * 128 * 4 + 2 * heads ||
        !(eps > 0.0f))
        return fail(ctx, ZG_E_MALFORMED, "GDN decode geometry");
    zg::GdnDecodeArgs d;
    d.proj = proj;
    d.proj_stride = proj_stride;
    d.conv_w = conv_w;
    d.ring = ring;
    d.pos = positions;
    d.dt = dt;
    d.ssm_a = ssm_a;
    d.eps = eps;
    d.scale = 1.0f / sqrtf(128.0f);
    d.state = state;
    d.core = core;
    d.H = (int)heads;
    d.xh = tiles;
    d.norm = norm;
    d.status = ctx->d_flag;
    ZG_HIP(zg::gdn_decode(d, rows, stream ? (hipStream_t)stream : ctx->stream));
    return ZG_COMPLETED;
}

size_t zg_attn_decode_workspace_bytes(size_t rows, size_t q_heads, size_t max_ctx) {
    return rows * q_heads * (max_ctx + 2) * 4;  // scores [rows][q_heads][max_ctx], then {max, 1/sum}
}

int zg_attn_decode_device(zg_ctx* ctx, size_t rows, size_t q_heads, size_t kv_heads, const float* proj,
                          size_t proj_stride, const float* q_norm, const float* k_norm, float eps, float theta_scale,
                          const int32_t* positions, void* kcache, void* vcache, size_t max_ctx, int kv_dtype,
                          void* workspace, float* out, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!proj || !q_norm || !k_norm || !positions || !kcache || !vcache || !workspace || !out || rows == 0 ||
        rows > 65535 || kv_heads == 0 || q_heads % kv_heads || q_heads / kv_heads > 4 || max_ctx == 0 ||
        max_ctx > (1u << 30) || proj_stride < (2 * q_heads + 2 * kv_heads) * 256 || !(eps > 0.0f) ||
        !(theta_scale > 0.0f && theta_scale <= 1.0f) || (kv_dtype != ZG_BF16 && kv_dtype != ZG_F32))
        return fail(ctx, ZG_E_MALFORMED, "attention decode geometry");
    zg::AttnDecodeArgs a;
    a.proj = proj;
    a.proj_stride = proj_stride;
    a.qnorm = q_norm;
    a.knorm = k_norm;
    a.eps = eps;
    a.theta_scale = theta_scale;
    a.scale = 1.0f / 16.0f;  // 1/sqrt(256)
    a.pos = positions;
    a.kcache = kcache;
    a.vcache = vcache;
    a.cache_row_stride = max_ctx * kv_heads * 256;
    a.kv_bf16 = kv_dtype == ZG_BF16;
    a.scores = (float*)workspace;
    a.score_stride = q_heads * max_ctx;
    a.head_stride = max_ctx;
    a.stats = (float*)workspace + rows * q_heads * max_ctx;
    a.out = out;
    a.out_stride = q_heads * 256;
    a.status = ctx->d_flag;
    a.nq = (int)q_heads;
    a.nkv = (int)kv_heads;
    a.max_ctx = (int)max_ctx;
    ZG_HIP(zg::attn_decode(a, rows, stream ? (hipStream_t)stream : ctx->stream));
    return ZG_COMPLETED;
}

size_t zg_attn_decode_split_workspace_bytes(size_t rows, size_t q_heads, size_t kv_heads, size_t max_ctx) {
    if (rows == 0 || kv_heads == 0 || !zg::attn_split_supported(rows, (int)q_heads, (int)kv_heads, max_ctx)) return 0;
    return zg::attn_split_part_bytes(rows, (int)q_heads, (int)kv_heads, max_ctx);
}

int zg_attn_decode_split_device(zg_ctx* ctx, size_t rows, size_t q_heads, size_t kv_heads, const float* proj,
                                size_t proj_stride, const float* q_norm, const float* k_norm, float eps,
                                float theta_scale, const int32_t* positions, void* kcache, void* vcache,
                                size_t max_ctx, int kv_dtype, void* workspace, float* out, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!proj || !q_norm || !k_norm || !positions || !kcache || !vcache || !workspace || !out || rows == 0 ||
        rows > 65535 || kv_heads == 0 || q_heads % kv_heads || q_heads / kv_heads > 4 || max_ctx == 0 ||
        max_ctx > (1u << 30) || proj_stride < (2 * q_heads + 2 * kv_heads) * 256 || !(eps > 0.0f) ||
        !(theta_scale > 0.0f && theta_scale <= 1.0f) || (kv_dtype != ZG_BF16 && kv_dtype != ZG_F32))
        return fail(ctx, ZG_E_MALFORMED, "attention decode geometry");
    if (!zg::attn_split_supported(rows, (int)q_heads, (int)kv_heads, max_ctx))
        return fail(ctx, ZG_E_LIMIT, "split attention offered for 1..64 rows and up to 262144 cached tokens");
    zg::AttnDecodeArgs a;
    a.proj = proj;
    a.proj_stride = proj_stride;
    a.qnorm = q_norm;
    a.knorm = k_norm;
    a.eps = eps;
    a.theta_scale = theta_scale;
    a.scale = 1.0f / 16.0f;  // 1/sqrt(256)
    a.pos = positions;
    a.kcache = kcache;
    a.vcache = vcache;
    a.cache_row_stride = max_ctx * kv_heads * 256;
    a.kv_bf16 = kv_dtype == ZG_BF16;
    a.out = out;
    a.out_stride = q_heads * 256;
    a.status = ctx->d_flag;
    a.nq = (int)q_heads;
    a.nkv = (int)kv_heads;
    a.max_ctx = (int)max_ctx;
    ZG_HIP(zg::attn_decode_split(a, rows, (float*)workspace, stream ? (hipStream_t)stream : ctx->stream));
    return ZG_COMPLETED;
}

int zg_rope_kv(zg_ctx* ctx, const float* query, const float* key, const float* value, size_t head_width,
               size_t query_heads, size_t kv_heads, size_t rotate, size_t position, float theta_scale, float* query_out,
               float* key_out, float* value_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!query || !key || !value || !query_out || !key_out || !value_out || head_width == 0 || query_heads == 0 ||
        kv_heads == 0 || query_heads % kv_heads || rotate == 0 || rotate > head_width || rotate % 2 ||
        position > 2147483647u || !std::isfinite(theta_scale) || theta_scale <= 0.0f || theta_scale > 1.0f ||
        !all_finite(query, query_heads * head_width) || !all_finite(key, kv_heads * head_width) ||
        !all_finite(value, kv_heads * head_width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source RoPE/KV geometry or FP32 input");
    if (head_width > 256 || rotate > 128) return fail(ctx, ZG_UNSUPPORTED, "RoPE offered for head width <= 256");
    const size_t nq = query_heads * head_width, nk = kv_heads * head_width;
    // The prep kernel reads q from a [q | gate] layout (stride 2*head_width);
    // lay the query out that way.
    std::vector<float> qpad(2 * nq, 0.0f);
    for (size_t h = 0; h < query_heads; ++h)
        std::memcpy(qpad.data() + h * 2 * head_width, query + h * head_width, head_width * 4);
    const size_t oq = 0, ok = align256(2 * nq * 4), ov = ok + align256(nk * 4), op = ov + align256(nk * 4),
                 oqr = op + 256, oko = oqr + align256(nq * 4), ovo = oko + align256(nk * 4);
    int rc = ensure(ctx, ctx->scratch, ovo + align256(nk * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const int p = (int)position;
    ZG_HIP(hipMemcpyAsync(b + oq, qpad.data(), 2 * nq * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ok, key, nk * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ov, value, nk * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + op, &p, 4, hipMemcpyHostToDevice, st));
    zg::AttnArgs a;
    a.B = 1;
    a.nq = (int)query_heads;
    a.nkv = (int)kv_heads;
    a.d = (int)head_width;
    a.rotate = (int)rotate;
    a.do_prep = 1;
    a.prep_only = 1;
    a.norm = 0;
    a.qproj = (const float*)(b + oq);
    a.q_stride = 2 * nq;
    a.kproj = (const float*)(b + ok);
    a.vproj = (const float*)(b + ov);
    a.kv_stride = nk;
    a.pos = (const int*)(b + op);
    a.theta_scale = theta_scale;
    a.qr = (float*)(b + oqr);
    a.qr_stride = nq;
    a.kout = (float*)(b + oko);
    a.vout = (float*)(b + ovo);
    ZG_HIP(zg::rope_prep(a, st));
    ZG_HIP(hipMemcpyAsync(query_out, b + oqr, nq * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(key_out, b + oko, nk * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(value_out, b + ovo, nk * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(query_out, nq) || !all_finite(key_out, nk))
        return fail(ctx, ZG_E_STATE, "incomplete/nonfinite RoPE proposal");
    return ZG_COMPLETED;
}

// QK + softmax + PV regions share one driver over f32 host keys/values.
static int attention_region(zg_ctx* ctx, const float* query, const float* keys, const float* values, size_t tokens,
                            size_t head_width, size_t query_heads, size_t kv_heads, float scale, float* dots,
                            float* scores, float* probs, float* out) {
    const size_t nq = query_heads * head_width, kw = kv_heads * head_width, ns = query_heads * tokens;
    const size_t oq = 0, ok = align256(nq * 4), ov = ok + align256(tokens * kw * 4), on = ov + align256(values ? tokens * kw * 4 : 4),
                 od = on + 256, osc = od + align256(ns * 4), opr = osc + align256(ns * 4),
                 oo = opr + align256(ns * 4);
    int rc = ensure(ctx, ctx->scratch, oo + align256(nq * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const int T = (int)tokens;
    ZG_HIP(hipMemcpyAsync(b + oq, query, nq * 4, hipMemcpyHostToDevice, st));
    if (keys) ZG_HIP(hipMemcpyAsync(b + ok, keys, tokens * kw * 4, hipMemcpyHostToDevice, st));
    if (values) ZG_HIP(hipMemcpyAsync(b + ov, values, tokens * kw * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + on, &T, 4, hipMemcpyHostToDevice, st));
    if (probs && !keys) ZG_HIP(hipMemcpyAsync(b + opr, probs, ns * 4, hipMemcpyHostToDevice, st));
    zg::AttnArgs a;
    a.B = 1;
    a.nq = (int)query_heads;
    a.nkv = (int)kv_heads;
    a.d = (int)head_width;
    a.tmax = T;
    a.kv_bf16 = 0;
    a.qr = (float*)(b + oq);
    a.qr_stride = nq;
    a.kcache = b + ok;
    a.vcache = b + ov;
    a.cache_row_stride = tokens * kw;
    a.ntok = (const int*)(b + on);
    a.scale = scale;
    a.dots = (float*)(b + od);
    a.scores = (float*)(b + osc);
    a.probs = (float*)(b + opr);
    a.score_stride = ns;
    a.out = out ? (float*)(b + oo) : nullptr;
    a.out_stride = nq;
    ZG_HIP(zg::attention_parts(a, keys != nullptr, keys != nullptr, out != nullptr, st));
    if (dots) ZG_HIP(hipMemcpyAsync(dots, b + od, ns * 4, hipMemcpyDeviceToHost, st));
    if (scores) ZG_HIP(hipMemcpyAsync(scores, b + osc, ns * 4, hipMemcpyDeviceToHost, st));
    if (probs && keys) ZG_HIP(hipMemcpyAsync(probs, b + opr, ns * 4, hipMemcpyDeviceToHost, st));
    if (out) ZG_HIP(hipMemcpyAsync(out, b + oo, nq * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

int zg_attention_qk(zg_ctx* ctx, const float* query, const float* keys, size_t tokens, size_t head_width,
                    size_t query_heads, size_t kv_heads, float scale, float* dots, float* scores) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!query || !keys || !dots || !scores || head_width == 0 || query_heads == 0 || kv_heads == 0 ||
        query_heads % kv_heads || tokens == 0 || !std::isfinite(scale) || scale <= 0.0f ||
        !all_finite(query, query_heads * head_width) || !all_finite(keys, tokens * kv_heads * head_width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source attention QK region");
    if (head_width != 256 || query_heads / kv_heads > 4)
        return fail(ctx, ZG_UNSUPPORTED, "attention offered for head width 256, GQA group <= 4");
    const size_t ns = query_heads * tokens;
    std::vector<float> probs(ns);
    int rc = attention_region(ctx, query, keys, nullptr, tokens, head_width, query_heads, kv_heads, scale, dots, scores,
                              probs.data(), nullptr);
    if (rc) return rc;
    for (size_t i = 0; i < ns; ++i)
        if (!std::isfinite(dots[i]) || scores[i] != dots[i] * scale)
            return fail(ctx, ZG_E_STATE, "incomplete/nonfinite QK proposal or wrong source scale");
    return ZG_COMPLETED;
}

int zg_attention_softmax(zg_ctx* ctx, const float* scores, size_t heads, size_t width, float* probabilities) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!scores || !probabilities || heads == 0 || width == 0 || !all_finite(scores, heads * width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source attention softmax region");
    const size_t ns = heads * width;
    const size_t osc = 0, on = align256(ns * 4), opr = on + 256;
    int rc = ensure(ctx, ctx->scratch, opr + align256(ns * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const int T = (int)width;
    ZG_HIP(hipMemcpyAsync(b + osc, scores, ns * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + on, &T, 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::softmax_rows((const float*)(b + osc), ns, (const int*)(b + on), (float*)(b + opr), heads, 1, st));
    ZG_HIP(hipMemcpyAsync(probabilities, b + opr, ns * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    for (size_t i = 0; i < ns; ++i)
        if (!std::isfinite(probabilities[i]) || probabilities[i] < 0.0f || probabilities[i] > 1.0f)
            return fail(ctx, ZG_E_STATE, "invalid source softmax probability");
    return ZG_COMPLETED;
}

int zg_attention_value(zg_ctx* ctx, const float* probabilities, const float* values, size_t tokens, size_t head_width,
                       size_t query_heads, size_t kv_heads, float* out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!probabilities || !values || !out || head_width == 0 || query_heads == 0 || kv_heads == 0 ||
        query_heads % kv_heads || tokens == 0 || !all_finite(values, tokens * kv_heads * head_width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source attention value region");
    for (size_t i = 0; i < query_heads * tokens; ++i)
        if (!std::isfinite(probabilities[i]) || std::signbit(probabilities[i]) || probabilities[i] > 1.0f)
            return fail(ctx, ZG_E_MALFORMED, "invalid source attention value region");
    if (head_width != 256 || query_heads / kv_heads > 4)
        return fail(ctx, ZG_UNSUPPORTED, "attention offered for head width 256, GQA group <= 4");
    std::vector<float> dummy(query_heads * head_width);
    int rc = attention_region(ctx, dummy.data(), nullptr, values, tokens, head_width, query_heads, kv_heads, 1.0f,
                              nullptr, nullptr, const_cast<float*>(probabilities), out);
    if (rc) return rc;
    if (!all_finite(out, query_heads * head_width))
        return fail(ctx, ZG_E_STATE, "incomplete/nonfinite source attention value proposal");
    return ZG_COMPLETED;
}

// greedy_finite (core/src/numerics.rs:124-140) on the device for `rows`
// rows of n logits: the first maximum wins (a later equal value, +0 after
// -0 included, never replaces it), a nonfinite logit is ZG_E_STATE and an
// empty or over-long vocabulary ZG_E_LIMIT.  The decode step's own greedy
// readout runs these kernels.  out[rows].
int zg_greedy(zg_ctx* ctx, const float* logits, size_t rows, size_t n, uint32_t* out) {
    if (!ctx || !logits || !out || rows == 0 || rows > 65535) return fail(ctx, ZG_E_MALFORMED, "invalid greedy arguments");
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (n == 0 || n > 0x7fffffffu) return fail(ctx, ZG_E_LIMIT, "greedy vocabulary extent");
    const size_t o_pm = align256(rows * n * 4), o_pi = o_pm + align256(zg::argmax_partials(rows) * 4),
                 o_gr = o_pi + align256(zg::argmax_partials(rows) * 4), o_st = o_gr + align256(rows * 4);
    int rc = ensure(ctx, ctx->scratch, o_st + 256);
    if (rc) return rc;
    char* base = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    ZG_HIP(hipMemsetAsync(base + o_st, 0, 4, st));
    ZG_HIP(hipMemcpyAsync(base, logits, rows * n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::argmax_step((const float*)base, n, n, rows, (uint32_t*)(base + o_gr), (int*)(base + o_st),
                           (float*)(base + o_pm), (int*)(base + o_pi), nullptr, st));
    int status = 0;
    ZG_HIP(hipMemcpyAsync(out, base + o_gr, rows * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(&status, base + o_st, 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (status) return fail(ctx, ZG_E_STATE, "greedy requires finite logits");
    return ZG_COMPLETED;
}

}  // extern "C"
