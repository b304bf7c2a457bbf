// C ABI of the gfx950 backend (include/zg_hip.h): context, resident weight
// cache, boundary-A region entry points and the device GEMV API.
#include <cmath>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "zg_context.hpp"

// Activation scratch of zg_gemv_device_noalloc: one array per GPU, held for
// the life of the process.  Host code never passes `scratch` itself to a
// kernel (the name is a host-side stand-in); zg_ctx_create looks up each
// device's address with hipGetSymbolAddress and keeps it in the context.
constexpr size_t kStaticScratchBytes = (size_t)4 << 20;
constexpr size_t kStaticScratchRows = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// Per device: the event recorded after the last use of that device's array
// (created with the first context on the device, kept for the process).
constexpr int kMaxDevices = 64;
struct ScratchOrder {
    std::mutex mu;
    hipEvent_t ev = nullptr;
    bool used = false;
};
static ScratchOrder g_scratch_order[kMaxDevices];

// The device's scratch-order event, created once (with that device current).
static bool scratch_order_event(int device) {
    ScratchOrder& so = g_scratch_order[device];
    std::lock_guard<std::mutex> lk(so.mu);
    if (!so.ev && hipEventCreateWithFlags(&so.ev, hipEventDisableTiming) != hipSuccess) {
        so.ev = nullptr;
        return false;
    }
    return true;
}

namespace zgc {

// Failure text per (thread, ctx): under the reference's Send + Sync
// contract (core/src/accelerator.rs:682) two threads may fail on one ctx at
// once, and each reads its own message back.  Only thread-local data is
// written, so fail() needs no lock; entries are keyed by the context's
// serial number, never reused within a process.
thread_local std::map<uint64_t, std::string> t_errors;
std::atomic<uint64_t> g_ctx_serial{1};

int fail(zg_ctx* ctx, int code, const std::string& msg) {
    if (ctx) t_errors[ctx->serial] = msg;
    return code;
}

std::string last_message(const zg_ctx* ctx) {
    if (!ctx) return "";
    auto it = t_errors.find(ctx->serial);
    return it == t_errors.end() ? std::string() : it->second;
}

void drop_weight(zg_ctx* ctx, zg_weight* w) {
    (void)hipDeviceSynchronize();
    for (auto it = ctx->weights.begin(); it != ctx->weights.end(); ++it)
        if (it->second.get() == w) {
            free_weight(w);
            ctx->weights.erase(it);
            return;
        }
}


bool all_finite(const float* x, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(x[i])) return false;
    return true;
}

int ensure(zg_ctx* ctx, DeviceBuffer& b, size_t bytes) {
    if (b.bytes >= bytes) return ZG_COMPLETED;
    if (b.ptr) {
        ZG_HIP(hipStreamSynchronize(ctx->stream));
        ZG_HIP(hipFree(b.ptr));
        b.ptr = nullptr;
        b.bytes = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    ZG_HIP(hipMalloc(&b.ptr, want));
    b.bytes = want;
    return ZG_COMPLETED;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

void free_weight(zg_weight* w) {
    if (!w) return;
    if (w->dw.qs) (void)hipFree(w->dw.qs);
    if (w->dw.hdr) (void)hipFree(w->dw.hdr);
    if (w->dw.qs_t) (void)hipFree(w->dw.qs_t);
    if (w->dw.hdr_t) (void)hipFree(w->dw.hdr_t);
    w->dw.qs = w->dw.hdr = w->dw.qs_t = w->dw.hdr_t = nullptr;
}

bool supported_type(int t) { return t == ZG_Q8_0 || t == ZG_Q4_K || t == ZG_F32 || t == ZG_Q4_1 || t == ZG_Q6_K; }

size_t block_elems(int t) { return (t == ZG_Q8_0 || t == ZG_Q4_1) ? 32 : (t == ZG_Q4_K || t == ZG_Q6_K) ? 256 : 1; }

// Upload and split one GGUF matrix.  Caller holds the ctx lock.
int build_weight(zg_ctx* ctx, int type, size_t cols, size_t rows, const void* bytes, size_t len,
                 std::unique_ptr<zg_weight>& out) {
    auto w = std::make_unique<zg_weight>();
    w->dw.type = type;
    w->dw.K = cols;
    w->dw.N = rows;
    if (type == ZG_Q8_0) {
        const size_t nbc = (cols / 32 + 3) / 4;
        w->dw.qs_bytes = (rows + 7) / 8 * nbc * 1024;
        w->dw.hdr_bytes = rows * nbc * 4 * 2;
    } else if (type == ZG_Q4_K) {
        const size_t rows16 = (rows + 15) / 16 * 16;  // q4k_chunk_offset's 16-row tiles
        w->dw.qs_bytes = rows16 * (cols / 2);
        w->dw.hdr_bytes = rows16 * (cols / 256) * 16;
    } else if (type == ZG_Q4_1) {
        const size_t nbc8 = (cols / 32 + 7) / 8;
        w->dw.qs_bytes = (rows + 7) / 8 * nbc8 * 1024;
        w->dw.hdr_bytes = rows * nbc8 * 8 * 4;
    } else if (type == ZG_Q6_K) {
        w->dw.qs_bytes = (rows + 7) / 8 * (cols / 256) * 64 * 24;
        w->dw.hdr_bytes = rows * (cols / 256) * 20;
    } else {
        w->dw.qs_bytes = rows * cols * 4;
        w->dw.hdr_bytes = 0;
    }
    void* staging = nullptr;
    ZG_HIP(hipMalloc(&w->dw.qs, w->dw.qs_bytes));
    if (w->dw.hdr_bytes) ZG_HIP(hipMalloc(&w->dw.hdr, w->dw.hdr_bytes));
    hipError_t e = hipMalloc(&staging, len);
    if (e != hipSuccess) {
        free_weight(w.get());
        return fail(ctx, ZG_E_RESOURCE, std::string("weight staging allocation: ") + hipGetErrorString(e));
    }
    ZG_HIP(hipMemsetAsync(ctx->d_flag, 0, sizeof(int), ctx->stream));
    ZG_HIP(hipMemcpyAsync(staging, bytes, len, hipMemcpyHostToDevice, ctx->stream));
    ZG_HIP(zg::repack_weight((const uint8_t*)staging, w->dw, ctx->d_flag, ctx->stream));
    int bad = 0;
    ZG_HIP(hipMemcpyAsync(&bad, ctx->d_flag, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    ZG_HIP(hipFree(staging));
    if (bad) {
        free_weight(w.get());
        return fail(ctx, ZG_E_MALFORMED, "nonfinite GGUF block scale");
    }
    out = std::move(w);
    return ZG_COMPLETED;
}

int check_matrix(zg_ctx* ctx, int type, size_t cols, size_t rows, const void* bytes, size_t len) {
    if (!bytes || cols == 0 || rows == 0 || rows > 1000000)
        return fail(ctx, ZG_E_MALFORMED, "invalid matrix geometry");
    if (!supported_type(type)) return fail(ctx, ZG_UNSUPPORTED, "ggml type not offered by this backend");
    if (cols % block_elems(type)) return fail(ctx, ZG_E_MALFORMED, "row not aligned to whole blocks");
    if (zg::gguf_row_bytes(type, cols) * rows != len) return fail(ctx, ZG_E_MALFORMED, "packed byte length mismatch");
    return ZG_COMPLETED;
}

int lookup_or_register(zg_ctx* ctx, uint64_t source, const char* name, int type, size_t cols, size_t rows,
                       const void* bytes, size_t len, zg_weight** out) {
    auto key = std::make_tuple(source, std::string(name), type, cols, rows);
    auto it = ctx->weights.find(key);
    if (it != ctx->weights.end()) {
        *out = it->second.get();
        return ZG_COMPLETED;
    }
    std::unique_ptr<zg_weight> w;
    int rc = build_weight(ctx, type, cols, rows, bytes, len, w);
    if (rc != ZG_COMPLETED) return rc;
    w->source = source;
    w->name = name;
    *out = w.get();
    ctx->weights.emplace(key, std::move(w));
    return ZG_COMPLETED;
}

}  // namespace zgc

using namespace zgc;

extern "C" {

const char* zg_version(void) { return "zerogravity_amd 0.1.0 (gfx950)"; }

int zg_ctx_create(int device, zg_ctx** out) {
    if (!out) return ZG_E_MALFORMED;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count || device >= kMaxDevices)
        return ZG_E_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return ZG_E_DEVICE;
    auto ctx = new zg_ctx();
    ctx->device = device;
    ctx->serial = g_ctx_serial.fetch_add(1);
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc(&ctx->d_flag, sizeof(int)) != hipSuccess ||
        hipGetSymbolAddress(&ctx->static_scratch, HIP_SYMBOL(scratch)) != hipSuccess || !ctx->static_scratch ||
        !scratch_order_event(device)) {
        if (ctx->d_flag) (void)hipFree(ctx->d_flag);
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return ZG_E_DEVICE;
    }
    *out = ctx;
    return ZG_COMPLETED;
}

void zg_ctx_destroy(zg_ctx* ctx) {
    if (!ctx) return;
    {
        std::lock_guard<std::recursive_mutex> g(ctx->mu);
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        for (auto& kv : ctx->weights) free_weight(kv.second.get());
        ctx->weights.clear();
        if (ctx->scratch.ptr) (void)hipFree(ctx->scratch.ptr);
        if (ctx->actbuf.ptr) (void)hipFree(ctx->actbuf.ptr);
        if (ctx->chunkbuf.ptr) (void)hipFree(ctx->chunkbuf.ptr);
        if (ctx->d_flag) (void)hipFree(ctx->d_flag);
        (void)hipStreamDestroy(ctx->stream);
    }
    t_errors.erase(ctx->serial);
    delete ctx;
}

const char* zg_last_error(const zg_ctx* ctx) {
    if (!ctx) return "null context";
    auto it = t_errors.find(ctx->serial);
    return it == t_errors.end() ? "" : it->second.c_str();
}

int zg_weight_register(zg_ctx* ctx, uint64_t source_id, const char* name, int ggml_type, size_t columns,
                       size_t rows, const void* bytes, size_t len, zg_weight** out) {
    if (!ctx || !out || !name || !*name) return fail(ctx, ZG_E_MALFORMED, "invalid registration arguments");
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (source_id == 0) return fail(ctx, ZG_E_MALFORMED, "unbound source identity cannot key a resident weight");
    int rc = check_matrix(ctx, ggml_type, columns, rows, bytes, len);
    if (rc == ZG_UNSUPPORTED) return fail(ctx, ZG_E_UNSUPPORTED, last_message(ctx));
    if (rc != ZG_COMPLETED) return rc;
    rc = lookup_or_register(ctx, source_id, name, ggml_type, columns, rows, bytes, len, out);
    if (rc == ZG_COMPLETED) (*out)->api_pinned = true;
    return rc;
}

int zg_source_release(zg_ctx* ctx, uint64_t source_id) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    ZG_HIP(hipDeviceSynchronize());
    // weights a loaded model still uses stay until its zg_model_destroy
    for (auto it = ctx->weights.begin(); it != ctx->weights.end();) {
        zg_weight* w = it->second.get();
        if (std::get<0>(it->first) == source_id) {
            w->api_pinned = false;
            if (w->model_refs == 0) {
                free_weight(w);
                it = ctx->weights.erase(it);
                continue;
            }
        }
        ++it;
    }
    return ZG_COMPLETED;
}

size_t zg_weight_device_bytes(const zg_weight* w) { return w ? w->dw.qs_bytes + w->dw.hdr_bytes : 0; }

int zg_weight_dequantize(zg_ctx* ctx, const zg_weight* w, float* out, size_t out_len) {
    if (!ctx || !w || !out) return fail(ctx, ZG_E_MALFORMED, "invalid arguments");
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    const size_t n = w->dw.N * w->dw.K;
    if (out_len != n) return fail(ctx, ZG_E_MALFORMED, "output length mismatch");
    int rc = ensure(ctx, ctx->scratch, n * 4);
    if (rc) return rc;
    ZG_HIP(zg::dequantize_rows(w->dw, 0, w->dw.N, (float*)ctx->scratch.ptr, ctx->stream));
    ZG_HIP(hipMemcpyAsync(out, ctx->scratch.ptr, n * 4, hipMemcpyDeviceToHost, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    return ZG_COMPLETED;
}

int zg_matvec(zg_ctx* ctx, uint64_t source_id, const char* tensor_name, int ggml_type, size_t columns, size_t rows,
              const void* packed_weights, size_t packed_len, const float* activation, size_t activation_len,
              float* out, size_t out_len) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!tensor_name || !*tensor_name || !activation || !out || activation_len != columns || out_len != rows)
        return fail(ctx, ZG_E_MALFORMED, "invalid matvec region");
    int rc = check_matrix(ctx, ggml_type, columns, rows, packed_weights, packed_len);
    if (rc != ZG_COMPLETED) return rc;
    if (!all_finite(activation, columns)) return fail(ctx, ZG_E_MALFORMED, "nonfinite GEMV input");
    if (!zg::gemv_supported(ggml_type, columns, 1)) return fail(ctx, ZG_UNSUPPORTED, "geometry not offered");
    zg_weight* w = nullptr;
    std::unique_ptr<zg_weight> temp;
    if (source_id != 0) {
        rc = lookup_or_register(ctx, source_id, tensor_name, ggml_type, columns, rows, packed_weights, packed_len, &w);
        if (rc) return rc;
        w->api_pinned = true;  // resident for the bound source until zg_source_release
    } else {
        rc = build_weight(ctx, ggml_type, columns, rows, packed_weights, packed_len, temp);
        if (rc) return rc;
        w = temp.get();
    }
    const size_t prep = zg::prepared_bytes(ggml_type, 1, columns);
    const size_t oy = align256(columns * 4) + align256(prep);
    rc = ensure(ctx, ctx->scratch, oy + align256(rows * 4));
    if (rc) {
        free_weight(temp.get());
        return rc;
    }
    char* base = (char*)ctx->scratch.ptr;
    float* xf = (float*)base;
    void* prepared = base + align256(columns * 4);
    float* y = (float*)(base + oy);
    ZG_HIP(hipMemcpyAsync(xf, activation, columns * 4, hipMemcpyHostToDevice, ctx->stream));
    ZG_HIP(zg::act_prepare_for(ggml_type, xf, 0, 1, columns, nullptr, 0.0f, prepared, ctx->stream));
    ZG_HIP(zg::gemv(w->dw, 1, prepared, y, ctx->stream));
    ZG_HIP(hipMemcpyAsync(out, y, rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    free_weight(temp.get());
    if (!all_finite(out, rows)) return fail(ctx, ZG_E_STATE, std::string("nonfinite result from matrix '") + tensor_name + "'");
    return ZG_COMPLETED;
}

int zg_embedding(zg_ctx* ctx, uint64_t source_id, const char* tensor_name, int ggml_type, const void* packed_weights,
                 size_t packed_len, uint32_t token, size_t width, size_t vocabulary, float* out, size_t out_len) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!tensor_name || !*tensor_name || !out || out_len != width || width == 0 || vocabulary == 0 || token >= vocabulary)
        return fail(ctx, ZG_E_MALFORMED, "invalid original source embedding region");
    int rc = check_matrix(ctx, ggml_type, width, vocabulary, packed_weights, packed_len);
    if (rc != ZG_COMPLETED) return rc;
    zg_weight* w = nullptr;
    std::unique_ptr<zg_weight> temp;
    if (source_id != 0) {
        rc = lookup_or_register(ctx, source_id, tensor_name, ggml_type, width, vocabulary, packed_weights, packed_len, &w);
        if (rc) return rc;
        w->api_pinned = true;
    } else {
        // Unbound: upload only the selected row.
        const size_t rb = zg::gguf_row_bytes(ggml_type, width);
        rc = build_weight(ctx, ggml_type, width, 1, (const char*)packed_weights + (size_t)token * rb, rb, temp);
        if (rc) return rc;
        w = temp.get();
        token = 0;
    }
    rc = ensure(ctx, ctx->scratch, width * 4);
    if (rc) return rc;
    ZG_HIP(zg::dequantize_rows(w->dw, token, 1, (float*)ctx->scratch.ptr, ctx->stream));
    ZG_HIP(hipMemcpyAsync(out, ctx->scratch.ptr, width * 4, hipMemcpyDeviceToHost, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    free_weight(temp.get());
    if (!all_finite(out, width)) return fail(ctx, ZG_E_STATE, "incomplete/nonfinite source embedding proposal");
    return ZG_COMPLETED;
}

}  // extern "C"

// Shared driver for the pointwise regions: upload n-float inputs, run, read back.
namespace {
template <typename F>
int run_pointwise(zg_ctx* ctx, size_t n_in, const float* const* ins, const size_t* lens, size_t n_out, float* out,
                  F launch) {
    size_t off[4] = {0, 0, 0, 0}, total = 0;
    for (size_t i = 0; i < n_in; ++i) {
        off[i] = total;
        total += align256(lens[i] * 4);
    }
    const size_t oo = total;
    total += align256(n_out * 4);
    int rc = ensure(ctx, ctx->scratch, total);
    if (rc) return rc;
    char* base = (char*)ctx->scratch.ptr;
    const float* dev[4] = {nullptr, nullptr, nullptr, nullptr};
    for (size_t i = 0; i < n_in; ++i) {
        if (ins[i]) {
            ZG_HIP(hipMemcpyAsync(base + off[i], ins[i], lens[i] * 4, hipMemcpyHostToDevice, ctx->stream));
            dev[i] = (const float*)(base + off[i]);
        }
    }
    ZG_HIP(launch(dev, (float*)(base + oo)));
    ZG_HIP(hipMemcpyAsync(out, base + oo, n_out * 4, hipMemcpyDeviceToHost, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    return ZG_COMPLETED;
}
}  // namespace

extern "C" {

int zg_rms_norm(zg_ctx* ctx, const float* input, const float* weights, size_t n, float eps, float* out) {
    return zg_grouped_rms_norm(ctx, input, weights, n, 1, eps, out);
}

int zg_grouped_rms_norm(zg_ctx* ctx, const float* input, const float* weights, size_t width, size_t groups, float eps,
                        float* out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!input || !weights || !out || width == 0 || groups == 0 || !std::isfinite(eps) || eps <= 0.0f)
        return fail(ctx, ZG_E_MALFORMED, "invalid grouped RMS normalization dimensions");
    if (!all_finite(input, width * groups)) return fail(ctx, ZG_E_MALFORMED, "nonfinite RMSNorm input");
    const float* ins[2] = {input, weights};
    const size_t lens[2] = {width * groups, width};
    int rc = run_pointwise(ctx, 2, ins, lens, width * groups, out, [&](const float* const* d, float* o) {
        return zg::rms_groups(d[0], d[1], width, groups, eps, o, ctx->stream);
    });
    if (rc) return rc;
    if (!all_finite(out, width * groups)) return fail(ctx, ZG_E_STATE, "physical normalization output malformed");
    return ZG_COMPLETED;
}

int zg_silu(zg_ctx* ctx, const float* input, const float* multiplier, size_t n, float* out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!input || !out || n == 0 || !all_finite(input, n) || (multiplier && !all_finite(multiplier, n)))
        return fail(ctx, ZG_E_MALFORMED, "invalid source SiLU inputs");
    const float* ins[2] = {input, multiplier};
    const size_t lens[2] = {n, multiplier ? n : 0};
    int rc = run_pointwise(ctx, 2, ins, lens, n, out, [&](const float* const* d, float* o) {
        return zg::silu(d[0], d[1], n, o, ctx->stream);
    });
    if (rc) return rc;
    if (!all_finite(out, n)) return fail(ctx, ZG_E_STATE, "physical SiLU output malformed");
    return ZG_COMPLETED;
}

int zg_binary(zg_ctx* ctx, int kind, const float* left, const float* right, size_t n, float* out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!left || !right || !out || n == 0 || (kind != 0 && kind != 1) || !all_finite(left, n) || !all_finite(right, n))
        return fail(ctx, ZG_E_MALFORMED, "invalid source binary region");
    const float* ins[2] = {left, right};
    const size_t lens[2] = {n, n};
    int rc = run_pointwise(ctx, 2, ins, lens, n, out, [&](const float* const* d, float* o) {
        return zg::binary(kind, d[0], d[1], n, o, ctx->stream);
    });
    if (rc) return rc;
    if (!all_finite(out, n)) return fail(ctx, ZG_E_STATE, "incomplete/nonfinite source binary proposal");
    return ZG_COMPLETED;
}

// ------------------------------------------------------------- device API

size_t zg_act_prepared_bytes(const zg_weight* w, size_t m_rows) {
    return w ? zg::prepared_bytes(w->dw.type, m_rows, w->dw.K) : 0;
}

int zg_act_prepare_device(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows,
                          const float* gamma, float eps, void* prepared, size_t prepared_len, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!w || !x || !prepared || m_rows == 0 || (x_dtype != ZG_BF16 && x_dtype != ZG_F32))
        return fail(ctx, ZG_E_MALFORMED, "invalid activation preparation");
    if (prepared_len < zg::prepared_bytes(w->dw.type, m_rows, w->dw.K))
        return fail(ctx, ZG_E_MALFORMED, "prepared activation buffer too small");
    if (!zg::gemv_supported(w->dw.type, w->dw.K, m_rows)) return fail(ctx, ZG_UNSUPPORTED, "geometry not offered");
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    ZG_HIP(zg::act_prepare_for(w->dw.type, x, x_dtype == ZG_BF16, m_rows, w->dw.K, gamma, eps, prepared, s));
    return ZG_COMPLETED;
}

int zg_gemv_prepared_device(zg_ctx* ctx, const zg_weight* w, size_t m_rows, const void* prepared, float* y,
                            void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!w || !y || !prepared) return fail(ctx, ZG_E_MALFORMED, "invalid gemv arguments");
    if (!zg::gemv_supported(w->dw.type, w->dw.K, m_rows)) return fail(ctx, ZG_UNSUPPORTED, "geometry not offered");
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    ZG_HIP(zg::gemv(w->dw, m_rows, prepared, y, s));
    return ZG_COMPLETED;
}

// f32 activations of a Q4_K weight from two rows on take the f16 MFMA
// kernels (weights read and dequantised once for all rows); measured per
// launch they beat the byte-dot kernel from two rows on.  Q8_0 beyond four
// rows takes the coded-once activation and one weight stream per 16 rows.
static bool device_batched(const zg_weight* w, size_t m_rows, int pro) {
    return (m_rows >= 2 && w->dw.type == zg::kQ4_K) ||
           (m_rows > 4 && w->dw.type == zg::kQ8_0 && zg::q8_rows_supported(w->dw.K, w->dw.N, pro)) ||
           (m_rows > 4 && w->dw.type == zg::kQ6_K && zg::q6k_rows_supported(w->dw.K, w->dw.N, pro));
}

int zg_gemv_device(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows, const float* gamma,
                   float eps, float* y, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!w || !x || !y || (x_dtype != ZG_BF16 && x_dtype != ZG_F32)) return fail(ctx, ZG_E_MALFORMED, "invalid gemv arguments");
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    const int pro = gamma ? zg::PRO_RMS : zg::PRO_PLAIN;
    if (x_dtype == ZG_F32 && m_rows > 0 && m_rows <= 65536 && zg::fused_gemv_supported(w->dw.type, w->dw.K, w->dw.N, pro)) {
        // f32 activations: the decode-step kernels themselves (one row: the
        // int8-MFMA GEMV; Q4_K from two rows: f16 MFMA; Q8_0 beyond four
        // rows: the coded-once activation; otherwise the activation prologue
        // in-kernel)
        zg::FusedGemvArgs f;
        f.M = (int)m_rows;
        f.pro = pro;
        f.epi = zg::EPI_STORE;
        f.x = (const float*)x;
        f.ldx = w->dw.K;
        f.gamma = gamma;
        f.eps = eps;
        f.y = y;
        f.ldy = w->dw.N;
        f.status = ctx->d_flag;
        if (device_batched(w, m_rows, pro)) {
            // Q4_K: the 32-row weight tiles, unless the 16-row kernel takes this shape
            if (w->dw.type == zg::kQ4_K && !w->dw.qs_t &&
                !zg::batched16_supported(m_rows, w->dw.K, w->dw.N, zg::EPI_STORE)) {
                ZG_HIP(hipStreamSynchronize(s));
                ZG_HIP(zg::ensure_mfma_tiles(const_cast<zg_weight*>(w)->dw, s));
            }
            const size_t need = zg::batched_scratch_bytes(m_rows, w->dw.K);
            if (ctx->actbuf.bytes < need) ZG_HIP(hipStreamSynchronize(s));
            int rc = ensure(ctx, ctx->actbuf, need);
            if (rc) return rc;
            ZG_HIP(zg::batched_gemv(w->dw, f, ctx->actbuf.ptr, s));
        } else {
            ZG_HIP(zg::fused_gemv(w->dw, f, s));
        }
        return ZG_COMPLETED;
    }
    if (!zg::gemv_supported(w->dw.type, w->dw.K, m_rows)) return fail(ctx, ZG_UNSUPPORTED, "geometry not offered");
    const size_t need = zg::prepared_bytes(w->dw.type, m_rows, w->dw.K);
    if (ctx->actbuf.bytes < need) {
        // Growing the buffer must not race work still queued on the caller stream.
        ZG_HIP(hipStreamSynchronize(s));
    }
    int rc = ensure(ctx, ctx->actbuf, need);
    if (rc) return rc;
    ZG_HIP(zg::act_prepare_for(w->dw.type, x, x_dtype == ZG_BF16, m_rows, w->dw.K, gamma, eps, ctx->actbuf.ptr, s));
    ZG_HIP(zg::gemv(w->dw, m_rows, ctx->actbuf.ptr, y, s));
    return ZG_COMPLETED;
}

static_assert(ZG_PRO_RMS == zg::PRO_RMS && ZG_PRO_GATED == zg::PRO_GATED && ZG_PRO_SILU_MUL == zg::PRO_SILU_MUL &&
                  ZG_PRO_PLAIN == zg::PRO_PLAIN && ZG_PRO_GATED_PRE == zg::PRO_GATED_PRE &&
                  ZG_EPI_STORE == zg::EPI_STORE && ZG_EPI_RESID == zg::EPI_RESID &&
                  ZG_EPI_GLU == zg::EPI_GLU,
              "C-ABI prologue/epilogue codes are the kernels' own");

size_t zg_gemv_greedy_parts(const zg_weight* w) {
    return w ? (size_t)zg::gemv1_greedy_parts(w->dw, zg::PRO_RMS) : 0;
}

// One projection of the decode step with its fused prologue and epilogue,
// through the dispatcher the step itself calls (zg::fused_gemv), so the
// same kernel and template variant runs for the same (weight, prologue,
// epilogue, rows).
int zg_gemv_device_fused(zg_ctx* ctx, const zg_weight* w, size_t m_rows, int prologue, int epilogue, float* x,
                         size_t ldx, const float* x2, size_t ldx2, const float* gamma, float eps, size_t group,
                         float* y, size_t ldy, const zg_weight* embedding, const uint32_t* token, float* greedy_max,
                         int32_t* greedy_idx, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!w || !x || !y || m_rows == 0 || m_rows > 4 ||
        !(prologue == ZG_PRO_RMS || prologue == ZG_PRO_GATED || prologue == ZG_PRO_SILU_MUL ||
          prologue == ZG_PRO_PLAIN || prologue == ZG_PRO_GATED_PRE) ||
        epilogue < ZG_EPI_STORE || epilogue > ZG_EPI_GLU)
        return fail(ctx, ZG_E_MALFORMED, "invalid fused gemv arguments");
    const size_t K = w->dw.K, N = w->dw.N;
    const bool needs_x2 = prologue == ZG_PRO_GATED || prologue == ZG_PRO_SILU_MUL || prologue == ZG_PRO_GATED_PRE;
    const bool needs_gamma = prologue == ZG_PRO_RMS || prologue == ZG_PRO_GATED;
    if ((needs_x2 && !x2) || (needs_gamma && !gamma) || ldx < K || (needs_x2 && ldx2 < K) ||
        ldy < (epilogue == ZG_EPI_GLU ? N / 2 : N) || !(eps > 0.0f || !needs_gamma))
        return fail(ctx, ZG_E_MALFORMED, "fused gemv operand missing or stride too short");
    if (prologue == ZG_PRO_GATED && (group == 0 || K % group)) return fail(ctx, ZG_E_MALFORMED, "gated norm group");
    if (prologue == ZG_PRO_GATED_PRE && (m_rows != 1 || group != 128 || epilogue == ZG_EPI_GLU ||
                                         !zg::gated_pre_supported(w->dw)))
        return fail(ctx, ZG_UNSUPPORTED, "formed gated product: one row, group 128, matrix-core Q4_K GEMV");
    if (!zg::fused_gemv_supported(w->dw.type, K, N, prologue))
        return fail(ctx, ZG_UNSUPPORTED, "no fused projection kernel for this weight and prologue");
    if (epilogue == ZG_EPI_GLU && !zg::fused_glu_supported(w->dw.type, K, N))
        return fail(ctx, ZG_UNSUPPORTED, "no SwiGLU epilogue for this weight");
    const bool greedy = greedy_max || greedy_idx;
    if (greedy && (!greedy_max || !greedy_idx || m_rows != 1 || epilogue != ZG_EPI_STORE ||
                   prologue != ZG_PRO_RMS || zg::gemv1_greedy_parts(w->dw, zg::PRO_RMS) <= 0))
        return fail(ctx, ZG_UNSUPPORTED, "greedy partials: one row, RMS prologue, store epilogue, matrix-core GEMV");
    if ((embedding || token) && (!embedding || !token || m_rows != 1 || prologue != ZG_PRO_RMS ||
                                 !zg::gemv1_embed_supported(w->dw, embedding->dw)))
        return fail(ctx, ZG_UNSUPPORTED, "embedding prologue: one row, RMS prologue, Q4_K embedding of width K");
    zg::FusedGemvArgs f;
    f.M = (int)m_rows;
    f.pro = prologue;
    f.epi = epilogue;
    f.x = x;
    f.ldx = ldx;
    f.x2 = x2;
    f.ldx2 = ldx2;
    f.gamma = gamma;
    f.eps = eps;
    f.group = (int)group;
    f.y = y;
    f.ldy = ldy;
    f.status = ctx->d_flag;
    if (greedy) {
        f.amax = greedy_max;
        f.aidx = greedy_idx;
    }
    if (embedding) {
        f.tok = token;
        f.emb_qs = embedding->dw.qs;
        f.emb_hdr = embedding->dw.hdr;
        f.emb_rows = (int)embedding->dw.N;
        f.x_out = x;
    }
    ZG_HIP(zg::fused_gemv(w->dw, f, stream ? (hipStream_t)stream : ctx->stream));
    return ZG_COMPLETED;
}


// zg_gemv_device with its activation scratch in the process-wide static
// array instead of a context buffer: no allocation on any path.  The same
// kernels in the same order, so the result is bit-identical.
int zg_gemv_device_noalloc(zg_ctx* ctx, const zg_weight* w, const void* x, int x_dtype, size_t m_rows,
                           const float* gamma, float eps, float* y, void* stream) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!w || !x || !y || (x_dtype != ZG_BF16 && x_dtype != ZG_F32)) return fail(ctx, ZG_E_MALFORMED, "invalid gemv arguments");
    if (m_rows == 0 || m_rows > kStaticScratchRows)
        return fail(ctx, ZG_E_LIMIT, "allocation-free GEMV takes 1 to 64 activation rows");
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    void* sp = ctx->static_scratch;
    const int pro = gamma ? zg::PRO_RMS : zg::PRO_PLAIN;
    const bool fused = x_dtype == ZG_F32 && zg::fused_gemv_supported(w->dw.type, w->dw.K, w->dw.N, pro);
    const bool batched = fused && device_batched(w, m_rows, pro);
    if (batched) {
        if (w->dw.type == zg::kQ4_K && !w->dw.qs_t && !zg::batched16_supported(m_rows, w->dw.K, w->dw.N, zg::EPI_STORE))
            return fail(ctx, ZG_E_STATE,
                        "weight has no batched tile layout yet: a zg_gemv_device call of this shape with 2 or more rows builds it");
        if (zg::batched_scratch_bytes(m_rows, w->dw.K) > kStaticScratchBytes)
            return fail(ctx, ZG_E_LIMIT, "activation exceeds the 4 MiB static scratch");
    } else if (!fused) {
        if (!zg::gemv_supported(w->dw.type, w->dw.K, m_rows)) return fail(ctx, ZG_UNSUPPORTED, "geometry not offered");
        if (zg::prepared_bytes(w->dw.type, m_rows, w->dw.K) > kStaticScratchBytes)
            return fail(ctx, ZG_E_LIMIT, "activation exceeds the 4 MiB static scratch");
    }
    // Uses of the device's array are ordered across streams, threads and
    // contexts: each call waits on the event the previous call recorded
    // after its kernels and records it after its own.  A call made while
    // its stream is being captured into a graph is ordered by the graph's
    // stream order instead (an event recorded outside a capture cannot be
    // waited on inside it); replaying such a graph beside other uses of the
    // array on the device races.
    ScratchOrder& so = g_scratch_order[ctx->device];
    std::lock_guard<std::mutex> order_lock(so.mu);
    if (!so.ev) return fail(ctx, ZG_E_STATE, "static scratch order event missing for this device");
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    ZG_HIP(hipStreamIsCapturing(s, &cs));
    const bool ordered = cs == hipStreamCaptureStatusNone;
    if (ordered && so.used) ZG_HIP(hipStreamWaitEvent(s, so.ev, 0));
    if (fused) {
        zg::FusedGemvArgs f;
        f.M = (int)m_rows;
        f.pro = pro;
        f.epi = zg::EPI_STORE;
        f.x = (const float*)x;
        f.ldx = w->dw.K;
        f.gamma = gamma;
        f.eps = eps;
        f.y = y;
        f.ldy = w->dw.N;
        f.status = ctx->d_flag;
        if (batched) ZG_HIP(zg::batched_gemv(w->dw, f, sp, s));
        else ZG_HIP(zg::fused_gemv(w->dw, f, s));
    } else {
        ZG_HIP(zg::act_prepare_for(w->dw.type, x, x_dtype == ZG_BF16, m_rows, w->dw.K, gamma, eps, sp, s));
        ZG_HIP(zg::gemv(w->dw, m_rows, sp, y, s));
    }
    if (ordered) {
        ZG_HIP(hipEventRecord(so.ev, s));
        so.used = true;
    }
    return ZG_COMPLETED;
}

}  // extern "C"
