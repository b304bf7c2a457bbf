// Context and resident-weight types shared by the C ABI translation units.
#pragma once
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>

#include "zg_hip.h"
#include "zg_internal.hpp"

struct zg_weight {
    zg::DeviceWeight dw;
    uint64_t source = 0;
    std::string name;
    // Lifetime: loaded models hold references (model_refs); a handle given
    // out by zg_weight_register / a bound zg_matvec pins the weight until
    // zg_source_release.  It is freed when neither holds it.
    int model_refs = 0;
    bool api_pinned = false;
};

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
};

struct zg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    // unique per context for the life of the process: failure texts are kept
    // per (thread, serial), so a context created later at a reused address
    // never reads an earlier one's message
    uint64_t serial = 0;
    std::map<std::tuple<uint64_t, std::string, int, size_t, size_t>, std::unique_ptr<zg_weight>> weights;
    DeviceBuffer scratch;    // region calls: inputs/outputs staged here
    DeviceBuffer actbuf;     // zg_gemv_device: prepared activations
    DeviceBuffer chunkbuf;   // zg_gdn_chunk_prefill_device: per-(chunk, head) records
    int* d_flag = nullptr;
    // device address of this device's copy of the static scratch array used
    // by zg_gemv_device_noalloc (set up at context creation)
    void* static_scratch = nullptr;
};

namespace zgc {

int fail(zg_ctx* ctx, int code, const std::string& msg);
// The calling thread's last failure text on ctx ("" if none).
std::string last_message(const zg_ctx* ctx);
int ensure(zg_ctx* ctx, DeviceBuffer& b, size_t bytes);
size_t align256(size_t n);
void free_weight(zg_weight* w);
int check_matrix(zg_ctx* ctx, int type, size_t cols, size_t rows, const void* bytes, size_t len);
int lookup_or_register(zg_ctx* ctx, uint64_t source, const char* name, int type, size_t cols, size_t rows,
                       const void* bytes, size_t len, zg_weight** out);
// Free a weight and remove it from the ctx cache (caller holds the lock).
void drop_weight(zg_ctx* ctx, zg_weight* w);
int build_weight(zg_ctx* ctx, int type, size_t cols, size_t rows, const void* bytes, size_t len,
                 std::unique_ptr<zg_weight>& out);
bool all_finite(const float* x, size_t n);
// ggml codecs with device kernels here, and their block length in elements
bool supported_type(int t);
size_t block_elems(int t);

}  // namespace zgc

#define ZG_HIP(expr)                                                                                     \
    do {                                                                                                 \
        hipError_t e_ = (expr);                                                                          \
        if (e_ != hipSuccess)                                                                            \
            return zgc::fail(ctx, ZG_E_DEVICE, std::string(#expr) + " failed: " + hipGetErrorString(e_)); \
    } while (0)
