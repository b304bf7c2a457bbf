// Host-side interface between the C ABI (zg_api.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace zg {

enum GgmlType { kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ4_K = 12, kBF16 = 30 };

// A registered weight matrix in its device layout.  The GGUF block stream is
// split once at registration into a streaming payload and a small per-block
// header array so every wavefront load is a coalesced 16-byte load:
//   Q8_0: qs  = int8 [N][K]            hdr = f16 scale [N][K/32]
//   Q4_K: qs  = nibbles [N][K/2]       hdr = 16-byte block header [N][K/256]
//         (d, dmin, 12 packed 6-bit scale/min bytes, unchanged)
//   F32 : qs  = float [N][K]           hdr = null
// Algorithmic bytes are unchanged: 1.0625 B/elem (Q8_0), 0.5625 (Q4_K).
struct DeviceWeight {
    int type = -1;
    size_t K = 0, N = 0;
    void* qs = nullptr;
    void* hdr = nullptr;
    size_t qs_bytes = 0, hdr_bytes = 0;
};

size_t gguf_row_bytes(int type, size_t K);

// Split a GGUF tensor (already on the device) into the layout above.  Any
// nonfinite block scale sets *d_bad to 1 (the reference codecs refuse it).
hipError_t repack_weight(const uint8_t* d_gguf, DeviceWeight& w, int* d_bad, hipStream_t s);

// Exact dequantization of rows [row0, row0+rows) of a registered weight into
// f32 [rows][K].
hipError_t dequantize_rows(const DeviceWeight& w, size_t row0, size_t rows, float* out, hipStream_t s);

// Activation preparation for M rows of width K: optional RMSNorm with gamma
// (f64 sum of f32 squares, f32 mean, 1/sqrtf, (x*inv)*gamma), then either
// f32 output (xf) and/or the dynamic Q8_0 coding (aq codes, ad f16-rounded
// scales).  x is bf16 when x_bf16 != 0, else f32.
hipError_t act_prep(const void* x, int x_bf16, size_t M, size_t K, const float* gamma, float eps,
                    float* xf, int8_t* aq, float* ad, hipStream_t s);

// y[M][N] = W x for a registered weight.  Q8_0 consumes (aq, ad); Q4_K and
// F32 consume xf.  Returns hipErrorInvalidValue for unsupported geometry.
hipError_t gemv(const DeviceWeight& w, size_t M, const float* xf, const int8_t* aq, const float* ad,
                float* y, hipStream_t s);
bool gemv_supported(int type, size_t K, size_t M);

// Pointwise / normalisation kernels (zg_elementwise.hip).
hipError_t rms_groups(const float* x, const float* w, size_t width, size_t groups, float eps, float* out,
                      hipStream_t s);
hipError_t silu(const float* x, const float* m, size_t n, float* out, hipStream_t s);
hipError_t binary(int kind, const float* a, const float* b, size_t n, float* out, hipStream_t s);

}  // namespace zg
