// Scalar device restatements of the reference's pointwise functions, shared
// by every kernel that fuses them.
#pragma once
#include "zg_device.hpp"

namespace zg {

// GGML Haswell vector exp (cpu/src/ops.rs:317-350): FMA range reduction,
// degree-5 polynomial, exponent built from the rounded multiple.  Every
// fmaf below is a v_fma_f32 (single rounding), matching the Rust mul_add.
__device__ __forceinline__ float ggml_exp(float x) {
    if (!finite_f32(x)) return __expf(x);
    const float r = __uint_as_float(0x4b400000u);
    const float z = fmaf(x, __uint_as_float(0x3fb8aa3bu), r);
    const float n = z - r;
    const float b = fmaf(-n, __uint_as_float(0x35bfbe8eu), fmaf(-n, __uint_as_float(0x3f317200u), x));
    const uint32_t e = __float_as_uint(z) << 23;
    const float k = __uint_as_float(e + 0x3f800000u);
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(__uint_as_float(0x3c072010u), b, __uint_as_float(0x3d2b9f17u)), u,
                              fmaf(__uint_as_float(0x3e2aaf33u), b, __uint_as_float(0x3efffedbu))),
                         u, __uint_as_float(0x3f7ffff6u) * b);
    if (fabsf(n) <= 126.0f) return fmaf(j, k, k);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = __uint_as_float(g + 0x7f000000u);
    const float s2 = __uint_as_float(e - g);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

// cpu/src/ops.rs:353-355
__device__ __forceinline__ float ggml_silu(float x) { return x / (1.0f + ggml_exp(0.0f - x)); }

// f32 transcendentals, correctly rounded: evaluated in double and rounded
// once.  The reference calls the platform libm (Rust f32::exp/ln/sin_cos) and
// no reference test pins their last bit; both this device code and the CPU
// oracle use the correctly rounded value, so they agree bit for bit.
__device__ __forceinline__ float cr_expf(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float cr_logf(float x) { return (float)log((double)x); }
__device__ __forceinline__ float cr_sinf(float x) { return (float)sin((double)x); }
__device__ __forceinline__ float cr_cosf(float x) { return (float)cos((double)x); }

// model-qwen35/src/lib.rs:324-326
__device__ __forceinline__ float source_sigmoid(float x) { return 1.0f / (1.0f + cr_expf(-x)); }

// lib.rs:328-336
__device__ __forceinline__ float source_softplus(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return cr_expf(x);
    return cr_logf(1.0f + cr_expf(x));
}

}  // namespace zg
