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

// The GDN gain alone, lib.rs:339-362: exp(softplus(alpha + dt) * a), the
// same operations as gdn_coef's gain.
__device__ __forceinline__ float gdn_gain(float alpha, float dt, float a) {
    const float biased = alpha + dt;
    const float sp = source_softplus(biased);
    const float gate_raw = sp * a;
    return cr_expf(gate_raw);
}

// GDN gates, lib.rs:339-362: sp = softplus(alpha + dt), gate_raw = sp * a,
// gain = exp(gate_raw), beta = sigmoid(beta projection).
__device__ __forceinline__ void gdn_coef(float alpha, float beta_p, float dt, float a, float& gain, float& beta,
                                         float& sp, float& gate_raw) {
    const float biased = alpha + dt;
    sp = source_softplus(biased);
    gate_raw = sp * a;
    gain = cr_expf(gate_raw);
    beta = source_sigmoid(beta_p);
}

// Eight lanes own one value column j.  The reference dot (source_dot_f32,
// model-qwen35/src/lib.rs:1394-1423) keeps 32 f32 accumulators, accumulator
// a = 8i + l taking elements a, a+32, a+64, a+96 in that order, then reduces
// combined[l] = (s[0][l]+s[2][l]) + (s[1][l]+s[3][l]),
// halves[m] = combined[m] + combined[m+4], (h0+h1)+(h2+h3).
// Lane s of the column holds accumulators 4s..4s+3, i.e. elements
// 32c + 4s + t (c, t in 0..3): one float4 per c, coalesced across the 8
// lanes.  XOR-4 then XOR-2 exchanges form `combined`, XOR-1 forms `halves`
// and the last two levels are local: the dot is bit-identical to the CPU.
// The XOR-4 exchange is a ds_swizzle in bit-mask mode (and 0x1f, xor 4),
// the XOR-2 and XOR-1 ones DPP quad permutes: no lane-index registers.
__device__ __forceinline__ float column_dot(const float (&a)[4][4], const float (&b)[4][4]) {
    float acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        float v = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) v = fmaf(a[c][t], b[c][t], v);
        acc[t] = v;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        acc[t] = acc[t] + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(acc[t]), 0x101f));
        acc[t] = acc[t] + dpp_f<kDppXor2>(acc[t]);
        acc[t] = acc[t] + dpp_f<kDppXor1>(acc[t]);
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

}  // namespace zg
