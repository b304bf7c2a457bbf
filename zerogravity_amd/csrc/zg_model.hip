// Resident Qwen3.5 hybrid model and decode sessions (boundary B).
//
// Schedule: forward::forward_token (model-qwen35/src/forward.rs:451-516)
// with gdn_layer (:518-632) and attention_layer (:634-755), run for B
// independent rows at once (continuous batch).  Each row keeps its own
// position; weights stream from HBM once per step for all rows.
//
// Per layer (B rows):
//   GDN:  prep(rms attn_norm) -> GEMV qkv, z, alpha, beta -> conv+SiLU ->
//         recurrence (L2 + coefficients fused) -> grouped RMS(ssm_norm) * silu(z)
//         -> prep -> GEMV ssm_out -> residual add
//   ATTN: prep(rms attn_norm) -> GEMV q|gate, k, v -> norm+RoPE+KV append ->
//         QK -> softmax -> PV -> sigmoid gate -> prep -> GEMV attn_output -> add
//   FFN:  prep(rms post_attention_norm) -> GEMV gate, up -> up*silu(gate) ->
//         prep -> GEMV down -> residual add
// Final: prep(rms output_norm) -> GEMV token_embd (tied LM head) -> argmax.
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "zg_device.hpp"
#include "zg_hip.h"
#include "zg_internal.hpp"

namespace zg {

// --------------------------------------------------------------- kernels

// Dequantize embedding rows: x[b] = token_embd[tokens[b]] (codecs/mod.rs:36-88).
__global__ void embed_q8_0_kernel(const int8_t* __restrict__ qs, const uint16_t* __restrict__ hdr,
                                  const uint32_t* __restrict__ tokens, float* __restrict__ x, int K, int V,
                                  int* __restrict__ status) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= K) return;
    const uint32_t t = tokens[b];
    if (t >= (uint32_t)V) {
        if (i == 0) atomicOr(status, 2);
        x[(size_t)b * K + i] = 0.0f;
        return;
    }
    const size_t nbc = ((size_t)K / 32 + 3) / 4;
    const float scale = f16_to_f32(hdr[(size_t)t * nbc * 4 + i / 32]);
    x[(size_t)b * K + i] = (float)qs[q8_tile_offset(t, i / 32, (i % 32) >> 2, nbc) + (i & 3)] * scale;
}

__global__ void embed_q4k_kernel(const uint8_t* __restrict__ qs, const v4u* __restrict__ hdr,
                                 const uint32_t* __restrict__ tokens, float* __restrict__ x, int K, int V,
                                 int* __restrict__ status) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= K) return;
    const uint32_t t = tokens[b];
    if (t >= (uint32_t)V) {
        if (i == 0) atomicOr(status, 2);
        x[(size_t)b * K + i] = 0.0f;
        return;
    }
    const v4u h = hdr[q4k_hdr_index(t, i / 256, K / 256)];
    const int e = i % 256, g = e / 32, pos = e % 32;
    const int sh = 8 * (g >> 1);
    const uint32_t b1 = (h.y >> sh) & 0xffu, b2 = (h.z >> sh) & 0xffu, b3 = (h.w >> sh) & 0xffu;
    uint32_t sc, mn;
    if ((g & 1) == 0) {
        sc = b1 & 63;
        mn = b2 & 63;
    } else {
        sc = b3 & 63;
        mn = (b1 >> 6) | ((b2 >> 6) << 2) | ((b3 >> 6) << 4);
    }
    const float d = f16_to_f32((uint16_t)(h.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
    const float scale = d * (float)sc, mnf = dmin * (float)mn;
    const uint8_t byte = qs[q4k_chunk_offset(t, i / 64, K) + (pos < 16 ? pos : 256 + pos - 16)];
    const uint32_t v = (g & 1) ? (byte >> 4) : (byte & 15);
    x[(size_t)b * K + i] = scale * (float)v - mnf;
}

__global__ void embed_f32_kernel(const float* __restrict__ w, const uint32_t* __restrict__ tokens,
                                 float* __restrict__ x, int K, int V, int* __restrict__ status) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= K) return;
    const uint32_t t = tokens[b];
    if (t >= (uint32_t)V) {
        if (i == 0) atomicOr(status, 2);
        x[(size_t)b * K + i] = 0.0f;
        return;
    }
    x[(size_t)b * K + i] = w[(size_t)t * K + i];
}


// Seeded counter-based normal samples (splitmix64 + Box-Muller) for the
// synthetic decode prefix.
__device__ __forceinline__ uint64_t splitmix(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    const uint64_t r = splitmix(seed ^ splitmix(i));
    const float u1 = ((float)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = ((float)((r >> 16) & 0xffffff) + 0.5f) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
}
__global__ void fill_normal_f32(float* __restrict__ p, size_t n, uint64_t seed, float sigma) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = sigma * normal_at(seed, i);
}
__global__ void fill_normal_bf16(uint16_t* __restrict__ p, size_t n, uint64_t seed, float sigma) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = __float_as_uint(sigma * normal_at(seed, i));
        b += 0x7fffu + ((b >> 16) & 1u);
        p[i] = (uint16_t)(b >> 16);
    }
}
__global__ void bf16_to_f32_kernel(const uint16_t* __restrict__ in, float* __restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = bf16_to_f32(in[i]);
}
__global__ void f32_to_bf16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t b = __float_as_uint(in[i]);
    b += 0x7fffu + ((b >> 16) & 1u);
    out[i] = (uint16_t)(b >> 16);
}
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, size_t n, uint32_t v) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

static unsigned blocks_for(size_t n, unsigned t = 256) { return (unsigned)((n + t - 1) / t); }

// Q4_1 / Q6_K token rows decoded from the device layouts (exact, as the
// reference's block decoders).
__global__ void embed_codec_kernel(int type, const void* __restrict__ qs, const void* __restrict__ hdr,
                                   const uint32_t* __restrict__ tokens, float* __restrict__ x, int K, int V,
                                   int* __restrict__ status) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= K) return;
    const uint32_t t = tokens[b];
    if (t >= (uint32_t)V) {
        if (i == 0) atomicOr(status, 2);
        x[(size_t)b * K + i] = 0.0f;
        return;
    }
    float v;
    if (type == kQ4_1) {
        v = q41_element((const uint16_t*)qs, (const uint32_t*)hdr, t, (size_t)i, (size_t)K);
    } else {
        const uint8_t* sc = (const uint8_t*)hdr;
        const float* d = (const float*)(sc + (size_t)V * (K / 256) * 16);
        v = q6k_element((const uint32_t*)qs, sc, d, t, (size_t)i, (size_t)V, (size_t)K);
    }
    x[(size_t)b * K + i] = v;
}

hipError_t embed(const DeviceWeight& w, const uint32_t* tokens, float* x, size_t B, int* status, hipStream_t s) {
    dim3 g(blocks_for(w.K), (unsigned)B);
    if (w.type == kQ8_0)
        hipLaunchKernelGGL(embed_q8_0_kernel, g, dim3(256), 0, s, (const int8_t*)w.qs, (const uint16_t*)w.hdr, tokens,
                           x, (int)w.K, (int)w.N, status);
    else if (w.type == kQ4_K)
        hipLaunchKernelGGL(embed_q4k_kernel, g, dim3(256), 0, s, (const uint8_t*)w.qs, (const v4u*)w.hdr, tokens, x,
                           (int)w.K, (int)w.N, status);
    else if (w.type == kQ4_1 || w.type == kQ6_K)
        hipLaunchKernelGGL(embed_codec_kernel, g, dim3(256), 0, s, w.type, w.qs, w.hdr, tokens, x, (int)w.K, (int)w.N,
                           status);
    else
        hipLaunchKernelGGL(embed_f32_kernel, g, dim3(256), 0, s, (const float*)w.qs, tokens, x, (int)w.K, (int)w.N,
                           status);
    return hipGetLastError();
}

hipError_t fill_normal(void* p, size_t n, bool bf16, uint64_t seed, float sigma, hipStream_t s) {
    const unsigned g = (unsigned)std::min<size_t>(blocks_for(n), 4096);
    if (bf16)
        hipLaunchKernelGGL(fill_normal_bf16, dim3(g), dim3(256), 0, s, (uint16_t*)p, n, seed, sigma);
    else
        hipLaunchKernelGGL(fill_normal_f32, dim3(g), dim3(256), 0, s, (float*)p, n, seed, sigma);
    return hipGetLastError();
}

hipError_t convert_kv(const void* in, void* out, size_t n, bool to_f32, hipStream_t s) {
    if (to_f32)
        hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(blocks_for(n)), dim3(256), 0, s, (const uint16_t*)in, (float*)out, n);
    else
        hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(blocks_for(n)), dim3(256), 0, s, (const float*)in, (uint16_t*)out, n);
    return hipGetLastError();
}

hipError_t fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks_for(n)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace zg
