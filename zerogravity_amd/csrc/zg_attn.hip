// GQA decode attention for the full-attention layers (gfx950).
//
// Reference semantics (zerogravity repository):
//   [q | gate] split, q/k grouped RMS   model-qwen35/src/forward.rs:660-695
//   RoPE (rotate 64, pairs (i, i+32),   lib.rs:1552-1577 (angle starts at the
//     iterative f32 angle, FMA form)      position, angle *= theta_scale)
//   KV append                            host_math.rs:1055-1064
//   QK dot * scale                       lib.rs:1427-1441
//   softmax (GGML exp, f64 sum)          lib.rs:1352-1387
//   PV                                   lib.rs:1276-1305
// Every f32 sum is formed in the reference's own order (the 32-accumulator
// FMA tree of its dot and value loops, the 8-wide softmax partials), so the
// outputs equal the CPU path's bit for bit.
//   sigmoid output gate                  forward.rs:751, lib.rs:1258-1271
//
// KV cache: [row][token][kv_head * d] in the element type KV (bf16 for the
// resident decode path, f32 for the host regions), token rows contiguous so
// a decode step streams each row's K and V once.
#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

template <typename KV>
__device__ __forceinline__ float kv_load(const KV* p);
template <>
__device__ __forceinline__ float kv_load<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float kv_load<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
    uint32_t b = __float_as_uint(v);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}
template <typename KV>
__device__ __forceinline__ KV kv_store(float v);
template <>
__device__ __forceinline__ float kv_store<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t kv_store<uint16_t>(float v) { return f32_to_bf16_rne(v); }

// ------------------------------------------------------ norm + RoPE + append

// Grid (B, q_heads + kv_heads), one wave per head, d <= 256 (4 per lane).
// q heads: q = q_proj[h*2d : h*2d+d], normed with q_norm, roped -> qr.
// kv heads: k normed with k_norm and roped -> K cache row at pos[b];
//           v copied -> V cache row at pos[b].
template <typename KV>
__global__ __launch_bounds__(64) void attn_prep_kernel(const float* __restrict__ qproj, size_t q_stride,
                                                       const float* __restrict__ kproj, const float* __restrict__ vproj,
                                                       size_t kv_stride, const float* __restrict__ qn,
                                                       const float* __restrict__ kn, const int* __restrict__ pos,
                                                       int nq, int nkv, int d, int rotate, float theta_scale,
                                                       float eps, int norm, float* __restrict__ qr, size_t qr_stride,
                                                       KV* __restrict__ kcache, KV* __restrict__ vcache,
                                                       size_t cache_row_stride, float* __restrict__ kout,
                                                       float* __restrict__ vout) {
    __shared__ float head[256];
    __shared__ double red;
    const int b = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
    const bool isq = hh < nq;
    const int h = isq ? hh : hh - nq;
    const float* src = isq ? qproj + (size_t)b * q_stride + (size_t)h * 2 * d : kproj + (size_t)b * kv_stride + (size_t)h * d;
    const float* gamma = isq ? qn : kn;
    double s = 0.0;
    for (int i = lane; i < d; i += 64) {
        const float v = src[i];
        head[i] = v;
        const float sq = v * v;
        s += (double)sq;
    }
    if (norm) {
        s = wave_sum_xor<double>(s, 64);
        if (lane == 0) red = s;
        __syncthreads();
        const float mean = (float)(red / (double)d);
        const float inv = 1.0f / sqrtf(mean + eps);
        for (int i = lane; i < d; i += 64) {
            const float t = head[i] * inv;
            head[i] = t * gamma[i];
        }
    }
    __syncthreads();
    const int p = pos[b];
    const int half = rotate / 2;
    if (lane < half) {
        float angle = (float)p;
        for (int t = 0; t < lane; ++t) angle *= theta_scale;
        const float sn = cr_sinf(angle), cs = cr_cosf(angle);
        const float a = head[lane], bb = head[lane + half];
        head[lane] = fmaf(a, cs, -(bb * sn));
        head[lane + half] = fmaf(a, sn, bb * cs);
    }
    __syncthreads();
    if (isq) {
        for (int i = lane; i < d; i += 64) qr[(size_t)b * qr_stride + (size_t)h * d + i] = head[i];
    } else if (kout) {
        const float* vsrc = vproj + (size_t)b * kv_stride + (size_t)h * d;
        for (int i = lane; i < d; i += 64) {
            kout[(size_t)b * kv_stride + (size_t)h * d + i] = head[i];
            vout[(size_t)b * kv_stride + (size_t)h * d + i] = vsrc[i];
        }
    } else {
        KV* krow = kcache + (size_t)b * cache_row_stride + (size_t)p * nkv * d + (size_t)h * d;
        KV* vrow = vcache + (size_t)b * cache_row_stride + (size_t)p * nkv * d + (size_t)h * d;
        const float* vsrc = vproj + (size_t)b * kv_stride + (size_t)h * d;
        for (int i = lane; i < d; i += 64) {
            krow[i] = kv_store<KV>(head[i]);
            vrow[i] = kv_store<KV>(vsrc[i]);
        }
    }
}

// -------------------------------------------------------------------- QK

template <typename KV>
__device__ __forceinline__ void kv_load4(const KV* p, float (&o)[4]);
template <>
__device__ __forceinline__ void kv_load4<float>(const float* p, float (&o)[4]) {
    const v4f v = *(const v4f*)p;
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
template <>
__device__ __forceinline__ void kv_load4<uint16_t>(const uint16_t* p, float (&o)[4]) {
    const uint2 v = *(const uint2*)p;
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
}

// The reference dot (source_dot_f32, lib.rs:1394-1423) gives element i to
// accumulator i % 32 (chained FMA over i, i+32, ...) and reduces the 32
// accumulators with a fixed tree.  Eight lanes share one token: lane s holds
// accumulators 4s..4s+3 (a float4 at 32c + 4s for c = 0..7), XOR 4/2/1
// shuffles form the tree's first three levels, the last two are local.
//
// Grid (ceil(Tmax/32), kv_heads, B), 4 waves x 8 tokens; the G query heads
// of one kv head share each key load.  q is [B][nq][256] (roped).
template <typename KV, int G>
__global__ __launch_bounds__(256) void attn_qk_kernel(const float* __restrict__ q, size_t q_stride,
                                                      const KV* __restrict__ kcache, size_t cache_row_stride,
                                                      const int* __restrict__ ntok, int nkv, float scale,
                                                      float* __restrict__ dots, float* __restrict__ scores,
                                                      size_t score_stride) {
    constexpr int D = 256;
    const int b = blockIdx.z, kvh = blockIdx.y;
    const int s = threadIdx.x & 7;
    const int t = blockIdx.x * 32 + (threadIdx.x >> 3);
    const int T = ntok[b];
    if (blockIdx.x * 32 >= T) return;  // uniform over the workgroup
    float acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[g][e] = 0.0f;
    if (t < T) {
        const float* qb = q + (size_t)b * q_stride + (size_t)kvh * G * D + 4 * s;
        const KV* krow = kcache + (size_t)b * cache_row_stride + ((size_t)t * nkv + kvh) * D + 4 * s;
#pragma unroll
        for (int c = 0; c < D / 32; ++c) {
            float kk[4];
            kv_load4<KV>(krow + 32 * c, kk);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const v4f qq = *(const v4f*)(qb + (size_t)g * D + 32 * c);
                acc[g][0] = fmaf(qq.x, kk[0], acc[g][0]);
                acc[g][1] = fmaf(qq.y, kk[1], acc[g][1]);
                acc[g][2] = fmaf(qq.z, kk[2], acc[g][2]);
                acc[g][3] = fmaf(qq.w, kk[3], acc[g][3]);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v = acc[g][e];
            v = v + __shfl_xor(v, 4, 64);
            v = v + __shfl_xor(v, 2, 64);
            v = v + __shfl_xor(v, 1, 64);
            acc[g][e] = v;
        }
    if (t < T && s == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float dot = (acc[g][0] + acc[g][1]) + (acc[g][2] + acc[g][3]);
            const size_t at = (size_t)b * score_stride + (size_t)(kvh * G + g) * T + t;
            if (dots) dots[at] = dot;
            scores[at] = dot * scale;
        }
    }
}

// --------------------------------------------------------------- softmax

// One workgroup per (head, row), lib.rs:1352-1387: max, e = ggml_exp(x -
// max) in blocks of 8 (zero past the end), block partial
// ((e0+e4)+(e2+e6))+((e1+e5)+(e3+e7)) in f32, partials summed in f64,
// inv = (float)(1/sum), p = e * inv.  Thread i owns blocks i, i+256, ...
__global__ __launch_bounds__(256) void attn_softmax_kernel(const float* __restrict__ scores, size_t score_stride,
                                                           const int* __restrict__ ntok, float* __restrict__ exps,
                                                           float* __restrict__ probs, double* __restrict__ sums) {
    __shared__ float smax[4];
    __shared__ double ssum[4];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int T = ntok[b];
    const float* row = scores + (size_t)b * score_stride + (size_t)h * T;
    float m = -INFINITY;
    for (int i = tid; i < T; i += 256) m = fmaxf(m, row[i]);
    m = wave_max(m);
    if ((tid & 63) == 0) smax[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    double s = 0.0;
    float* prow = probs + (size_t)b * score_stride + (size_t)h * T;
    float* erow = exps ? exps + (size_t)b * score_stride + (size_t)h * T : nullptr;
    for (int blk = tid; blk * 8 < T; blk += 256) {
        float e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int at = blk * 8 + i;
            e[i] = at < T ? ggml_exp(row[at] - m) : 0.0f;
        }
        const float partial = ((e[0] + e[4]) + (e[2] + e[6])) + ((e[1] + e[5]) + (e[3] + e[7]));
        s += (double)partial;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int at = blk * 8 + i;
            if (at < T) {
                prow[at] = e[i];
                if (erow) erow[at] = e[i];
            }
        }
    }
    s = wave_sum_xor<double>(s, 64);
    if ((tid & 63) == 0) ssum[tid >> 6] = s;
    __syncthreads();
    const double total = (ssum[0] + ssum[1]) + (ssum[2] + ssum[3]);
    const float inv = (float)(1.0 / total);
    if (sums && tid == 0) sums[(size_t)b * gridDim.x + h] = total;
    for (int blk = tid; blk * 8 < T; blk += 256) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int at = blk * 8 + i;
            if (at < T) prow[at] = prow[at] * inv;
        }
    }
}

// -------------------------------------------------------------------- PV

// lib.rs:1276-1305: out[h][j] = tree over 32 accumulators, accumulator a
// chaining fmaf(v[t][j], p[h][t], acc) over tokens t = a, a+32, ... (the
// reference's zero padding adds +0*+0 terms, which change nothing).
//
// Grid (256/8, kv_heads, B), 4 waves: wave w holds accumulators 8w..8w+7 of
// 8 value channels (lane = channel*8 + a%8) for the G query heads of one kv
// head, so each value load feeds G chains.  The tree runs from LDS, then
// the sigmoid output gate (forward.rs:751) is applied when given.
template <typename KV, int G>
__global__ __launch_bounds__(256) void attn_pv_kernel(const float* __restrict__ probs, size_t score_stride,
                                                      const KV* __restrict__ vcache, size_t cache_row_stride,
                                                      const int* __restrict__ ntok, int nkv,
                                                      const float* __restrict__ gate, size_t gate_stride,
                                                      float* __restrict__ out, size_t out_stride) {
    constexpr int D = 256;
    __shared__ float red[G][8][33];
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ch = lane >> 3, a = w * 8 + (lane & 7);
    const int j = blockIdx.x * 8 + ch;
    const int T = ntok[b];
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
    const float* pb = probs + (size_t)b * score_stride + (size_t)kvh * G * T;
    const KV* vb = vcache + (size_t)b * cache_row_stride + (size_t)kvh * D + j;
    const size_t vstep = (size_t)nkv * D;
    for (int t = a; t < T; t += 32) {
        const float v = kv_load<KV>(vb + (size_t)t * vstep);
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g] = fmaf(v, pb[(size_t)g * T + t], acc[g]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) red[g][ch][a] = acc[g];
    __syncthreads();
    if (threadIdx.x < G * 8) {
        const int g = threadIdx.x >> 3, c = threadIdx.x & 7;
        const float* r = red[g][c];
        float comb[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) comb[l] = (r[l] + r[16 + l]) + (r[8 + l] + r[24 + l]);
        const float h0 = comb[0] + comb[4], h1 = comb[1] + comb[5], h2 = comb[2] + comb[6], h3 = comb[3] + comb[7];
        float v = (h0 + h1) + (h2 + h3);
        const int jj = blockIdx.x * 8 + c;
        const int h = kvh * G + g;
        if (gate) v = v * source_sigmoid(gate[(size_t)b * gate_stride + (size_t)h * 2 * D + D + jj]);
        out[(size_t)b * out_stride + (size_t)h * D + jj] = v;
    }
}

// ------------------------------------------------------------------ host

template <typename KV>
static hipError_t launch_prep(const AttnArgs& a, hipStream_t s) {
    if (a.d > 256 || a.rotate > 128 || a.rotate > a.d) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_prep_kernel<KV>, dim3(a.B, a.nq + a.nkv), dim3(64), 0, s, a.qproj, a.q_stride, a.kproj,
                       a.vproj, a.kv_stride, a.qnorm, a.knorm, a.pos, a.nq, a.nkv, a.d, a.rotate, a.theta_scale, a.eps,
                       a.norm, a.qr, a.qr_stride, (KV*)a.kcache, (KV*)a.vcache, a.cache_row_stride, a.kout, a.vout);
    return hipGetLastError();
}

template <typename KV, int G>
static void launch_group(const AttnArgs& a, bool qk, bool softmax, bool pv, hipStream_t s) {
    constexpr int D = 256;
    if (qk)
        hipLaunchKernelGGL((attn_qk_kernel<KV, G>), dim3((a.tmax + 31) / 32, a.nkv, a.B), dim3(256), 0, s, a.qr,
                           a.qr_stride, (const KV*)a.kcache, a.cache_row_stride, a.ntok, a.nkv, a.scale, a.dots,
                           a.scores, a.score_stride);
    if (softmax)
        hipLaunchKernelGGL(attn_softmax_kernel, dim3(a.nq, a.B), dim3(256), 0, s, a.scores, a.score_stride, a.ntok,
                           a.exps, a.probs, a.sums);
    if (pv)
        hipLaunchKernelGGL((attn_pv_kernel<KV, G>), dim3(D / 8, a.nkv, a.B), dim3(256), 0, s, a.probs,
                           a.score_stride, (const KV*)a.vcache, a.cache_row_stride, a.ntok, a.nkv, a.gate,
                           a.gate_stride, a.out, a.out_stride);
}

template <typename KV>
static hipError_t launch_parts(const AttnArgs& a, bool qk, bool softmax, bool pv, hipStream_t s) {
    if (a.d != 256 || a.nkv <= 0 || a.nq % a.nkv || a.tmax <= 0) return hipErrorInvalidValue;
    switch (a.nq / a.nkv) {
        case 1: launch_group<KV, 1>(a, qk, softmax, pv, s); break;
        case 2: launch_group<KV, 2>(a, qk, softmax, pv, s); break;
        case 3: launch_group<KV, 3>(a, qk, softmax, pv, s); break;
        case 4: launch_group<KV, 4>(a, qk, softmax, pv, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t rope_prep(const AttnArgs& a, hipStream_t s) {
    return a.kv_bf16 ? launch_prep<uint16_t>(a, s) : launch_prep<float>(a, s);
}

hipError_t attention_parts(const AttnArgs& a, bool qk, bool softmax, bool pv, hipStream_t s) {
    return a.kv_bf16 ? launch_parts<uint16_t>(a, qk, softmax, pv, s) : launch_parts<float>(a, qk, softmax, pv, s);
}

hipError_t attention(const AttnArgs& a, hipStream_t s) {
    if (a.do_prep) {
        hipError_t e = rope_prep(a, s);
        if (e != hipSuccess || a.prep_only) return e;
    }
    return attention_parts(a, true, true, true, s);
}

hipError_t softmax_rows(const float* scores, size_t score_stride, const int* ntok, float* probs, size_t heads, size_t B,
                        hipStream_t s) {
    hipLaunchKernelGGL(attn_softmax_kernel, dim3((unsigned)heads, (unsigned)B), dim3(256), 0, s, scores, score_stride,
                       ntok, nullptr, probs, nullptr);
    return hipGetLastError();
}

}  // namespace zg
