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
        const float sn = sinf(angle), cs = cosf(angle);
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

// Grid (ceil(Tmax/16), B); 4 waves x 4 tokens, 16 lanes per token, 16 dims
// per lane (d = 256).  Lane keeps its 16 dims of every query head in
// registers; the 16-lane dot partials reduce with a 4-step XOR tree.
template <typename KV>
__global__ __launch_bounds__(256) void attn_qk_kernel(const float* __restrict__ q, size_t q_stride,
                                                      const KV* __restrict__ kcache, size_t cache_row_stride,
                                                      const int* __restrict__ ntok, int nq, int nkv, float scale,
                                                      float* __restrict__ dots, float* __restrict__ scores,
                                                      size_t score_stride) {
    constexpr int D = 256, NQ = 8;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, sub = lane & 15;
    const int t = blockIdx.x * 16 + (threadIdx.x >> 6) * 4 + g;
    const int T = ntok[b];
    float qv[NQ][16];
#pragma unroll
    for (int h = 0; h < NQ; ++h)
#pragma unroll
        for (int e = 0; e < 16; ++e) qv[h][e] = h < nq ? q[(size_t)b * q_stride + (size_t)h * D + sub * 16 + e] : 0.0f;
    const int group = nq / nkv;
    float acc[NQ];
#pragma unroll
    for (int h = 0; h < NQ; ++h) acc[h] = 0.0f;
    if (t < T) {
        const KV* krow = kcache + (size_t)b * cache_row_stride + (size_t)t * nkv * D;
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
            if (h < nq) {
                const KV* kk = krow + (size_t)(h / group) * D + sub * 16;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[h] = fmaf(qv[h][e], kv_load<KV>(kk + e), acc[h]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < NQ; ++h) acc[h] = wave_sum_xor(acc[h], 16);
    if (t < T && sub == 0) {
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
            if (h < nq) {
                if (dots) dots[(size_t)b * score_stride + (size_t)h * T + t] = acc[h];
                scores[(size_t)b * score_stride + (size_t)h * T + t] = acc[h] * scale;
            }
        }
    }
}

// --------------------------------------------------------------- softmax

// One workgroup per (head, row): max, e = ggml_exp(x - max), f64 sum,
// inv = (float)(1/sum), p = e * inv.
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
    for (int i = tid; i < T; i += 256) {
        const float e = ggml_exp(row[i] - m);
        prow[i] = e;
        if (exps) exps[(size_t)b * score_stride + (size_t)h * T + i] = e;
        s += (double)e;
    }
    s = wave_sum_xor<double>(s, 64);
    if ((tid & 63) == 0) ssum[tid >> 6] = s;
    __syncthreads();
    const double total = (ssum[0] + ssum[1]) + (ssum[2] + ssum[3]);
    const float inv = (float)(1.0 / total);
    if (sums && tid == 0) sums[(size_t)b * gridDim.x + h] = total;
    for (int i = tid; i < T; i += 256) prow[i] = prow[i] * inv;
}

// -------------------------------------------------------------------- PV

// Grid (splits, kv_heads, B).  Each workgroup covers a contiguous token
// range for the `group` query heads of one kv head; lanes own 4 of the 256
// value dims, waves interleave tokens.  Partial sums go to
// part[b][split][h][d]; attn_combine adds the splits in order.
template <typename KV>
__global__ __launch_bounds__(256) void attn_pv_kernel(const float* __restrict__ probs, size_t score_stride,
                                                      const KV* __restrict__ vcache, size_t cache_row_stride,
                                                      const int* __restrict__ ntok, int nq, int nkv, int splits,
                                                      float* __restrict__ part) {
    constexpr int D = 256, G = 4;
    __shared__ float red[4][G][D];
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int T = ntok[b];
    const int per = (T + splits - 1) / splits;
    const int t0 = split * per, t1 = min(T, t0 + per);
    const int group = nq / nkv;
    float acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[g][e] = 0.0f;
    const float* pb = probs + (size_t)b * score_stride;
    for (int t = t0 + wave; t < t1; t += 4) {
        const KV* v = vcache + (size_t)b * cache_row_stride + (size_t)t * nkv * D + (size_t)kvh * D + lane * 4;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vv[e] = kv_load<KV>(v + e);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (g < group) {
                const float p = pb[(size_t)(kvh * group + g) * T + t];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[g][e] = fmaf(vv[e], p, acc[g][e]);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[wave][g][lane * 4 + e] = acc[g][e];
    __syncthreads();
    for (int i = threadIdx.x; i < group * D; i += 256) {
        const int g = i / D, dd = i % D;
        const float sum = (red[0][g][dd] + red[1][g][dd]) + (red[2][g][dd] + red[3][g][dd]);
        part[(((size_t)b * splits + split) * nq + kvh * group + g) * D + dd] = sum;
    }
}

// out[b][h][d] = sum over splits (in order), times sigmoid(gate) when gate.
__global__ void attn_combine_kernel(const float* __restrict__ part, int splits, int nq,
                                    const float* __restrict__ gate, size_t gate_stride, float* __restrict__ out,
                                    size_t out_stride, int B) {
    constexpr int D = 256;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)B * nq * D) return;
    const size_t b = i / (nq * D), hd = i % (nq * D);
    float s = 0.0f;
    for (int k = 0; k < splits; ++k) s += part[((size_t)b * splits + k) * nq * D + hd];
    if (gate) {
        const size_t h = hd / D, dd = hd % D;
        s = s * source_sigmoid(gate[b * gate_stride + h * 2 * D + D + dd]);
    }
    out[b * out_stride + hd] = s;
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

template <typename KV>
static hipError_t launch_parts(const AttnArgs& a, bool qk, bool softmax, bool pv, hipStream_t s) {
    const int D = a.d;
    if (D != 256 || a.nq > 8 || a.nq % a.nkv || a.nq / a.nkv > 4) return hipErrorInvalidValue;
    if (qk)
        hipLaunchKernelGGL(attn_qk_kernel<KV>, dim3((a.tmax + 15) / 16, a.B), dim3(256), 0, s, a.qr, a.qr_stride,
                           (const KV*)a.kcache, a.cache_row_stride, a.ntok, a.nq, a.nkv, a.scale, a.dots, a.scores,
                           a.score_stride);
    if (softmax)
        hipLaunchKernelGGL(attn_softmax_kernel, dim3(a.nq, a.B), dim3(256), 0, s, a.scores, a.score_stride, a.ntok,
                           a.exps, a.probs, a.sums);
    if (pv) {
        hipLaunchKernelGGL(attn_pv_kernel<KV>, dim3(a.splits, a.nkv, a.B), dim3(256), 0, s, a.probs, a.score_stride,
                           (const KV*)a.vcache, a.cache_row_stride, a.ntok, a.nq, a.nkv, a.splits, a.part);
        const size_t n = (size_t)a.B * a.nq * D;
        hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.part, a.splits,
                           a.nq, a.gate, a.gate_stride, a.out, a.out_stride, a.B);
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
