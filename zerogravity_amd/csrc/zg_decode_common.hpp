#pragma once
// Fused kernels of the resident decode step (gfx950).
//
// A decode step is a chain of dependent launches; at batch 1 each launch is
// latency-bound, so the step is built from as few launches as the data
// dependencies allow:
//   GDN layer:  [RMS + in-proj (qkv|z|alpha|beta)] [conv + L2 + gates +
//               recurrence] [gated RMS + ssm_out + residual]
//   attention:  [RMS + in-proj (q|gate, k, v)] [q/k norm + RoPE + KV append
//               + QK] [softmax + PV + sigmoid gate] [o-proj + residual]
//   FFN:        [RMS + gate|up] [SiLU product + down + residual]
//   head:       [RMS + LM head] [argmax + position advance]
// Each GEMV launch prepares its own activation in its prologue and adds the
// residual in its epilogue.  Every rounding point is the reference's
// (model-qwen35/src/forward.rs:451-755, lib.rs:263-362,1276-1577), in the
// reference's order, so the Q8_0 path is bit-identical to the CPU.
#include <algorithm>

#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

// ======================================================= activation values

__device__ __forceinline__ float rms_inv(double total, int n, float eps) {
    const float mean = (float)(total / (double)n);
    const float root = sqrtf(mean + eps);
    return 1.0f / root;
}

__device__ __forceinline__ void epilogue(const FusedGemvArgs& a, int m, int row, float acc, int epi) {
    float* p = a.y + (size_t)m * a.ldy + row;
    if (epi == EPI_RESID) {
        const float v = *p + acc;  // source_binary Add, lib.rs:1258-1271
        *p = v;
        if (!finite_f32(v)) atomicOr(a.status, 1);
    } else {
        *p = acc;
    }
}

// ================================================ workgroup prologue

constexpr int kCodecQ4K = 0, kCodecQ8 = 1, kCodecQ81 = 2, kCodecQ8K = 3, kCodecF32 = 4;
constexpr int kRecWords = 36;  // Q4_K record: 32 dwords of code bytes + {xs_lo, xs_hi, sum_lo, sum_hi}

// Activation row m prepared once per workgroup.  Thread t holds the float4
// slabs k = 4t + 1024j (all loads issued together), so the 8 threads of a
// 32-element group are adjacent lanes and the group statistics are 3-step
// XOR shuffles.  The values are coded straight into LDS:
//   Q8_0 (cpu/src/source/quantization.rs:37-61): per 32-block amax,
//     d = amax/127, code = clamp(rint(v*127/amax)), d rounded to f16;
//     codes [8][nbp + 4] words (word l of block b at l * (nbp + 4) + b,
//     nbp = K/32 rounded up to 4; the 4 words of padding put the 8 words of
//     a block in different LDS banks), scales [K/32].
//   Q8_1 (quantization.rs:37-61, Q4_1 pairing): as Q8_0 (codes [8][nb8 + 4],
//     nb8 = K/32 rounded up to 8, the rows padded out of one bank), plus per block s = f16(sum of codes *
//     unrounded d) in `extra`.
//   Q8_K (quantization.rs:66-92, Q6_K pairing): per 256-block (one
//     wavefront) the first element of largest magnitude gives the signed
//     max, inv = -127/max, d = 1/inv in `extra` [K/256], codes as Q8_0 laid
//     out lane-major (word w of block sb at (w%8)*(K/32 + 4) + 8sb + w/8), and
//     the sums of 16 codes in `bsums` [K/16].
//   F32: the values themselves, floats [K] at `codes`.
//   Q4_K: per 32-group int16 fixed point, xq = rint(v*32767/amax), with the
//     group's scale amax/32767 and its f32 sum; records [K/64][36] dwords:
//     xq = 256*hi + lo split into bytes, dword e/4 holding the signed high
//     bytes of elements e..e+3 (e % 4 == 0), dword 8 + e/4 their unsigned
//     low bytes, the pair's high group +16, then {scale lo, scale hi,
//     sum lo, sum hi}.
// Ends with a barrier.  K <= 1024 * JMAX, K % 32 == 0 (K % 256 for Q8_K).
//
// The loads are a phase of their own (wg_prologue_load) so that a kernel can
// issue them before its weight loads: a wave's vector loads complete in
// issue order, so activation loads queued behind the weights would hold
// the prologue until the weights have arrived.
template <int JMAX>
struct ProIn {
    v4f v[JMAX], w[JMAX], g[JMAX];
};

template <int PRO, int JMAX>
__device__ __forceinline__ void wg_prologue_load(const FusedGemvArgs& a, int m, bool valid, ProIn<JMAX>& in) {
    const int tid = threadIdx.x, K = a.K;
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
        const int k = 4 * tid + 1024 * j;
        in.v[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        in.w[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        in.g[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (valid && k < K) {
            in.v[j] = *(const v4f*)(a.x + (size_t)m * a.ldx + k);
            if (PRO == PRO_RMS) in.w[j] = *(const v4f*)(a.gamma + k);
            if (PRO == PRO_GATED || PRO == PRO_SILU_MUL) in.w[j] = *(const v4f*)(a.x2 + (size_t)m * a.ldx2 + k);
        }
        if (PRO == PRO_GATED && k < K) in.g[j] = *(const v4f*)(a.gamma + (k & (a.group - 1)));
    }
}

template <int PRO, int CODEC, int JMAX>
__device__ void wg_prologue_code(const FusedGemvArgs& a, bool valid, const ProIn<JMAX>& in, uint32_t* rec, int* codes,
                                 float* scales, float* extra = nullptr, int* bsums = nullptr) {
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, K = a.K;
    const v4f* v = in.v;
    const v4f* w = in.w;
    float inv = 1.0f;
    if (PRO == PRO_RMS) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < JMAX; ++j) {
            const float q0 = v[j].x * v[j].x, q1 = v[j].y * v[j].y, q2 = v[j].z * v[j].z, q3 = v[j].w * v[j].w;
            s += (double)q0;
            s += (double)q1;
            s += (double)q2;
            s += (double)q3;
        }
        s = group_sum_last<64>(s);
        if (lane == 63) red[tid >> 6] = s;
        __syncthreads();
        inv = rms_inv((red[0] + red[1]) + (red[2] + red[3]), K, a.eps);
    }
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
        const int k = 4 * tid + 1024 * j;
        if (1024 * j >= K) break;  // uniform
        float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        const float o[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
        if (PRO == PRO_RMS) {
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = (e[t] * inv) * o[t];
        } else if (PRO == PRO_GATED) {
            // per 128-element group (32 adjacent lanes): f64 sum of f32 squares
            double s = 0.0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float q = e[t] * e[t];
                s += (double)q;
            }
            s = group_sum_last<32>(s);
            s = __shfl(s, (lane & 32) | 31, 64);
            const float gi = rms_inv(s, a.group, a.eps);
            const float gg[4] = {in.g[j].x, in.g[j].y, in.g[j].z, in.g[j].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = ((e[t] * gi) * gg[t]) * ggml_silu(o[t]);
        } else if (PRO == PRO_SILU_MUL) {
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = o[t] * ggml_silu(e[t]);
        }
        if (!(valid && k < K)) e[0] = e[1] = e[2] = e[3] = 0.0f;
        if (CODEC == kCodecF32) {
            if (k < K) *(v4f*)((float*)codes + k) = v4f{e[0], e[1], e[2], e[3]};
            continue;
        }
        if (CODEC == kCodecQ8K) {
            // first element of largest magnitude in the 256-block of this
            // wavefront: (|v| bits, 63 - lane) maximised, ties to the lower lane
            float lam = 0.0f, lsg = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (fabsf(e[t]) > lam) {
                    lam = fabsf(e[t]);
                    lsg = e[t];
                }
            uint32_t key_hi = __float_as_uint(lam), key_lo = 63u - (uint32_t)lane;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const uint32_t oh = __shfl_xor(key_hi, off, 64), ol = __shfl_xor(key_lo, off, 64);
                if (oh > key_hi || (oh == key_hi && ol > key_lo)) {
                    key_hi = oh;
                    key_lo = ol;
                }
            }
            const float amax = __uint_as_float(key_hi);
            const float msg = __shfl(lsg, 63 - (int)key_lo, 64);
            const float qi = amax == 0.0f ? 0.0f : -127.0f / msg;
            const float d = amax == 0.0f ? 0.0f : 1.0f / qi;
            uint32_t word = 0;
            int csum = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float r = rintf(e[t] * qi);
                r = fminf(fmaxf(r, -128.0f), 127.0f);
                word |= ((uint32_t)(int)r & 0xffu) << (8 * t);
                csum += (int)r;
            }
            csum += __shfl_xor(csum, 1, 64);
            csum += __shfl_xor(csum, 2, 64);
            if (k < K) {
                // lane-major: the 8 words a consumer lane reads per 256-block
                // (word w of block sb: lane w % 8, slot w / 8) are adjacent;
                // lane rows K/32 + 4 words apart (out of one bank)
                const int w = (k >> 2) & 63, sb = k >> 8;
                codes[(size_t)(w & 7) * ((K >> 5) + 4) + sb * 8 + (w >> 3)] = (int)word;
                if ((lane & 3) == 0) bsums[k >> 4] = csum;
                if (lane == 0) extra[k >> 8] = d;
            }
            continue;
        }
        float amax = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
        amax = group8_max_all(amax);
        const int l = tid & 7;
        if (CODEC == kCodecQ81) {
            const float d = amax / 127.0f;
            const float qi = amax == 0.0f ? 0.0f : 127.0f / amax;
            uint32_t word = 0;
            float csum = 0.0f;  // integer-valued, |sum| <= 4096: exact in f32
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float r = rintf(e[t] * qi);
                r = fminf(fmaxf(r, -128.0f), 127.0f);
                word |= ((uint32_t)(int)r & 0xffu) << (8 * t);
                csum += r;
            }
            csum = group8_sum_all(csum);
            if (k < K) {
                // lane-major: word l * (nb8 + 4) + block (nb8 = blocks
                // rounded to 8), so that two 16-byte reads serve an 8-block
                // chunk
                const int nb8 = ((K >> 5) + 7) & ~7;
                codes[(size_t)l * (nb8 + 4) + (k >> 5)] = (int)word;
                if (l == 0) {
                    scales[k >> 5] = f16_roundtrip(d);
                    extra[k >> 5] = f16_roundtrip(csum * d);
                }
            }
            continue;
        }
        if (k < K) {
            if (CODEC == kCodecQ8) {
                const float d = amax / 127.0f;
                const float qi = amax == 0.0f ? 0.0f : 127.0f / amax;
                uint32_t word = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float r = rintf(e[t] * qi);
                    r = fminf(fmaxf(r, -128.0f), 127.0f);
                    word |= ((uint32_t)(int)r & 0xffu) << (8 * t);
                }
                // lane-major: word l * (nbp + 4) + block (nbp = blocks
                // rounded to 4), so that one 16-byte read serves four blocks
                const int nbp = ((K >> 5) + 3) & ~3;
                codes[(size_t)l * (nbp + 4) + (k >> 5)] = (int)word;
                if (l == 0) scales[k >> 5] = f16_roundtrip(d);
            }
        }
        if (CODEC == kCodecQ4K) {
            float sum = ((e[0] + e[1]) + e[2]) + e[3];
            sum = group8_sum_all(sum);
            if (k < K) {
                const float qi = amax == 0.0f ? 0.0f : 32767.0f / amax;
                const int q[4] = {(int)rintf(e[0] * qi), (int)rintf(e[1] * qi), (int)rintf(e[2] * qi),
                                  (int)rintf(e[3] * qi)};
                const int g = k >> 5, hi = g & 1;
                uint32_t* r = rec + (size_t)(g >> 1) * kRecWords;
                uint32_t hb = 0, lb = 0;  // q = 256 * (q >> 8) + (q & 255)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    hb |= ((uint32_t)(q[t] >> 8) & 0xffu) << (8 * t);
                    lb |= ((uint32_t)q[t] & 0xffu) << (8 * t);
                }
                r[hi * 16 + l] = hb;
                r[hi * 16 + 8 + l] = lb;
                if (l == 0) {
                    r[32 + hi] = __float_as_uint(amax / 32767.0f);
                    r[34 + hi] = __float_as_uint(sum);
                }
            }
        }
    }
    __syncthreads();
}

template <int PRO, int CODEC, int JMAX>
__device__ __forceinline__ void wg_prologue(const FusedGemvArgs& a, int m, bool valid, uint32_t* rec, int* codes,
                                            float* scales, float* extra = nullptr, int* bsums = nullptr) {
    ProIn<JMAX> in;
    wg_prologue_load<PRO, JMAX>(a, m, valid, in);
    wg_prologue_code<PRO, CODEC, JMAX>(a, valid, in, rec, codes, scales, extra, bsums);
}


}  // namespace zg
