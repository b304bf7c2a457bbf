// GGUF block-quantized GEMV / skinny GEMM for gfx950, plus the weight repack,
// exact dequantization and activation-preparation kernels it depends on.
//
// Reference semantics (zerogravity repository):
//   Q8_0 x dynamic-Q8_0 activation: cpu/src/source/quantization.rs:37-61,171-196
//   Q4_K x f32 activation (dot_row): cpu/src/source.rs:431-459
//   codecs: artifacts/src/codecs/q8.rs:6-15, q4.rs:39-70
//   RMSNorm prologue: model-qwen35/src/lib.rs:263-284
//
// Design: memory-bound.  Each wavefront owns `64/lpr` weight rows at a time,
// `lpr` lanes per row, every lane streaming 16-byte nontemporal loads of the
// row payload.  A lane always covers the same K positions, so its share of
// the activation lives in registers for the whole launch and is reused by
// every row it visits; the only per-row reduction is a log2(lpr)-step XOR
// shuffle tree.
#include <algorithm>

#include "zg_device.hpp"
#include "zg_internal.hpp"

namespace zg {

size_t gguf_row_bytes(int type, size_t K) {
    switch (type) {
    case kQ8_0: return K / 32 * 34;
    case kQ4_K: return K / 256 * 144;
    case kF32: return K * 4;
    case kQ4_1: return K / 32 * 20;
    case kQ6_K: return K / 256 * 210;
    default: return 0;
    }
}

// ------------------------------------------------------------------ repack

__global__ void repack_q8_0_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ qs,
                                   uint16_t* __restrict__ hdr, size_t N, size_t nb, int* bad) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * nb) return;
    const size_t row = i / nb, b = i % nb;
    const uint8_t* blk = src + i * 34;
    uint16_t d = (uint16_t)(blk[0] | (blk[1] << 8));
    if ((d & 0x7c00u) == 0x7c00u) atomicOr(bad, 1);
    const size_t nbc = (nb + 3) / 4;
    hdr[row * nbc * 4 + b] = d;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        uint32_t word = (uint32_t)blk[2 + 4 * l] | ((uint32_t)blk[3 + 4 * l] << 8) | ((uint32_t)blk[4 + 4 * l] << 16) |
                        ((uint32_t)blk[5 + 4 * l] << 24);
        *(uint32_t*)(qs + q8_tile_offset(row, b, l, nbc)) = word;
    }
}

// GGUF Q4_K 6-bit scale/min unpack (artifacts/src/codecs/q4.rs:58-65).
__device__ __forceinline__ void q4k_scale_min(const uint8_t* s, int g, uint32_t& sc, uint32_t& mn) {
    if (g < 4) {
        sc = s[g] & 63;
        mn = s[g + 4] & 63;
    } else {
        sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4);
        mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
}

// One GGUF block (row b / nbk, block b % nbk) into the 16-row tile layout
// (q4k_chunk_offset, q4k_hdr_index) with the header's scale bytes repacked.
__global__ void repack_q4k_kernel(const v4i* __restrict__ src, uint8_t* __restrict__ qs, v4u* __restrict__ hdr,
                                  size_t nblocks, size_t nbk, size_t K, int* bad) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const size_t row = b / nbk, kb = b % nbk;
    const v4i* blk = src + b * 9;  // 144 bytes = 9 x 16
    v4i h = blk[0];
    uint32_t w0 = (uint32_t)h.x;
    if ((w0 & 0x7c00u) == 0x7c00u || ((w0 >> 16) & 0x7c00u) == 0x7c00u) atomicOr(bad, 1);
    uint8_t s[12];
    const uint32_t hw[3] = {(uint32_t)h.y, (uint32_t)h.z, (uint32_t)h.w};
#pragma unroll
    for (int i = 0; i < 12; ++i) s[i] = (uint8_t)(hw[i >> 2] >> (8 * (i & 3)));
    uint32_t d1 = 0, d2 = 0, d3 = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(s, 2 * p, sc0, mn0);
        q4k_scale_min(s, 2 * p + 1, sc1, mn1);
        d1 |= (sc0 | ((mn1 & 3u) << 6)) << (8 * p);
        d2 |= (mn0 | (((mn1 >> 2) & 3u) << 6)) << (8 * p);
        d3 |= (sc1 | (((mn1 >> 4) & 3u) << 6)) << (8 * p);
    }
    hdr[q4k_hdr_index(row, kb, nbk)] = v4u{w0, d1, d2, d3};
#pragma unroll
    for (int i = 0; i < 8; ++i)  // 16-byte half i % 2 of chunk 4 kb + i / 2
        *(v4i*)(qs + q4k_chunk_offset(row, 4 * kb + (i >> 1), K) + 256 * (i & 1)) = blk[1 + i];
}

// GGUF Q4_1 block (codecs/q4.rs:22-36): d f16, m f16, 16 nibble bytes.
__global__ void repack_q41_kernel(const uint8_t* __restrict__ src, uint16_t* __restrict__ qs,
                                  uint32_t* __restrict__ hdr, size_t N, size_t nb, int* bad) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * nb) return;
    const size_t row = i / nb, b = i % nb, nbc8 = (nb + 7) / 8;
    const uint8_t* blk = src + i * 20;
    const uint32_t d = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
    const uint32_t m = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8);
    if ((d & 0x7c00u) == 0x7c00u || (m & 0x7c00u) == 0x7c00u) atomicOr(bad, 1);
    hdr[row * nbc8 * 8 + b] = d | (m << 16);
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * l + j;
            const uint32_t nib = e < 16 ? (blk[4 + e] & 15u) : (uint32_t)(blk[4 + e - 16] >> 4);
            word |= nib << (4 * j);
        }
        qs[q41_word_index(row, b, l, nbc8)] = (uint16_t)word;
    }
}

// GGUF Q6_K superblock (codecs/q6.rs): ql[128], qh[64], int8 scales[16], d f16.
__global__ void repack_q6k_kernel(const uint8_t* __restrict__ src, uint32_t* __restrict__ qs,
                                  uint8_t* __restrict__ scales, float* __restrict__ dplane, size_t N, size_t K,
                                  int* bad) {
    const size_t nsb = K / 256;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * nsb) return;
    const size_t row = i / nsb, sb = i % nsb;
    const uint8_t* blk = src + i * 210;
    const uint16_t d = (uint16_t)(blk[208] | (blk[209] << 8));
    if ((d & 0x7c00u) == 0x7c00u) atomicOr(bad, 1);
    dplane[i] = f16_to_f32(d);
    for (int t = 0; t < 16; ++t) scales[i * 16 + t] = blk[192 + t];
    auto dw = [&](int at) {
        return (uint32_t)blk[at] | ((uint32_t)blk[at + 1] << 8) | ((uint32_t)blk[at + 2] << 16) |
               ((uint32_t)blk[at + 3] << 24);
    };
    uint32_t* pb = qs + q6k_b_offset(N, K);
    for (int L = 0; L < 8; ++L) {
        uint32_t* a = qs + q6k_a_index(row, sb, L, nsb);
        a[0] = dw(4 * L);
        a[1] = dw(32 + 4 * L);
        a[2] = dw(64 + 4 * L);
        a[3] = dw(96 + 4 * L);
        uint32_t* h = pb + q6k_b_index(row, sb, L, nsb);
        h[0] = dw(128 + 4 * L);
        h[1] = dw(128 + 32 + 4 * L);
    }
}

hipError_t repack_weight(const uint8_t* d_gguf, DeviceWeight& w, int* d_bad, hipStream_t s) {
    if (w.type == kQ8_0) {
        const size_t nb = w.K / 32, n = w.N * nb;
        hipError_t e = hipMemsetAsync(w.qs, 0, w.qs_bytes, s);
        if (e == hipSuccess) e = hipMemsetAsync(w.hdr, 0, w.hdr_bytes, s);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(repack_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_gguf,
                           (int8_t*)w.qs, (uint16_t*)w.hdr, w.N, nb, d_bad);
    } else if (w.type == kQ4_K) {
        size_t nb = w.N * (w.K / 256);
        unsigned grid = (unsigned)((nb + 255) / 256);
        // the rows completing the last tile stay zero (d = dmin = 0)
        hipError_t e = hipMemsetAsync(w.qs, 0, w.qs_bytes, s);
        if (e == hipSuccess) e = hipMemsetAsync(w.hdr, 0, w.hdr_bytes, s);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(repack_q4k_kernel, dim3(grid), dim3(256), 0, s, (const v4i*)d_gguf, (uint8_t*)w.qs,
                           (v4u*)w.hdr, nb, w.K / 256, w.K, d_bad);
    } else if (w.type == kF32) {
        return hipMemcpyAsync(w.qs, d_gguf, w.qs_bytes, hipMemcpyDeviceToDevice, s);
    } else if (w.type == kQ4_1) {
        const size_t nb = w.K / 32, n = w.N * nb;
        hipError_t e = hipMemsetAsync(w.qs, 0, w.qs_bytes, s);
        if (e == hipSuccess) e = hipMemsetAsync(w.hdr, 0, w.hdr_bytes, s);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(repack_q41_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_gguf,
                           (uint16_t*)w.qs, (uint32_t*)w.hdr, w.N, nb, d_bad);
    } else if (w.type == kQ6_K) {
        const size_t n = w.N * (w.K / 256);
        hipError_t e = hipMemsetAsync(w.qs, 0, w.qs_bytes, s);
        if (e != hipSuccess) return e;
        uint8_t* sc = (uint8_t*)w.hdr;
        float* dp = (float*)(sc + w.N * (w.K / 256) * 16);
        hipLaunchKernelGGL(repack_q6k_kernel, dim3((unsigned)((n + 63) / 64)), dim3(64), 0, s, d_gguf,
                           (uint32_t*)w.qs, sc, dp, w.N, w.K, d_bad);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------- dequantize

__global__ void dequant_codec_kernel(int type, const void* __restrict__ qs, const void* __restrict__ hdr,
                                     float* __restrict__ out, size_t row0, size_t rows, size_t N, size_t K) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * K) return;
    const size_t row = row0 + i / K, e = i % K;
    if (type == kQ4_1) {
        out[i] = q41_element((const uint16_t*)qs, (const uint32_t*)hdr, row, e, K);
    } else {
        const uint8_t* sc = (const uint8_t*)hdr;
        const float* d = (const float*)(sc + N * (K / 256) * 16);
        out[i] = q6k_element((const uint32_t*)qs, sc, d, row, e, N, K);
    }
}

__global__ void dequant_q8_0_kernel(const int8_t* __restrict__ qs, const uint16_t* __restrict__ hdr,
                                    float* __restrict__ out, size_t row0, size_t rows, size_t nb) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const size_t row = row0 + i / nb, b = i % nb, nbc = (nb + 3) / 4;
    const float scale = f16_to_f32(hdr[row * nbc * 4 + b]);
#pragma unroll
    for (int e = 0; e < 32; ++e)
        out[i * 32 + e] = (float)qs[q8_tile_offset(row, b, e >> 2, nbc) + (e & 3)] * scale;
}

__global__ void dequant_q4k_kernel(const uint8_t* __restrict__ qs, const v4u* __restrict__ hdr,
                                   float* __restrict__ out, size_t row0, size_t nblocks, size_t nbk, size_t K) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const size_t row = row0 + b / nbk, kb = b % nbk;
    const v4u h = hdr[q4k_hdr_index(row, kb, nbk)];
    float d = f16_to_f32((uint16_t)(h.x & 0xffffu));
    float dmin = f16_to_f32((uint16_t)(h.x >> 16));
    for (int g = 0; g < 8; ++g) {
        uint32_t sc, mn;
        q4k_dev_scale_min(h, g, sc, mn);
        float scale = d * (float)sc;
        float mnf = dmin * (float)mn;
        const uint8_t* q = qs + q4k_chunk_offset(row, 4 * kb + (g >> 1), K);
        for (int i = 0; i < 32; ++i) {
            uint8_t byte = q[i < 16 ? i : 256 + i - 16];
            uint32_t v = (g & 1) ? (byte >> 4) : (byte & 15);
            out[b * 256 + g * 32 + i] = scale * (float)v - mnf;
        }
    }
}


hipError_t dequantize_rows(const DeviceWeight& w, size_t row0, size_t rows, float* out, hipStream_t s) {
    if (row0 + rows > w.N) return hipErrorInvalidValue;
    if (w.type == kQ8_0) {
        const size_t nb = w.K / 32, n = rows * nb;
        hipLaunchKernelGGL(dequant_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           (const int8_t*)w.qs, (const uint16_t*)w.hdr, out, row0, rows, nb);
    } else if (w.type == kQ4_K) {
        const size_t bpr = w.K / 256, nb = rows * bpr;
        hipLaunchKernelGGL(dequant_q4k_kernel, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, s,
                           (const uint8_t*)w.qs, (const v4u*)w.hdr, out, row0, nb, bpr, w.K);
    } else if (w.type == kF32) {
        return hipMemcpyAsync(out, (const float*)w.qs + row0 * w.K, rows * w.K * 4, hipMemcpyDeviceToDevice, s);
    } else if (w.type == kQ4_1 || w.type == kQ6_K) {
        const size_t n = rows * w.K;
        hipLaunchKernelGGL(dequant_codec_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w.type, w.qs,
                           w.hdr, out, row0, rows, w.N, w.K);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// --------------------------------------------------------- activation prep

// One workgroup per activation row.  RMS: f64 sum of f32-rounded squares
// (order-free to within f64 rounding), mean rounded to f32, inv = 1/sqrtf,
// y = (x*inv)*gamma.  Q8_0 coding per 32-block: amax, d = amax/127,
// inv = 127/amax, code = clamp(rint(y*inv)), scale stored f16-rounded.
template <bool XBF16>
__global__ __launch_bounds__(256) void act_prep_kernel(const void* __restrict__ x, int K,
                                                       const float* __restrict__ gamma, float eps,
                                                       float* __restrict__ xf, int8_t* __restrict__ aq,
                                                       float* __restrict__ ad, int16_t* __restrict__ x4,
                                                       float* __restrict__ m4) {
    extern __shared__ float sx[];
    __shared__ double red[4];
    __shared__ float inv_s;
    const size_t m = blockIdx.x;
    const int tid = threadIdx.x;
    for (int i = tid; i < K; i += 256) {
        sx[i] = XBF16 ? bf16_to_f32(((const uint16_t*)x)[m * K + i]) : ((const float*)x)[m * K + i];
    }
    __syncthreads();
    if (gamma) {
        double s = 0.0;
        for (int i = tid; i < K; i += 256) {
            float v = sx[i];
            float sq = v * v;
            s += (double)sq;
        }
        s = wave_sum_xor<double>(s, 64);
        if ((tid & 63) == 0) red[tid >> 6] = s;
        __syncthreads();
        if (tid == 0) {
            double total = (red[0] + red[1]) + (red[2] + red[3]);
            float mean = (float)(total / (double)K);
            float root = sqrtf(mean + eps);
            inv_s = 1.0f / root;
        }
        __syncthreads();
        const float inv = inv_s;
        for (int i = tid; i < K; i += 256) {
            float t = sx[i] * inv;
            sx[i] = t * gamma[i];
        }
        __syncthreads();
    }
    if (xf) {
        for (int i = tid; i < K; i += 256) xf[m * K + i] = sx[i];
    }
    if (aq) {
        const int nb = K >> 5;
        const int l = tid & 31;
        for (int b = tid >> 5; b < nb; b += 8) {
            float v = sx[b * 32 + l];
            float amax = fabsf(v);
            for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
            float d = amax / 127.0f;
            float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
            float r = rintf(v * inv);
            r = fminf(fmaxf(r, -128.0f), 127.0f);
            aq[m * K + b * 32 + l] = (int8_t)(int)r;
            if (l == 0) ad[m * nb + b] = f16_roundtrip(d);
        }
    }
    if (x4) {
        // Q4_K record per 64-element group pair (see gemv_q4k_kernel): 32
        // dwords of int16 pairs ordered XL0[8] XL1[8] XH0[8] XH1[8] where for
        // element t of a group, dword = (t&1 ? 8 : 0) + (t>>2), half = (t>>1)&1,
        // plus {xs_lo, xs_hi, sum_lo, sum_hi}.
        const int npc = K >> 6;
        const int l = tid & 31;
        for (int gi = tid >> 5; gi < 2 * npc; gi += 8) {  // one 32-lane group per 32 elements
            const int pc = gi >> 1, hi = gi & 1;
            const float v = sx[gi * 32 + l];
            float amax = fabsf(v), sum = v;
            for (int off = 16; off > 0; off >>= 1) {
                amax = fmaxf(amax, __shfl_xor(amax, off, 32));
                sum += __shfl_xor(sum, off, 32);
            }
            const float inv = amax == 0.0f ? 0.0f : 32767.0f / amax;
            const int q = (int)rintf(v * inv);
            const int dw = hi * 16 + ((l & 1) ? 8 : 0) + (l >> 2);
            const int half = (l >> 1) & 1;
            x4[((size_t)m * npc + pc) * 64 + dw * 2 + half] = (int16_t)q;
            if (l == 0) {
                m4[((size_t)m * npc + pc) * 4 + hi] = amax / 32767.0f;
                m4[((size_t)m * npc + pc) * 4 + 2 + hi] = sum;
            }
        }
    }
}

hipError_t act_prep(const void* x, int x_bf16, size_t M, size_t K, const float* gamma, float eps,
                    float* xf, int8_t* aq, float* ad, int16_t* x4, float* m4, hipStream_t s) {
    if (M == 0 || K == 0 || K > 8192 || (aq && K % 32) || (x4 && K % 256)) return hipErrorInvalidValue;
    size_t lds = K * sizeof(float);
    if (x_bf16)
        hipLaunchKernelGGL(act_prep_kernel<true>, dim3((unsigned)M), dim3(256), lds, s, x, (int)K, gamma, eps, xf,
                           aq, ad, x4, m4);
    else
        hipLaunchKernelGGL(act_prep_kernel<false>, dim3((unsigned)M), dim3(256), lds, s, x, (int)K, gamma, eps, xf,
                           aq, ad, x4, m4);
    return hipGetLastError();
}

size_t prepared_bytes(int type, size_t M, size_t K) {
    auto a = [](size_t n) { return (n + 255) & ~(size_t)255; };
    if (type == kQ8_0) return a(M * K) + a(M * (K / 32) * 4);
    if (type == kQ4_K) return a(M * K * 2) + a(M * (K / 64) * 16);
    return a(M * K * 4);
}

hipError_t act_prepare_for(int type, const void* x, int x_bf16, size_t M, size_t K, const float* gamma, float eps,
                           void* prepared, hipStream_t s) {
    auto a = [](size_t n) { return (n + 255) & ~(size_t)255; };
    char* base = (char*)prepared;
    if (type == kQ8_0) return act_prep(x, x_bf16, M, K, gamma, eps, nullptr, (int8_t*)base, (float*)(base + a(M * K)),
                                       nullptr, nullptr, s);
    if (type == kQ4_K) return act_prep(x, x_bf16, M, K, gamma, eps, nullptr, nullptr, nullptr, (int16_t*)base,
                                       (float*)(base + a(M * K * 2)), s);
    return act_prep(x, x_bf16, M, K, gamma, eps, (float*)base, nullptr, nullptr, nullptr, nullptr, s);
}

// ----------------------------------------------------------------- GEMV Q8_0

// Reference order (cpu/src/source/quantization.rs:171-196): for every row,
// eight f32 accumulators; accumulator l takes, block after block, the int32
// dot of elements 4l..4l+3 with the activation codes, fused-multiply-added
// with scale = f16(w.d) * act.d; the row value is
// ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)).  Here lane (row%8)*8 + l of a
// wavefront IS accumulator l of row (8 rows per wave), it walks the blocks
// in order, and the final tree is the XOR-4/2/1 shuffle tree (IEEE addition
// commutes, so each step reproduces the reference sum exactly): the result
// is bit-identical to the CPU.  The tile layout gives the wavefront one
// contiguous 1 KB load per 4 blocks; the MT activation rows (codes and
// scales) sit in LDS and every weight word is reused MT times.
template <int MT>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(const v4i* __restrict__ qs, const uint16_t* __restrict__ hdr,
                                                        const int8_t* __restrict__ aq, const float* __restrict__ ad,
                                                        float* __restrict__ y, int N, int K, int M) {
    extern __shared__ int lds_q8[];
    const int nb = K >> 5, nbc = (nb + 3) >> 2;
    int* codes = lds_q8;                          // [MT][K/4] words
    float* scales = (float*)(lds_q8 + MT * (K >> 2));  // [MT][nb]
    const int m0 = blockIdx.y * MT;
    for (int i = threadIdx.x; i < MT * (K >> 2); i += blockDim.x) {
        const int m = i / (K >> 2), w = i % (K >> 2);
        codes[i] = m0 + m < M ? ((const int*)aq)[(size_t)(m0 + m) * (K >> 2) + w] : 0;
    }
    for (int i = threadIdx.x; i < MT * nb; i += blockDim.x) {
        const int m = i / nb, b = i % nb;
        scales[i] = m0 + m < M ? ad[(size_t)(m0 + m) * nb + b] : 0.0f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int rl = lane >> 3, l = lane & 7;
    const int groups = (N + 7) >> 3;
    const int nwaves = gridDim.x * (blockDim.x >> 6);
    for (int R = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); R < groups; R += nwaves) {
        const int row = R * 8 + rl;
        const uint16_t* hrow = hdr + (size_t)(row < N ? row : N - 1) * nbc * 4;
        const v4i* tile = qs + (size_t)R * nbc * 64 + lane;
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int c = 0; c < nbc; ++c) {
            const v4i w4 = load_nt(tile + (size_t)c * 64);
            const uint2 h2 = *(const uint2*)(hrow + 4 * c);
            const int ww[4] = {w4.x, w4.y, w4.z, w4.w};
            const uint32_t hw[4] = {h2.x & 0xffffu, h2.x >> 16, h2.y & 0xffffu, h2.y >> 16};
#pragma unroll
            for (int bi = 0; bi < 4; ++bi) {
                const int b = 4 * c + bi;
                if (b < nb) {
                    const float wd = f16_to_f32((uint16_t)hw[bi]);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const int pair = __builtin_amdgcn_sdot4(ww[bi], codes[m * (K >> 2) + b * 8 + l], 0, false);
                        const float scale = wd * scales[m * nb + b];
                        acc[m] = fmaf((float)pair, scale, acc[m]);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[m] = acc[m] + __shfl_xor(acc[m], 4, 64);
            acc[m] = acc[m] + __shfl_xor(acc[m], 2, 64);
            acc[m] = acc[m] + __shfl_xor(acc[m], 1, 64);
        }
        if (l == 0 && row < N) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m0 + m < M) y[(size_t)(m0 + m) * N + row] = acc[m];
        }
    }
}

// ----------------------------------------------------------------- GEMV Q4_K

// A lane owns whole "pair chunks": 32 payload bytes = all 64 elements of the
// group pair (2p, 2p+1) of one 256-element block (low nibbles -> group 2p,
// high nibbles -> group 2p+1).  With lpr a multiple of 4 every chunk of a lane
// has the same p, so one header decode serves 64 elements.  The activation
// is carried as int16 fixed point per (lane, group): xq = rint(x * 32767/amax),
// relative precision 2^-15 of the group's max; nibble pairs are spread into
// int16 pairs with one mask (and a shift) and reduced with v_dot2_i32_i16 into
// an exact int32 group sum.  Per group:
//   acc += (d*sc) * (xs * isum) - (dmin*mn) * sum(x)        (f32)
// where sum(x) is the exact f32 sum of the group's activations.  MT
// activation rows share every converted weight dword.
template <int CH, int MT>
__global__ __launch_bounds__(256) void gemv_q4k_kernel(const uint8_t* __restrict__ qs,
                                                       const v4u* __restrict__ hdr,
                                                       const int16_t* __restrict__ xq, const float* __restrict__ xm,
                                                       float* __restrict__ y, int N, int K, int M, int lpr_log2) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int sub = lane & (lpr - 1);
    const int rsub = lane >> lpr_log2;
    const int rpw = 64 >> lpr_log2;
    const int nchunk = K >> 6;  // pair chunks per row
    const int nbk = K >> 8;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * (blockDim.x >> 6);
    const int m0 = blockIdx.y * MT;
    const int p = sub & 3;

    // activation records prepared by act_prep_kernel (int16 pairs in the
    // weight pair order, group scales and exact f32 group sums)
    int xl0[MT][CH][8], xl1[MT][CH][8], xh0[MT][CH][8], xh1[MT][CH][8];
    float xs_lo[MT][CH], xs_hi[MT][CH], sx_lo[MT][CH], sx_hi[MT][CH];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = sub + i * lpr;
            const bool ok = c < nchunk && m0 + m < M;
            if (ok) {
                const v4i* rec = (const v4i*)(xq + ((size_t)(m0 + m) * nchunk + c) * 64);
                const v4f mt4 = *(const v4f*)(xm + ((size_t)(m0 + m) * nchunk + c) * 4);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v4i r0 = rec[j], r1 = rec[2 + j], r2 = rec[4 + j], r3 = rec[6 + j];
                    xl0[m][i][4 * j + 0] = r0.x; xl0[m][i][4 * j + 1] = r0.y; xl0[m][i][4 * j + 2] = r0.z; xl0[m][i][4 * j + 3] = r0.w;
                    xl1[m][i][4 * j + 0] = r1.x; xl1[m][i][4 * j + 1] = r1.y; xl1[m][i][4 * j + 2] = r1.z; xl1[m][i][4 * j + 3] = r1.w;
                    xh0[m][i][4 * j + 0] = r2.x; xh0[m][i][4 * j + 1] = r2.y; xh0[m][i][4 * j + 2] = r2.z; xh0[m][i][4 * j + 3] = r2.w;
                    xh1[m][i][4 * j + 0] = r3.x; xh1[m][i][4 * j + 1] = r3.y; xh1[m][i][4 * j + 2] = r3.z; xh1[m][i][4 * j + 3] = r3.w;
                }
                xs_lo[m][i] = mt4.x;
                xs_hi[m][i] = mt4.y;
                sx_lo[m][i] = mt4.z;
                sx_hi[m][i] = mt4.w;
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) xl0[m][i][q] = xl1[m][i][q] = xh0[m][i][q] = xh1[m][i][q] = 0;
                xs_lo[m][i] = xs_hi[m][i] = sx_lo[m][i] = sx_hi[m][i] = 0.0f;
            }
        }
    }
    for (int rg = wave; rg * rpw < N; rg += nwaves) {
        const int row = rg * rpw + rsub;
        const bool rv = row < N;
        v4i w0[CH], w1[CH];
        v4u h[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = sub + i * lpr;
            if (rv && c < nchunk) {
                const uint8_t* base = qs + q4k_chunk_offset(row, c, K);
                w0[i] = load_nt(base);
                w1[i] = load_nt(base + 256);
                h[i] = hdr[q4k_hdr_index(row, c >> 2, nbk)];
            } else {
                w0[i] = v4i{0, 0, 0, 0};
                w1[i] = v4i{0, 0, 0, 0};
                h[i] = v4u{0u, 0u, 0u, 0u};
            }
        }
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const uint32_t ww[8] = {(uint32_t)w0[i].x, (uint32_t)w0[i].y, (uint32_t)w0[i].z, (uint32_t)w0[i].w,
                                    (uint32_t)w1[i].x, (uint32_t)w1[i].y, (uint32_t)w1[i].z, (uint32_t)w1[i].w};
            int ilo[MT], ihi[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) ilo[m] = ihi[m] = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t d = ww[q];
                const v2s L0 = __builtin_bit_cast(v2s, d & 0x000f000fu);
                const v2s L1 = __builtin_bit_cast(v2s, (d >> 8) & 0x000f000fu);
                const v2s H0 = __builtin_bit_cast(v2s, (d >> 4) & 0x000f000fu);
                const v2s H1 = __builtin_bit_cast(v2s, (d >> 12) & 0x000f000fu);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    ilo[m] = __builtin_amdgcn_sdot2(L0, __builtin_bit_cast(v2s, xl0[m][i][q]), ilo[m], false);
                    ilo[m] = __builtin_amdgcn_sdot2(L1, __builtin_bit_cast(v2s, xl1[m][i][q]), ilo[m], false);
                    ihi[m] = __builtin_amdgcn_sdot2(H0, __builtin_bit_cast(v2s, xh0[m][i][q]), ihi[m], false);
                    ihi[m] = __builtin_amdgcn_sdot2(H1, __builtin_bit_cast(v2s, xh1[m][i][q]), ihi[m], false);
                }
            }
            uint32_t sc0, mn0, sc1, mn1;
            q4k_dev_scale_min(h[i], 2 * p, sc0, mn0);
            q4k_dev_scale_min(h[i], 2 * p + 1, sc1, mn1);
            const float d = f16_to_f32((uint16_t)(h[i].x & 0xffffu));
            const float dmin = f16_to_f32((uint16_t)(h[i].x >> 16));
            const float s0 = d * (float)sc0, n0 = dmin * (float)mn0;
            const float s1 = d * (float)sc1, n1 = dmin * (float)mn1;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                acc[m] = fmaf(s0, xs_lo[m][i] * (float)ilo[m], acc[m]);
                acc[m] = fmaf(-n0, sx_lo[m][i], acc[m]);
                acc[m] = fmaf(s1, xs_hi[m][i] * (float)ihi[m], acc[m]);
                acc[m] = fmaf(-n1, sx_hi[m][i], acc[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = wave_sum_xor(acc[m], lpr);
        if (rv && sub == 0) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m0 + m < M) y[(size_t)(m0 + m) * N + row] = acc[m];
        }
    }
}

// ------------------------------------------------------------- dispatch

static int pick_lpr_log2(int nchunk, int target) {
    int l = 3;  // 8 lanes minimum: Q4_K needs lpr % 8 == 0
    while (l < 6 && (nchunk + (1 << l) - 1) / (1 << l) > target) ++l;
    return l;
}

static unsigned grid_for(size_t N, int lpr_log2) {
    const size_t rpw = 64u >> lpr_log2;
    size_t waves = (N + rpw - 1) / rpw;
    size_t wgs = (waves + 3) / 4;
    const size_t cap = 256 * 8;  // 8 workgroups per CU on 256 CUs, grid-stride beyond
    return (unsigned)(wgs < cap ? wgs : cap);
}

bool gemv_supported(int type, size_t K, size_t M) {
    if (M == 0 || M > 64 || K == 0) return false;
    switch (type) {
    case kQ8_0: return K % 32 == 0 && K <= 8192;
    case kQ4_K: return K % 256 == 0 && K <= 16384;
    case kQ4_1: return K % 32 == 0 && K <= 8192;
    case kQ6_K: return K % 256 == 0 && K <= 8192;
    case kF32: return K % 4 == 0 && K <= 8192;
    default: return false;
    }
}

hipError_t gemv(const DeviceWeight& w, size_t M, const void* prepared, float* y, hipStream_t s) {
    if (!gemv_supported(w.type, w.K, M)) return hipErrorInvalidValue;
    const int K = (int)w.K, N = (int)w.N;
    auto a = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const char* base = (const char*)prepared;
    const float* xf = (const float*)base;
    const int8_t* aq = (const int8_t*)base;
    const float* ad = (const float*)(base + a(M * w.K));
    const int16_t* x4 = (const int16_t*)base;
    const float* m4 = (const float*)(base + a(M * w.K * 2));
    if (w.type == kQ8_0 && M > 4 && q8_rows_supported(w.K, w.N, PRO_PLAIN))
        return q8_rows_prepared(w, M, prepared, y, s);  // weights streamed once per 16 rows
    if (w.type == kQ8_0) {
        int mt = M == 1 ? 1 : (M == 2 ? 2 : (M <= 4 ? 4 : 8));
        while (mt > 1 && (size_t)mt * (K + (K / 32) * 4) > 65536) mt >>= 1;
        const size_t lds = (size_t)mt * (K + (K / 32) * 4);
        const size_t groups = (w.N + 7) / 8;
        const unsigned wgs = (unsigned)std::min<size_t>((groups + 3) / 4, 256 * 8);
        dim3 g(wgs, (unsigned)((M + mt - 1) / mt));
        const v4i* q = (const v4i*)w.qs;
        const uint16_t* h = (const uint16_t*)w.hdr;
        if (mt == 1) hipLaunchKernelGGL(gemv_q8_0_kernel<1>, g, dim3(256), lds, s, q, h, aq, ad, y, N, K, (int)M);
        else if (mt == 2) hipLaunchKernelGGL(gemv_q8_0_kernel<2>, g, dim3(256), lds, s, q, h, aq, ad, y, N, K, (int)M);
        else if (mt == 4) hipLaunchKernelGGL(gemv_q8_0_kernel<4>, g, dim3(256), lds, s, q, h, aq, ad, y, N, K, (int)M);
        else hipLaunchKernelGGL(gemv_q8_0_kernel<8>, g, dim3(256), lds, s, q, h, aq, ad, y, N, K, (int)M);
    } else if (w.type == kQ4_K) {
        const int nchunk = K / 64;
        int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
        const int minch = (nchunk + 63) / 64;  // chunks per lane at 64 lanes per row
        while (mt > 1 && minch * mt > 4) mt >>= 1;
        const int chmax = 4 / mt;
        // Fewer chunks per lane keeps VGPRs (and so occupancy) in check; more
        // only when the row is too long for 64 lanes.
        const int target = minch > (2 / mt) ? minch : (mt == 1 ? 2 : 1);
        int l = 2;
        while (l < 6 && (nchunk + (1 << l) - 1) / (1 << l) > target) ++l;
        const int ch = (nchunk + (1 << l) - 1) >> l;
        if (ch > chmax) return hipErrorInvalidValue;
        dim3 g(grid_for(w.N, l), (unsigned)((M + mt - 1) / mt));
        const uint8_t* q = (const uint8_t*)w.qs;
        const v4u* h = (const v4u*)w.hdr;
#define ZG_Q4(C, T) hipLaunchKernelGGL((gemv_q4k_kernel<C, T>), g, dim3(256), 0, s, q, h, x4, m4, y, N, K, (int)M, l)
        if (mt == 1) {
            switch (ch) {
            case 1: ZG_Q4(1, 1); break;
            case 2: ZG_Q4(2, 1); break;
            case 3: ZG_Q4(3, 1); break;
            default: ZG_Q4(4, 1); break;
            }
        } else if (mt == 2) {
            if (ch == 1) ZG_Q4(1, 2); else ZG_Q4(2, 2);
        } else {
            ZG_Q4(1, 4);
        }
#undef ZG_Q4
    } else {
        // Q4_1, Q6_K and F32 over the f32 activation: the decode-step kernels
        // with a plain prologue (activation coding in-kernel)
        FusedGemvArgs f;
        f.M = (int)M;
        f.pro = PRO_PLAIN;
        f.epi = EPI_STORE;
        f.x = xf;
        f.ldx = w.K;
        f.y = y;
        f.ldy = w.N;
        return fused_gemv(w, f, s);
    }
    return hipGetLastError();
}

}  // namespace zg
