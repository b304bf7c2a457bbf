/*
 * zg_oracle.c — CPU restatement of zerogravity's GGUF Qwen3.5 decode path.
 * TEST INFRASTRUCTURE ONLY (parity checker + timed CPU baseline); the product
 * library never links or loads it.  Compiled -O2 -ffp-contract=off: every
 * fused multiply-add below is an explicit fmaf() standing for a Rust mul_add.
 * Citations are file:line in the zerogravity repository.
 */
#include "zg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int finite_all(const float* x, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(x[i])) return 0;
    return 1;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static float    bits_f32(uint32_t w) { float f; memcpy(&f, &w, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t w; memcpy(&w, &f, 4); return w; }

/* ---------------------------------------------------------------- codecs */

/* artifacts/src/codecs/mod.rs:13-32 */
float zgo_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)(bits & 0x8000u)) << 16;
    uint32_t exp = (bits >> 10) & 0x1f;
    uint32_t mant = bits & 0x03ffu;
    uint32_t word;
    if (exp == 0 && mant == 0) {
        word = sign;
    } else if (exp == 0) {
        uint32_t m = mant;
        int32_t e = 127 - 14;
        while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
        word = sign | ((uint32_t)e << 23) | ((m & 0x3ffu) << 13);
    } else if (exp == 31) {
        word = sign | 0x7f800000u | (mant << 13);
    } else {
        word = sign | ((exp + 112) << 23) | (mant << 13);
    }
    return bits_f32(word);
}

/* artifacts/src/codecs/mod.rs:205-237 */
uint16_t zgo_f32_to_f16_rne(float value) {
    uint32_t bits = f32_bits(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exponent = (int32_t)((bits >> 23) & 0xff);
    uint32_t fraction = bits & 0x7fffffu;
    if (exponent == 255)
        return (uint16_t)(sign | 0x7c00u | (fraction == 0 ? 0 : (((fraction >> 13) & 0xffffu) | 0x0200u)));
    int32_t half_exp = exponent - 127 + 15;
    if (half_exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (half_exp <= 0) {
        if (half_exp < -10) return sign;
        uint32_t mantissa = fraction | 0x800000u;
        uint32_t shift = (uint32_t)(14 - half_exp);
        uint32_t half = (mantissa + ((1u << (shift - 1)) - 1) + ((mantissa >> shift) & 1)) >> shift;
        return (uint16_t)(sign | (uint16_t)half);
    }
    uint32_t rounded = fraction + 0x0fffu + ((fraction >> 13) & 1);
    if (rounded >= 0x800000u) return (uint16_t)(sign | (uint16_t)((half_exp + 1) << 10));
    return (uint16_t)(sign | (uint16_t)(half_exp << 10) | (uint16_t)(rounded >> 13));
}

/* core/src/encoding.rs:52-62 (elements per block, bytes per block) */
int zgo_block_geometry(int t, uint64_t* elements, uint64_t* bytes) {
    switch (t) {
    case ZGO_F32: *elements = 1; *bytes = 4; return ZGO_OK;
    case ZGO_F16: case ZGO_BF16: *elements = 1; *bytes = 2; return ZGO_OK;
    case ZGO_Q4_0: *elements = 32; *bytes = 18; return ZGO_OK;
    case ZGO_Q4_1: *elements = 32; *bytes = 20; return ZGO_OK;
    case ZGO_Q8_0: *elements = 32; *bytes = 34; return ZGO_OK;
    case ZGO_Q4_K: *elements = 256; *bytes = 144; return ZGO_OK;
    case ZGO_Q6_K: *elements = 256; *bytes = 210; return ZGO_OK;
    default: return ZGO_E_UNSUPPORTED;
    }
}

/* Q4_K 6-bit scale/min unpack, codecs/q4.rs:58-65 */
static void q4k_scale_min(const uint8_t* packed, int group, uint8_t* sc, uint8_t* mn) {
    if (group < 4) {
        *sc = packed[group] & 63;
        *mn = packed[group + 4] & 63;
    } else {
        *sc = (uint8_t)((packed[group + 4] & 15) | ((packed[group - 4] >> 6) << 4));
        *mn = (uint8_t)((packed[group + 4] >> 4) | ((packed[group] >> 6) << 4));
    }
}

/* codecs/mod.rs:36-88 with q8.rs:6-15, q4.rs:6-70, q6.rs */
int zgo_dequantize(int t, const uint8_t* data, size_t nbytes, size_t elements, float* out) {
    uint64_t be, bb;
    if (zgo_block_geometry(t, &be, &bb) != ZGO_OK) return ZGO_E_UNSUPPORTED;
    if (elements % be != 0) return ZGO_E_MALFORMED;
    if ((uint64_t)nbytes != (elements / be) * bb) return ZGO_E_MALFORMED;
    size_t nb = elements / be;
    switch (t) {
    case ZGO_F32:
        memcpy(out, data, elements * 4);
        return ZGO_OK;
    case ZGO_F16:
        for (size_t i = 0; i < elements; ++i) out[i] = zgo_f16_to_f32(rd16(data + 2 * i));
        return ZGO_OK;
    case ZGO_BF16:
        for (size_t i = 0; i < elements; ++i) out[i] = bits_f32((uint32_t)rd16(data + 2 * i) << 16);
        return ZGO_OK;
    case ZGO_Q8_0:
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = data + b * 34;
            float scale = zgo_f16_to_f32(rd16(blk));
            if (!isfinite(scale)) return ZGO_E_MALFORMED;
            for (int i = 0; i < 32; ++i) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * scale;
        }
        return ZGO_OK;
    case ZGO_Q4_0:
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = data + b * 18;
            float scale = zgo_f16_to_f32(rd16(blk));
            if (!isfinite(scale)) return ZGO_E_MALFORMED;
            for (int i = 0; i < 16; ++i) out[b * 32 + i] = (float)(blk[2 + i] & 15) * scale - 8.0f * scale;
            for (int i = 0; i < 16; ++i) out[b * 32 + 16 + i] = (float)(blk[2 + i] >> 4) * scale - 8.0f * scale;
        }
        return ZGO_OK;
    case ZGO_Q4_1:
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = data + b * 20;
            float scale = zgo_f16_to_f32(rd16(blk));
            float mn = zgo_f16_to_f32(rd16(blk + 2));
            if (!isfinite(scale) || !isfinite(mn)) return ZGO_E_MALFORMED;
            for (int i = 0; i < 16; ++i) out[b * 32 + i] = fmaf((float)(blk[4 + i] & 15), scale, mn);
            for (int i = 0; i < 16; ++i) out[b * 32 + 16 + i] = fmaf((float)(blk[4 + i] >> 4), scale, mn);
        }
        return ZGO_OK;
    case ZGO_Q4_K:
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = data + b * 144;
            float d = zgo_f16_to_f32(rd16(blk));
            float dmin = zgo_f16_to_f32(rd16(blk + 2));
            if (!isfinite(d) || !isfinite(dmin)) return ZGO_E_MALFORMED;
            const uint8_t* packed = blk + 4;
            const uint8_t* values = blk + 16;
            for (int g = 0; g < 8; ++g) {
                uint8_t sc, mn;
                q4k_scale_min(packed, g, &sc, &mn);
                float scale = d * (float)sc;
                float mnf = dmin * (float)mn;
                int start = (g / 2) * 32;
                for (int i = 0; i < 32; ++i) {
                    uint8_t byte = values[start + i];
                    uint8_t v = (g & 1) ? (byte >> 4) : (byte & 15);
                    out[b * 256 + g * 32 + i] = scale * (float)v - mnf;
                }
            }
        }
        return ZGO_OK;
    case ZGO_Q6_K:
        /* codecs/q6.rs: ql[128] qh[64] scales[16] d(f16) */
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = data + b * 210;
            float d = zgo_f16_to_f32(rd16(blk + 208));
            if (!isfinite(d)) return ZGO_E_MALFORMED;
            for (int half = 0; half < 2; ++half) {
                const uint8_t* low = blk + half * 64;
                const uint8_t* high = blk + 128 + half * 32;
                const uint8_t* sc = blk + 192 + half * 8;
                for (int lane = 0; lane < 32; ++lane) {
                    uint8_t hi = high[lane];
                    for (int group = 0; group < 4; ++group) {
                        uint8_t lo = group < 2 ? (low[lane + group * 32] & 15) : (low[lane + (group - 2) * 32] >> 4);
                        float q = (float)((int)(lo | (((hi >> (2 * group)) & 3) << 4)) - 32);
                        float s = (float)(int8_t)sc[group * 2 + lane / 16];
                        out[b * 256 + half * 128 + group * 32 + lane] = d * s * q;
                    }
                }
            }
        }
        return ZGO_OK;
    default:
        return ZGO_E_UNSUPPORTED;
    }
}

/* ------------------------------------------------- activation coding (Q8_0) */

/* cpu/src/source/quantization.rs:37-61: per 32-block amax, d = amax/127,
 * inv = 127/amax, q = clamp(round_ties_even(x*inv)), d and s f16-roundtripped. */
int zgo_q8_activation(const float* x, size_t n, int8_t* qs, float* d, float* s) {
    if (!finite_all(x, n)) return ZGO_E_MALFORMED;
    if (n % 32 != 0) return ZGO_E_MALFORMED;
    for (size_t b = 0; b < n / 32; ++b) {
        const float* blk = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(blk[i]));
        float dd = amax / 127.0f;
        float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
        int32_t sum = 0;
        for (int i = 0; i < 32; ++i) {
            float r = rintf(blk[i] * inv);
            if (r < -128.0f) r = -128.0f;
            if (r > 127.0f) r = 127.0f;
            int8_t v = (int8_t)r;
            qs[b * 32 + i] = v;
            sum += v;
        }
        d[b] = zgo_f16_to_f32(zgo_f32_to_f16_rne(dd));
        if (s) s[b] = zgo_f16_to_f32(zgo_f32_to_f16_rne((float)sum * dd));
    }
    return ZGO_OK;
}

/* quantization.rs:171-196: per block scale = f16(w.d) * act.d; eight f32 lanes,
 * lane l accumulates fma(int dot of elements 4l..4l+3, scale, lane); final
 * ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)). */
float zgo_dot_q8_0_row(const uint8_t* row, const int8_t* qs, const float* d, size_t nblocks) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* w = row + b * 34;
        float scale = zgo_f16_to_f32(rd16(w)) * d[b];
        for (int lane = 0; lane < 8; ++lane) {
            int32_t pair = 0;
            for (int i = lane * 4; i < lane * 4 + 4; ++i)
                pair += (int32_t)(int8_t)w[2 + i] * (int32_t)qs[b * 32 + i];
            lanes[lane] = fmaf((float)pair, scale, lanes[lane]);
        }
    }
    float r0 = lanes[0] + lanes[4], r1 = lanes[1] + lanes[5];
    float r2 = lanes[2] + lanes[6], r3 = lanes[3] + lanes[7];
    return (r0 + r2) + (r1 + r3);
}

/* quantization.rs:66-92 (GgmlQ8K, Q6_K/Q4_K pairing): per 256-block the
 * FIRST element of largest magnitude (strict > while scanning in order)
 * gives the signed max; inv = -127/max_signed, d = 1/inv (0 for an all-zero
 * block), q = clamp(round_ties_even(x*inv)).  bsums (sums of 16 codes, used
 * by the Q6_K offset correction) are optional. */
int zgo_q8k_activation(const float* x, size_t n, int8_t* qs, float* d, int32_t* bsums) {
    if (!finite_all(x, n)) return ZGO_E_MALFORMED;
    if (n % 256 != 0) return ZGO_E_MALFORMED;
    for (size_t b = 0; b < n / 256; ++b) {
        const float* blk = x + b * 256;
        float max_signed = 0.0f, amax = 0.0f;
        for (int i = 0; i < 256; ++i)
            if (fabsf(blk[i]) > amax) {
                amax = fabsf(blk[i]);
                max_signed = blk[i];
            }
        float inv = amax == 0.0f ? 0.0f : -127.0f / max_signed;
        d[b] = amax == 0.0f ? 0.0f : 1.0f / inv;
        for (int i = 0; i < 256; ++i) {
            float r = rintf(blk[i] * inv);
            if (r < -128.0f) r = -128.0f;
            if (r > 127.0f) r = 127.0f;
            qs[b * 256 + i] = (int8_t)r;
        }
        if (bsums)
            for (int g = 0; g < 16; ++g) {
                int32_t t = 0;
                for (int i = 0; i < 16; ++i) t += qs[b * 256 + g * 16 + i];
                bsums[b * 16 + g] = t;
            }
    }
    return ZGO_OK;
}

/* quantization.rs:133-170 (Q4_0 x Q8_0, rows not a multiple of 8): eight f32
 * lanes, lane l takes elements 4l..4l+3 of each block (weights below 16 are
 * low nibbles of bytes i, the rest high nibbles of bytes i-16, minus 8),
 * lane = fma(d_w*d_a, int dot, lane); the same final tree as Q8_0. */
float zgo_dot_q4_0_row(const uint8_t* row, const int8_t* qs, const float* d, size_t nblocks) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* w = row + b * 18;
        float dd = zgo_f16_to_f32(rd16(w)) * d[b];
        const uint8_t* packed = w + 2;
        for (int lane = 0; lane < 8; ++lane) {
            int32_t dot = 0;
            for (int j = lane * 4; j < lane * 4 + 4; ++j) {
                int32_t q = j < 16 ? (int32_t)(packed[j] & 15) - 8 : (int32_t)(packed[j - 16] >> 4) - 8;
                dot += q * (int32_t)qs[b * 32 + j];
            }
            lanes[lane] = fmaf(dd, (float)dot, lanes[lane]);
        }
    }
    float r0 = lanes[0] + lanes[4], r1 = lanes[1] + lanes[5];
    float r2 = lanes[2] + lanes[6], r3 = lanes[3] + lanes[7];
    return (r0 + r2) + (r1 + r3);
}

/* quantization.rs:105-124 (Q4_0 x Q8_0, rows a multiple of 8, the GGML
 * 8x8-repacked schedule): one int32 sum per block, one fma per block. */
float zgo_dot_q4_0_repacked_row(const uint8_t* row, const int8_t* qs, const float* d, size_t nblocks) {
    float acc = 0.0f;
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* w = row + b * 18;
        const uint8_t* packed = w + 2;
        int32_t sum = 0;
        for (int i = 0; i < 16; ++i) {
            sum += ((int32_t)(packed[i] & 15) - 8) * (int32_t)qs[b * 32 + i];
            sum += ((int32_t)(packed[i] >> 4) - 8) * (int32_t)qs[b * 32 + i + 16];
        }
        float scale = zgo_f16_to_f32(rd16(w)) * d[b];
        acc = fmaf((float)sum, scale, acc);
    }
    return acc;
}

/* quantization.rs:198-227 (Q4_1 x Q8_1): eight f32 lanes as Q8_0 over the
 * unsigned nibbles, scale = d_w * d_a; the zero points accumulate apart,
 * summs = summs + m_w * s_a (product, then sum), added after the tree. */
float zgo_dot_q4_1_row(const uint8_t* row, const int8_t* qs, const float* d, const float* s, size_t nblocks) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float summs = 0.0f;
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* w = row + b * 20;
        float d0 = zgo_f16_to_f32(rd16(w));
        float m = zgo_f16_to_f32(rd16(w + 2));
        float ms = m * s[b];
        summs = summs + ms;
        float scale = d0 * d[b];
        const uint8_t* packed = w + 4;
        for (int lane = 0; lane < 8; ++lane) {
            int32_t partial = 0;
            for (int i = lane * 4; i < lane * 4 + 4; ++i) {
                int32_t q = i < 16 ? (int32_t)(packed[i] & 15) : (int32_t)(packed[i - 16] >> 4);
                partial += q * (int32_t)qs[b * 32 + i];
            }
            lanes[lane] = fmaf((float)partial, scale, lanes[lane]);
        }
    }
    float r0 = lanes[0] + lanes[4], r1 = lanes[1] + lanes[5];
    float r2 = lanes[2] + lanes[6], r3 = lanes[3] + lanes[7];
    return ((r0 + r2) + (r1 + r3)) + summs;
}

/* quantization.rs:228-285 (Q6_K x Q8_K): per 256-superblock eight int32
 * lanes; element at = 128*half + 32*group + lane32 (code = 6-bit value
 * before the -32 shift, local scale int8 scales[8*half + 2*group +
 * lane32/16]) adds code*scale*q8 to lane (at % 32) / 4.  Lane L then
 * subtracts 32 * sum over the contiguous 16-groups 2L, 2L+1 of
 * (bsum * scales[group16]); lane = fma((float)int, d_a * d_w, lane); the
 * Q8_0 final tree. */
float zgo_dot_q6k_row(const uint8_t* row, const int8_t* qs, const float* d, const int32_t* bsums, size_t nblocks) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* w = row + b * 210;
        const int8_t* q8 = qs + b * 256;
        float scale = d[b] * zgo_f16_to_f32(rd16(w + 208));
        int32_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int half = 0; half < 2; ++half) {
            const uint8_t* low = w + half * 64;
            const uint8_t* high = w + 128 + half * 32;
            const uint8_t* sc = w + 192 + half * 8;
            for (int lane = 0; lane < 32; ++lane) {
                uint8_t hi = high[lane];
                for (int group = 0; group < 4; ++group) {
                    uint8_t nib = group < 2 ? (low[lane + group * 32] & 15) : (low[lane + (group - 2) * 32] >> 4);
                    int32_t code = (int32_t)(nib | (((hi >> (2 * group)) & 3) << 4));
                    int32_t sub = (int32_t)(int8_t)sc[group * 2 + lane / 16];
                    int at = half * 128 + group * 32 + lane;
                    acc[(at % 32) / 4] += code * sub * (int32_t)q8[at];
                }
            }
        }
        const uint8_t* scales = w + 192;
        for (int L = 0; L < 8; ++L) {
            int32_t offset = 0;
            for (int sub = 0; sub < 2; ++sub) {
                int g16 = L * 2 + sub;
                offset += bsums[b * 16 + g16] * (int32_t)(int8_t)scales[g16];
            }
            acc[L] -= 32 * offset;
            lanes[L] = fmaf((float)acc[L], scale, lanes[L]);
        }
    }
    float r0 = lanes[0] + lanes[4], r1 = lanes[1] + lanes[5];
    float r2 = lanes[2] + lanes[6], r3 = lanes[3] + lanes[7];
    return (r0 + r2) + (r1 + r3);
}

/* cpu/src/source.rs:431-459: serial f32, sum += (q*scale - min) * x, no FMA. */
float zgo_dot_q4k_row(const uint8_t* row, const float* x, size_t nblocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* blk = row + b * 144;
        float d = zgo_f16_to_f32(rd16(blk));
        float dm = zgo_f16_to_f32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* q = blk + 16;
        const float* inp = x + b * 256;
        for (int g = 0; g < 8; ++g) {
            uint8_t sc, mn;
            q4k_scale_min(scales, g, &sc, &mn);
            float scale = d * (float)sc;
            float mnf = dm * (float)mn;
            const uint8_t* gb = q + (g / 2) * 32;
            const float* gx = inp + g * 32;
            for (int i = 0; i < 32; ++i) {
                uint8_t v = (g & 1) ? (gb[i] >> 4) : (gb[i] & 15);
                float t = (float)v * scale;
                t = t - mnf;
                t = t * gx[i];
                sum = sum + t;
            }
        }
    }
    return sum;
}

/* cpu/src/source.rs:325-366: 4x8 FMA accumulators over 32-element steps. */
float zgo_dot_f32_row(const uint8_t* row, const float* x, size_t n) {
    size_t np = n & ~(size_t)31;
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    for (size_t base = 0; base < np; base += 32)
        for (int j = 0; j < 4; ++j)
            for (int lane = 0; lane < 8; ++lane) {
                size_t idx = base + j * 8 + lane;
                float w;
                memcpy(&w, row + idx * 4, 4);
                acc[j][lane] = fmaf(w, x[idx], acc[j][lane]);
            }
    float red[8];
    for (int lane = 0; lane < 8; ++lane)
        red[lane] = (acc[0][lane] + acc[2][lane]) + (acc[1][lane] + acc[3][lane]);
    float h0 = red[0] + red[4], h1 = red[1] + red[5], h2 = red[2] + red[6], h3 = red[3] + red[7];
    float result = (h0 + h1) + (h2 + h3);
    for (size_t i = np; i < n; ++i) {
        float w;
        memcpy(&w, row + i * 4, 4);
        result += w * x[i];
    }
    return result;
}

/* dot_row (cpu/src/source.rs:431-459) of four rows at once: each row keeps
 * its own serial chain with exactly zgo_dot_q4k_row's operations and order
 * (so each result is bit-identical to it); interleaving four independent
 * chains only lets one core overlap their add latencies. */
static void dot_q4k_rows4(const uint8_t* const row[4], const float* x, size_t nblocks, float out[4]) {
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t b = 0; b < nblocks; ++b) {
        const float* inp = x + b * 256;
        float d[4], dm[4];
        const uint8_t* sc4[4];
        const uint8_t* q4[4];
        for (int r = 0; r < 4; ++r) {
            const uint8_t* blk = row[r] + b * 144;
            d[r] = zgo_f16_to_f32(rd16(blk));
            dm[r] = zgo_f16_to_f32(rd16(blk + 2));
            sc4[r] = blk + 4;
            q4[r] = blk + 16;
        }
        for (int g = 0; g < 8; ++g) {
            float scale[4], mnf[4];
            for (int r = 0; r < 4; ++r) {
                uint8_t sc, mn;
                q4k_scale_min(sc4[r], g, &sc, &mn);
                scale[r] = d[r] * (float)sc;
                mnf[r] = dm[r] * (float)mn;
            }
            const float* gx = inp + g * 32;
            for (int i = 0; i < 32; ++i) {
                for (int r = 0; r < 4; ++r) {
                    const uint8_t byte = q4[r][(g / 2) * 32 + i];
                    const uint8_t v = (g & 1) ? (byte >> 4) : (byte & 15);
                    float t = (float)v * scale[r];
                    t = t - mnf[r];
                    t = t * gx[i];
                    sum[r] = sum[r] + t;
                }
            }
        }
    }
    for (int r = 0; r < 4; ++r) out[r] = sum[r];
}

/* cpu/src/source.rs:234-313 (Source profile) with the pairing of
 * core/src/numerics.rs:96-122.  Q8_0 and Q4_0 pair with the dynamic Q8_0
 * activation (Q4_0 in the repacked schedule when rows % 8 == 0,
 * source.rs:286-296), Q4_1 with Q8_1, Q6_K with Q8_K; Q4_K uses dot_row
 * (source.rs:431-459) because the reference refuses a source-exact Q4_K
 * projection (source.rs:265-270); F32 uses the 4x8 FMA reduction.  Rows run
 * in parallel (Rayon, :285-305). */
int zgo_matvec(int t, const uint8_t* w, size_t wbytes, size_t rows, size_t cols,
               const float* x, float* y, int threads) {
    if (rows == 0 || rows > 1000000 || cols == 0 || !finite_all(x, cols)) return ZGO_E_MALFORMED;
    uint64_t be, bb;
    if (zgo_block_geometry(t, &be, &bb) != ZGO_OK) return ZGO_E_UNSUPPORTED;
    if (cols % be) return ZGO_E_MALFORMED;
    size_t row_bytes = (size_t)(cols / be * bb);
    if (row_bytes * rows != wbytes) return ZGO_E_MALFORMED;
    if (t != ZGO_Q8_0 && t != ZGO_Q4_K && t != ZGO_F32 && t != ZGO_Q4_0 && t != ZGO_Q4_1 && t != ZGO_Q6_K)
        return ZGO_E_UNSUPPORTED;
    int8_t* qs = NULL;
    float* dd = NULL;
    float* ss = NULL;
    int32_t* bs = NULL;
    if (t == ZGO_Q8_0 || t == ZGO_Q4_0 || t == ZGO_Q4_1) {
        qs = (int8_t*)malloc(cols);
        dd = (float*)malloc(sizeof(float) * (cols / 32));
        ss = (float*)malloc(sizeof(float) * (cols / 32));
        int rc = zgo_q8_activation(x, cols, qs, dd, ss);
        if (rc) { free(qs); free(dd); free(ss); return rc; }
    } else if (t == ZGO_Q6_K) {
        qs = (int8_t*)malloc(cols);
        dd = (float*)malloc(sizeof(float) * (cols / 256));
        bs = (int32_t*)malloc(sizeof(int32_t) * (cols / 16));
        int rc = zgo_q8k_activation(x, cols, qs, dd, bs);
        if (rc) { free(qs); free(dd); free(bs); return rc; }
    }
    long long nrows = (long long)rows;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (long long r = 0; r < nrows; ++r) {
        const uint8_t* row = w + (size_t)r * row_bytes;
        if (t == ZGO_Q4_K) {
            /* rows in groups of four per iteration (the whole group belongs
             * to the thread holding its first row) */
            if (r % 4) continue;
            if (r + 4 <= nrows) {
                const uint8_t* rows4[4] = {row, row + row_bytes, row + 2 * row_bytes, row + 3 * row_bytes};
                dot_q4k_rows4(rows4, x, cols / 256, y + r);
            } else {
                for (long long q = r; q < nrows; ++q) y[q] = zgo_dot_q4k_row(w + (size_t)q * row_bytes, x, cols / 256);
            }
        } else if (t == ZGO_Q8_0) y[r] = zgo_dot_q8_0_row(row, qs, dd, cols / 32);
        else if (t == ZGO_Q4_0 && rows % 8 == 0) y[r] = zgo_dot_q4_0_repacked_row(row, qs, dd, cols / 32);
        else if (t == ZGO_Q4_0) y[r] = zgo_dot_q4_0_row(row, qs, dd, cols / 32);
        else if (t == ZGO_Q4_1) y[r] = zgo_dot_q4_1_row(row, qs, dd, ss, cols / 32);
        else if (t == ZGO_Q6_K) y[r] = zgo_dot_q6k_row(row, qs, dd, bs, cols / 256);
        else y[r] = zgo_dot_f32_row(row, x, cols);
    }
    (void)threads;
    free(qs);
    free(dd);
    free(ss);
    free(bs);
    return finite_all(y, rows) ? ZGO_OK : ZGO_E_MALFORMED;
}

/* ------------------------------------------------------------------ norms */

/* model-qwen35/src/lib.rs:263-284: sum of f32 squares in f64, mean rounded
 * to f32, inv = 1/sqrtf(mean+eps), y = (x*inv)*w. */
int zgo_rms_norm(const float* x, const float* w, size_t n, float eps, float* out) {
    if (n == 0 || !isfinite(eps) || eps <= 0.0f) return ZGO_E_MALFORMED;
    if (!finite_all(x, n)) return ZGO_E_MALFORMED;
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        float sq = x[i] * x[i];
        sum += (double)sq;
    }
    float mean = (float)(sum / (double)n);
    float root = sqrtf(mean + eps);
    float inv = 1.0f / root;
    for (size_t i = 0; i < n; ++i) {
        float t = x[i] * inv;
        out[i] = t * w[i];
    }
    return finite_all(out, n) ? ZGO_OK : ZGO_E_MALFORMED;
}

/* lib.rs:289-306: independent per-group RMS sharing one gamma. */
int zgo_grouped_rms_norm(const float* x, const float* w, size_t width, size_t groups, float eps,
                         float* out) {
    if (width == 0 || groups == 0) return ZGO_E_MALFORMED;
    for (size_t g = 0; g < groups; ++g) {
        int rc = zgo_rms_norm(x + g * width, w, width, eps, out + g * width);
        if (rc) return rc;
    }
    return ZGO_OK;
}

/* --------------------------------------------------------- exp / SiLU / misc */

/* f32 transcendentals of the reference's platform libm: Rust f32::exp, ln,
 * sin_cos (lib.rs:324-336, 357, 1566) call the C library's expf, logf, sinf
 * and cosf on Linux, so the default mode (ZGO_LIBM_GLIBC) calls exactly
 * those.  ZGO_LIBM_CORRECT evaluates in double and rounds once: the
 * correctly rounded f32 value, which is what the HIP kernels compute; the
 * bit-exact device regression tests select it.  glibc's f32 routines miss
 * the correctly rounded value by one ulp on a small fraction of inputs. */
static int g_libm_mode = ZGO_LIBM_GLIBC;
int zgo_set_libm_mode(int mode) {
    const int old = g_libm_mode;
    if (mode == ZGO_LIBM_GLIBC || mode == ZGO_LIBM_CORRECT) g_libm_mode = mode;
    return old;
}
int zgo_libm_mode(void) { return g_libm_mode; }
static float cr_expf(float x) { return g_libm_mode == ZGO_LIBM_GLIBC ? expf(x) : (float)exp((double)x); }
static float cr_logf(float x) { return g_libm_mode == ZGO_LIBM_GLIBC ? logf(x) : (float)log((double)x); }
static float cr_sinf(float x) { return g_libm_mode == ZGO_LIBM_GLIBC ? sinf(x) : (float)sin((double)x); }
static float cr_cosf(float x) { return g_libm_mode == ZGO_LIBM_GLIBC ? cosf(x) : (float)cos((double)x); }

/* cpu/src/ops.rs:317-350: GGML Haswell vector exp, scalar form. */
float zgo_ggml_exp(float x) {
    if (!isfinite(x)) return expf(x);
    const float r = bits_f32(0x4b400000u);
    float z = fmaf(x, bits_f32(0x3fb8aa3bu), r);
    float n = z - r;
    float b = fmaf(-n, bits_f32(0x35bfbe8eu), fmaf(-n, bits_f32(0x3f317200u), x));
    uint32_t e = f32_bits(z) << 23;
    float k = bits_f32(e + 0x3f800000u);
    float u = b * b;
    float j = fmaf(fmaf(fmaf(bits_f32(0x3c072010u), b, bits_f32(0x3d2b9f17u)), u,
                        fmaf(bits_f32(0x3e2aaf33u), b, bits_f32(0x3efffedbu))),
                   u, bits_f32(0x3f7ffff6u) * b);
    if (fabsf(n) <= 126.0f) return fmaf(j, k, k);
    uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    float s1 = bits_f32(g + 0x7f000000u);
    float s2 = bits_f32(e - g);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

/* ops.rs:353-355 */
float zgo_ggml_silu(float x) { return x / (1.0f + zgo_ggml_exp(0.0f - x)); }

/* lib.rs:310-321: y = silu(x), optionally m[i]*y. */
int zgo_silu(const float* x, const float* m, size_t n, float* out) {
    if (n == 0 || !finite_all(x, n) || (m && !finite_all(m, n))) return ZGO_E_MALFORMED;
    for (size_t i = 0; i < n; ++i) {
        float y = zgo_ggml_silu(x[i]);
        out[i] = m ? m[i] * y : y;
    }
    return ZGO_OK;
}

/* lib.rs:324-326 */
float zgo_sigmoid(float x) { return 1.0f / (1.0f + cr_expf(-x)); }

/* lib.rs:328-336 */
float zgo_softplus(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return cr_expf(x);
    return cr_logf(1.0f + cr_expf(x));
}

/* lib.rs:1258-1271: kind 0 = Add, 1 = SigmoidGate a*sigmoid(b). */
int zgo_binary(int kind, const float* a, const float* b, size_t n, float* out) {
    if (n == 0 || !finite_all(a, n) || !finite_all(b, n)) return ZGO_E_MALFORMED;
    for (size_t i = 0; i < n; ++i) out[i] = kind == 0 ? a[i] + b[i] : a[i] * zgo_sigmoid(b[i]);
    return finite_all(out, n) ? ZGO_OK : ZGO_E_MALFORMED;
}

/* ---------------------------------------------------------------- GDN ops */

/* cpu/src/ops/gdn.rs:7-44: raw = c0*w0 + c1*w1 + c2*w2 + x*w3 (left to
 * right, no FMA); history becomes [c1, c2, x]. */
int zgo_gdn_conv_step(const float* act, const float* w, float* history, float* raw, size_t channels) {
    if (channels == 0 || !finite_all(act, channels) || !finite_all(w, channels * 4) ||
        !finite_all(history, channels * 3))
        return ZGO_E_MALFORMED;
    for (size_t c = 0; c < channels; ++c) {
        float* h = history + c * 3;
        const float* ww = w + c * 4;
        float t0 = h[0] * ww[0];
        float t1 = h[1] * ww[1];
        float t2 = h[2] * ww[2];
        float t3 = act[c] * ww[3];
        float s = t0 + t1;
        s = s + t2;
        s = s + t3;
        raw[c] = s;
        h[0] = h[1];
        h[1] = h[2];
        h[2] = act[c];
    }
    return finite_all(raw, channels) ? ZGO_OK : ZGO_E_MALFORMED;
}

/* lib.rs:339-362 */
int zgo_gdn_coefficients(const float* alpha, const float* beta, const float* dt, const float* a,
                         size_t heads, float scale, float* gain, float* beta_out,
                         float* softplus_out, float* gate_raw_out) {
    if (heads == 0 || !finite_all(alpha, heads) || !finite_all(beta, heads) ||
        !finite_all(dt, heads) || !finite_all(a, heads) || !isfinite(scale) || scale <= 0.0f)
        return ZGO_E_MALFORMED;
    for (size_t h = 0; h < heads; ++h) {
        float biased = alpha[h] + dt[h];
        float sp = zgo_softplus(biased);
        float gr = sp * a[h];
        if (softplus_out) softplus_out[h] = sp;
        if (gate_raw_out) gate_raw_out[h] = gr;
        gain[h] = cr_expf(gr);
        beta_out[h] = zgo_sigmoid(beta[h]);
        if (!isfinite(sp) || !isfinite(gr) || !isfinite(gain[h]) || !isfinite(beta_out[h]))
            return ZGO_E_STATE;
    }
    return ZGO_OK;
}

/* lib.rs:1394-1423: 4x8 FMA accumulators, tree, f64 tail. */
float zgo_source_dot_f32(const float* a, const float* b, size_t n) {
    size_t np = n & ~(size_t)31;
    float sums[4][8];
    memset(sums, 0, sizeof sums);
    for (size_t idx = 0; idx < np; idx += 32)
        for (int i = 0; i < 4; ++i)
            for (int lane = 0; lane < 8; ++lane) {
                size_t at = idx + i * 8 + lane;
                sums[i][lane] = fmaf(a[at], b[at], sums[i][lane]);
            }
    float comb[8];
    for (int i = 0; i < 8; ++i) comb[i] = (sums[0][i] + sums[2][i]) + (sums[1][i] + sums[3][i]);
    float h0 = comb[0] + comb[4], h1 = comb[1] + comb[5], h2 = comb[2] + comb[6], h3 = comb[3] + comb[7];
    float reduced = (h0 + h1) + (h2 + h3);
    double tail = 0.0;
    for (size_t i = np; i < n; ++i) {
        float p = a[i] * b[i];
        tail += (double)p;
    }
    return (float)((double)reduced + tail);
}

/* lib.rs:1446-1499: value-major state [j][i]; per column: decay, residual
 * dot with k, delta = (v_j - prev)*beta, col = fma(k, delta, col),
 * out_j = dot(col, q) * scale. */
int zgo_gdn_recurrent_step(float* state, const float* q, const float* k, const float* v,
                           float gain, float beta, float scale, float* out, size_t d) {
    if (d == 0 || !isfinite(gain) || !isfinite(beta) || !isfinite(scale) || !finite_all(q, d) ||
        !finite_all(k, d) || !finite_all(v, d) || !finite_all(state, d * d))
        return ZGO_E_MALFORMED;
    for (size_t j = 0; j < d; ++j) {
        float* col = state + j * d;
        for (size_t i = 0; i < d; ++i) col[i] *= gain;
        float prev = zgo_source_dot_f32(col, k, d);
        float delta = (v[j] - prev) * beta;
        for (size_t i = 0; i < d; ++i) col[i] = fmaf(k[i], delta, col[i]);
        out[j] = zgo_source_dot_f32(col, q, d) * scale;
    }
    if (!finite_all(state, d * d) || !finite_all(out, d)) return ZGO_E_MALFORMED;
    return ZGO_OK;
}

/* ------------------------------------------------------------- attention */

/* lib.rs:1552-1577: per head, angle starts at position, multiplied by
 * theta_scale after each pair; pairs (i, i + rotate/2); FMA form. */
int zgo_rope_kv(float* q, float* k, size_t hw, size_t qh, size_t kvh, size_t rotate, size_t pos,
                float theta_scale) {
    if (hw == 0 || qh == 0 || kvh == 0 || qh % kvh || rotate == 0 || rotate > hw || rotate % 2 ||
        pos > 2147483647u || !isfinite(theta_scale) || theta_scale <= 0.0f || theta_scale > 1.0f)
        return ZGO_E_MALFORMED;
    if (!finite_all(q, qh * hw) || !finite_all(k, kvh * hw)) return ZGO_E_MALFORMED;
    size_t half = rotate / 2;
    for (size_t hd = 0; hd < qh + kvh; ++hd) {
        float* head = hd < qh ? q + hd * hw : k + (hd - qh) * hw;
        float angle = (float)pos;
        for (size_t i = 0; i < half; ++i) {
            float s = cr_sinf(angle), c = cr_cosf(angle);
            float a = head[i], b = head[i + half];
            head[i] = fmaf(a, c, -(b * s));
            head[i + half] = fmaf(a, s, b * c);
            angle *= theta_scale;
        }
    }
    return ZGO_OK;
}

/* lib.rs:1427-1441: dots via source_dot_f32 over the kv head of each query
 * head (GQA), scores = dot * scale (separately rounded).  keys: [T][kvh*hw]. */
int zgo_attention_qk(const float* q, const float* keys, size_t T, size_t hw, size_t qh, size_t kvh,
                     float scale, float* dots, float* scores) {
    if (hw == 0 || qh == 0 || kvh == 0 || qh % kvh || T == 0 || !isfinite(scale) || scale <= 0.0f)
        return ZGO_E_MALFORMED;
    size_t group = qh / kvh, kvw = kvh * hw;
    for (size_t h = 0; h < qh; ++h) {
        size_t start = (h / group) * hw;
        for (size_t t = 0; t < T; ++t) {
            float dd = zgo_source_dot_f32(q + h * hw, keys + t * kvw + start, hw);
            if (dots) dots[h * T + t] = dd;
            scores[h * T + t] = dd * scale;
        }
    }
    return finite_all(scores, qh * T) ? ZGO_OK : ZGO_E_STATE;
}

/* lib.rs:1352-1387: per row max, exp_ggml(x-max) in 8-wide blocks, block
 * partial ((e0+e4)+(e2+e6))+((e1+e5)+(e3+e7)) summed in f64,
 * inv = (float)(1/sum), p = e*inv. */
int zgo_attention_softmax(const float* scores, size_t heads, size_t width, float* exps, float* probs,
                          double* sums) {
    if (heads == 0 || width == 0 || !finite_all(scores, heads * width)) return ZGO_E_MALFORMED;
    for (size_t h = 0; h < heads; ++h) {
        const float* row = scores + h * width;
        float mx = -INFINITY;
        for (size_t i = 0; i < width; ++i) mx = fmaxf(mx, row[i]);
        double sum = 0.0;
        for (size_t b = 0; b < width; b += 8) {
            float e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (size_t i = 0; i < 8 && b + i < width; ++i) e[i] = zgo_ggml_exp(row[b + i] - mx);
            float partial = ((e[0] + e[4]) + (e[2] + e[6])) + ((e[1] + e[5]) + (e[3] + e[7]));
            sum += (double)partial;
            for (size_t i = 0; i < 8 && b + i < width; ++i) {
                if (exps) exps[h * width + b + i] = e[i];
                probs[h * width + b + i] = e[i];
            }
        }
        double reciprocal = 1.0 / sum;
        float inv = (float)reciprocal;
        if (sums) sums[h] = sum;
        if (!isfinite(sum) || sum < 1.0) return ZGO_E_STATE;
        for (size_t i = 0; i < width; ++i) probs[h * width + i] = probs[h * width + i] * inv;
    }
    return ZGO_OK;
}

/* lib.rs:1276-1305: per (head, channel) 4x8 FMA lanes over tokens padded to
 * `padded` with +0*+0 terms; values: [T][kvh*hw]; probs: [qh][T]. */
int zgo_attention_value(const float* probs, const float* values, size_t T, size_t hw, size_t qh,
                        size_t kvh, size_t padded, float* out) {
    if (hw == 0 || qh == 0 || kvh == 0 || qh % kvh || T == 0 || padded < T || padded % 32)
        return ZGO_E_MALFORMED;
    size_t group = qh / kvh, kvw = kvh * hw;
    for (size_t h = 0; h < qh; ++h) {
        size_t kv = h / group;
        for (size_t j = 0; j < hw; ++j) {
            float sums[4][8];
            memset(sums, 0, sizeof sums);
            for (size_t p = 0; p < padded; ++p) {
                float value = 0.0f, prob = 0.0f;
                if (p < T) {
                    value = values[p * kvw + kv * hw + j];
                    prob = probs[h * T + p];
                }
                size_t lane = p % 32;
                sums[lane / 8][lane % 8] = fmaf(value, prob, sums[lane / 8][lane % 8]);
            }
            float red[8];
            for (int l = 0; l < 8; ++l) red[l] = (sums[0][l] + sums[2][l]) + (sums[1][l] + sums[3][l]);
            float t0 = red[0] + red[4], t1 = red[1] + red[5], t2 = red[2] + red[6], t3 = red[3] + red[7];
            out[h * hw + j] = (t0 + t1) + (t2 + t3);
        }
    }
    return finite_all(out, qh * hw) ? ZGO_OK : ZGO_E_STATE;
}

/* core/src/numerics.rs:126-140: first maximum wins; nonfinite is an error. */
int zgo_greedy(const float* logits, size_t n, uint32_t* out) {
    if (n == 0) return ZGO_E_MALFORMED;
    size_t best = 0;
    for (size_t i = 0; i < n; ++i) {
        if (!isfinite(logits[i])) return ZGO_E_MALFORMED;
        if (logits[i] > logits[best]) best = i;
    }
    *out = (uint32_t)best;
    return ZGO_OK;
}

/* ------------------------------------------------- chunked GDN prefill */

/* Unit-lower solve, numerics/torch_cpu/gdn/chunk.rs:16-76: separate products,
 * four interleaved accumulators, (s0+s2)+(s1+s3), scalar tail, then one
 * subtraction from the RHS.  Never FMA. a: [C][C], x: [C][W] in place. */
static void solve_unit_lower(const float* a, float* x, size_t C, size_t W) {
    for (size_t row = 0; row < C; ++row) {
        size_t vend = row / 4 * 4;
        for (size_t col = 0; col < W; ++col) {
            float s[4] = {0, 0, 0, 0};
            for (size_t st = 0; st < vend; st += 4)
                for (int l = 0; l < 4; ++l) {
                    float p = a[row * C + st + l] * x[(st + l) * W + col];
                    s[l] = s[l] + p;
                }
            float sum = (s[0] + s[2]) + (s[1] + s[3]);
            for (size_t kk = vend; kk < row; ++kk) {
                float p = a[row * C + kk] * x[kk * W + col];
                sum = sum + p;
            }
            x[row * W + col] -= sum;
        }
    }
}

/* matmul of chunk/core.rs:367-400: one FMA chain per output. */
static void mm(const float* A, const float* B, float* Cout, size_t m, size_t n, size_t k, int ta, int tb) {
    for (size_t r = 0; r < m; ++r)
        for (size_t c = 0; c < n; ++c) {
            float sum = 0.0f;
            for (size_t z = 0; z < k; ++z) {
                float av = ta ? A[z * m + r] : A[r * k + z];
                float bv = tb ? B[c * k + z] : B[z * n + c];
                sum = fmaf(av, bv, sum);
            }
            Cout[r * n + c] += sum;
        }
}

/* One chunk step of numerics/torch_cpu/gdn/chunk/core.rs:152-363 for one
 * head.  Inputs are already normalized (q carries the output scale), state
 * is key-major [k][v] and updated in place; out: [rows][W]. */
static void chunk_head(const float* qn, const float* kn, const float* v, const float* beta,
                       const float* logd, size_t rows, size_t C, size_t W, float* S, float* out,
                       float* work) {
    float* kb = work;                 /* C*W */
    float* vb = kb + C * W;           /* C*W */
    float* A = vb + C * W;            /* C*C */
    float* intra = A + C * C;         /* C*C */
    float* W2 = intra + C * C;        /* C*W  cumulative key */
    float* corr = W2 + C * W;         /* C*W */
    float* core = corr + C * W;       /* C*W */
    float* dq = core + C * W;         /* C*W */
    float* dk = dq + C * W;           /* C*W */
    float* g = dk + C * W;            /* C */
    float* qp = g + C;                /* C*W padded q */
    float* kp = qp + C * W;           /* C*W padded k */
    memset(work, 0, sizeof(float) * (C * W * 9 + C * C * 2 + C));
    double running = 0.0;
    for (size_t t = 0; t < C; ++t) {
        if (t < rows) {
            running += (double)logd[t];
            for (size_t d = 0; d < W; ++d) {
                qp[t * W + d] = qn[t * W + d];
                kp[t * W + d] = kn[t * W + d];
                kb[t * W + d] = kn[t * W + d] * beta[t];
                vb[t * W + d] = v[t * W + d] * beta[t];
            }
        } else {
            running += 0.0;
        }
        g[t] = (float)running;
    }
    memset(A, 0, sizeof(float) * C * C);
    memset(intra, 0, sizeof(float) * C * C);
    mm(kb, kp, A, C, C, W, 0, 1);
    mm(qp, kp, intra, C, C, W, 0, 1);
    for (size_t t = 0; t < C; ++t)
        for (size_t s = 0; s < C; ++s) {
            float decay = s <= t ? cr_expf(g[t] - g[s]) : 0.0f;
            A[t * C + s] *= decay;
            intra[t * C + s] *= decay;
        }
    /* decayed beta key (in W2) and new values (in vb) */
    for (size_t t = 0; t < C; ++t) {
        float e = cr_expf(g[t]);
        for (size_t d = 0; d < W; ++d) W2[t * W + d] = kb[t * W + d] * e;
        for (size_t d = 0; d < W; ++d) dq[t * W + d] = qp[t * W + d] * e;
    }
    solve_unit_lower(A, vb, C, W);
    solve_unit_lower(A, W2, C, W);
    float last = g[C - 1];
    for (size_t t = 0; t < C; ++t) {
        float e = cr_expf(last - g[t]);
        for (size_t d = 0; d < W; ++d) dk[t * W + d] = kp[t * W + d] * e;
    }
    float chunk_decay = cr_expf(last);
    float* pred = core; /* reuse: predicted = W2 * S */
    memset(pred, 0, sizeof(float) * C * W);
    mm(W2, S, pred, C, W, W, 0, 0);
    for (size_t i = 0; i < C * W; ++i) corr[i] = vb[i] - pred[i];
    float* inter = W2; /* W2 no longer needed */
    memset(inter, 0, sizeof(float) * C * W);
    mm(dq, S, inter, C, W, W, 0, 0);
    memset(core, 0, sizeof(float) * C * W);
    mm(intra, corr, core, C, W, C, 0, 0);
    for (size_t i = 0; i < C * W; ++i) core[i] += inter[i];
    float* news = A; /* need W*W: allocate separately */
    (void)news;
    float* S1 = (float*)calloc(W * W, sizeof(float));
    mm(dk, corr, S1, W, W, C, 1, 0);
    for (size_t i = 0; i < W * W; ++i) S1[i] += S[i] * chunk_decay;
    memcpy(S, S1, sizeof(float) * W * W);
    free(S1);
    for (size_t t = 0; t < rows; ++t) memcpy(out + t * W, core + t * W, sizeof(float) * W);
}

/* Chunked prefill over `tokens` for `heads` heads.  q, k, v: [T][H][d]
 * (raw; q and k are L2-normalized here with the GGUF two-stage rule of
 * forward.rs:564-576, and q carries the 1/sqrt(d) output scale);
 * beta, log_decay: [T][H]; state value-major [H][v][k] (the GGUF layout,
 * lib.rs:81-83), updated in place; out: [T][H][d]. */
int zgo_gdn_chunk_prefill(const float* q, const float* k, const float* v, const float* beta,
                          const float* log_decay, size_t T, size_t H, size_t d, size_t chunk,
                          float* state, float* out) {
    if (T == 0 || H == 0 || d == 0 || chunk == 0) return ZGO_E_MALFORMED;
    float inv_sqrt = 1.0f / sqrtf((float)d);
    float* scale = (float*)malloc(sizeof(float) * d);
    for (size_t i = 0; i < d; ++i) scale[i] = inv_sqrt;
    float eps = 1e-6f / (float)d;
    size_t C = chunk;
    float* qn = (float*)malloc(sizeof(float) * C * d);
    float* kn = (float*)malloc(sizeof(float) * C * d);
    float* vv = (float*)malloc(sizeof(float) * C * d);
    float* bb = (float*)malloc(sizeof(float) * C);
    float* ll = (float*)malloc(sizeof(float) * C);
    float* oo = (float*)malloc(sizeof(float) * C * d);
    float* work = (float*)malloc(sizeof(float) * (C * d * 9 + C * C * 2 + C));
    float* S = (float*)malloc(sizeof(float) * d * d);
    int rc = ZGO_OK;
    for (size_t h = 0; h < H && rc == ZGO_OK; ++h) {
        /* value-major -> key-major */
        float* sv = state + h * d * d;
        for (size_t j = 0; j < d; ++j)
            for (size_t i = 0; i < d; ++i) S[i * d + j] = sv[j * d + i];
        for (size_t t0 = 0; t0 < T && rc == ZGO_OK; t0 += C) {
            size_t rows = T - t0 < C ? T - t0 : C;
            for (size_t t = 0; t < rows; ++t) {
                size_t src = ((t0 + t) * H + h) * d;
                rc |= zgo_rms_norm(q + src, scale, d, eps, qn + t * d);
                rc |= zgo_rms_norm(k + src, scale, d, eps, kn + t * d);
                for (size_t i = 0; i < d; ++i) qn[t * d + i] *= inv_sqrt;
                memcpy(vv + t * d, v + src, sizeof(float) * d);
                bb[t] = beta[(t0 + t) * H + h];
                ll[t] = log_decay[(t0 + t) * H + h];
            }
            chunk_head(qn, kn, vv, bb, ll, rows, C, d, S, oo, work);
            for (size_t t = 0; t < rows; ++t)
                memcpy(out + ((t0 + t) * H + h) * d, oo + t * d, sizeof(float) * d);
        }
        for (size_t j = 0; j < d; ++j)
            for (size_t i = 0; i < d; ++i) sv[j * d + i] = S[i * d + j];
    }
    free(scale); free(qn); free(kn); free(vv); free(bb); free(ll); free(oo); free(work); free(S);
    return rc ? ZGO_E_MALFORMED : ZGO_OK;
}

/* ------------------------------------------------------------ whole model */

typedef struct layer_w {
    int full;                    /* 1 = full attention, 0 = GDN */
    const zgo_tensor *attn_norm, *post_norm, *ffn_gate, *ffn_up, *ffn_down;
    const zgo_tensor *qkv, *gate, *alpha, *beta, *ssm_out, *conv, *ssm_norm, *ssm_a, *ssm_dt;
    const zgo_tensor *wq, *wk, *wv, *wo, *q_norm, *k_norm;
} layer_w;

struct zgo_model {
    zgo_geometry g;
    int threads;
    const zgo_tensor* embd;
    const zgo_tensor* out_norm;
    layer_w* layers;
    char err[256];
};

struct zgo_session {
    zgo_model* m;
    unsigned layers;  /* kept here: destroying a session must not read its model */
    int position;
    float** conv;     /* per layer [3*6144] or NULL */
    float** rec;      /* per layer [H][d][d] value-major or NULL */
    float** keys;     /* per layer [max_ctx][kvw] or NULL */
    float** values;
    int kv_bf16;      /* round appended K/V to bf16 (device cache storage) */
};

static const zgo_tensor* find(const zgo_tensor* ts, size_t n, const char* name) {
    for (size_t i = 0; i < n; ++i)
        if (strcmp(ts[i].name, name) == 0) return &ts[i];
    return NULL;
}

static const zgo_tensor* findl(zgo_model* m, const zgo_tensor* ts, size_t n, unsigned layer,
                               const char* suffix) {
    char name[96];
    snprintf(name, sizeof name, "blk.%u.%s", layer, suffix);
    const zgo_tensor* t = find(ts, n, name);
    if (!t) snprintf(m->err, sizeof m->err, "missing tensor %s", name);
    return t;
}

zgo_model* zgo_model_create(const zgo_geometry* g, const zgo_tensor* ts, size_t n, int threads) {
    zgo_model* m = (zgo_model*)calloc(1, sizeof(zgo_model));
    m->g = *g;
    m->threads = threads;
    m->layers = (layer_w*)calloc(g->layers, sizeof(layer_w));
    m->embd = find(ts, n, "token_embd.weight");
    m->out_norm = find(ts, n, "output_norm.weight");
    if (!m->embd || !m->out_norm) {
        snprintf(m->err, sizeof m->err, "missing global tensors");
        return m;
    }
    for (unsigned i = 0; i < g->layers; ++i) {
        layer_w* L = &m->layers[i];
        /* config.rs:146-167: full attention where (i+1) % interval == 0 */
        L->full = ((i + 1) % g->full_attention_interval) == 0;
        L->attn_norm = findl(m, ts, n, i, "attn_norm.weight");
        L->post_norm = findl(m, ts, n, i, "post_attention_norm.weight");
        L->ffn_gate = findl(m, ts, n, i, "ffn_gate.weight");
        L->ffn_up = findl(m, ts, n, i, "ffn_up.weight");
        L->ffn_down = findl(m, ts, n, i, "ffn_down.weight");
        if (L->full) {
            L->wq = findl(m, ts, n, i, "attn_q.weight");
            L->wk = findl(m, ts, n, i, "attn_k.weight");
            L->wv = findl(m, ts, n, i, "attn_v.weight");
            L->wo = findl(m, ts, n, i, "attn_output.weight");
            L->q_norm = findl(m, ts, n, i, "attn_q_norm.weight");
            L->k_norm = findl(m, ts, n, i, "attn_k_norm.weight");
        } else {
            L->qkv = findl(m, ts, n, i, "attn_qkv.weight");
            L->gate = findl(m, ts, n, i, "attn_gate.weight");
            L->alpha = findl(m, ts, n, i, "ssm_alpha.weight");
            L->beta = findl(m, ts, n, i, "ssm_beta.weight");
            L->ssm_out = findl(m, ts, n, i, "ssm_out.weight");
            L->conv = findl(m, ts, n, i, "ssm_conv1d.weight");
            L->ssm_norm = findl(m, ts, n, i, "ssm_norm.weight");
            L->ssm_a = findl(m, ts, n, i, "ssm_a");
            L->ssm_dt = findl(m, ts, n, i, "ssm_dt.bias");
        }
    }
    return m;
}

void zgo_model_destroy(zgo_model* m) {
    if (!m) return;
    free(m->layers);
    free(m);
}

const char* zgo_model_error(const zgo_model* m) { return m->err[0] ? m->err : NULL; }

static size_t conv_ch(const zgo_model* m) { return (size_t)m->g.gdn_heads * m->g.gdn_dim * 3; }
static size_t kvw(const zgo_model* m) { return (size_t)m->g.kv_heads * m->g.head_dim; }

/* Round to the nearest bf16 (ties to even), kept as f32.  Models a device
 * KV cache stored in bf16; the reference itself keeps f32 keys and values. */
static float bf16_round(float x) {
    uint32_t b = f32_bits(x);
    b += 0x7fffu + ((b >> 16) & 1u);
    return bits_f32(b & 0xffff0000u);
}

void zgo_session_set_kv_bf16(zgo_session* s, int on) { s->kv_bf16 = on != 0; }

zgo_session* zgo_session_create(zgo_model* m) {
    if (m->err[0]) return NULL;
    zgo_session* s = (zgo_session*)calloc(1, sizeof(zgo_session));
    s->m = m;
    unsigned nl = m->g.layers;
    s->layers = nl;
    s->conv = (float**)calloc(nl, sizeof(float*));
    s->rec = (float**)calloc(nl, sizeof(float*));
    s->keys = (float**)calloc(nl, sizeof(float*));
    s->values = (float**)calloc(nl, sizeof(float*));
    size_t dd = (size_t)m->g.gdn_dim;
    for (unsigned i = 0; i < nl; ++i) {
        if (m->layers[i].full) {
            s->keys[i] = (float*)calloc((size_t)m->g.max_context * kvw(m), sizeof(float));
            s->values[i] = (float*)calloc((size_t)m->g.max_context * kvw(m), sizeof(float));
        } else {
            s->conv[i] = (float*)calloc(conv_ch(m) * 3, sizeof(float));
            s->rec[i] = (float*)calloc((size_t)m->g.gdn_heads * dd * dd, sizeof(float));
        }
    }
    return s;
}

void zgo_session_destroy(zgo_session* s) {
    if (!s) return;
    for (unsigned i = 0; i < s->layers; ++i) {
        free(s->conv[i]); free(s->rec[i]); free(s->keys[i]); free(s->values[i]);
    }
    free(s->conv); free(s->rec); free(s->keys); free(s->values);
    free(s);
}

int zgo_session_position(const zgo_session* s) { return s->position; }

static int project(zgo_model* m, const zgo_tensor* t, const float* x, float* y) {
    return zgo_matvec(t->ggml_type, t->data, t->nbytes, t->shape1, t->shape0, x, y, m->threads);
}

static const float* vec(const zgo_tensor* t) { return (const float*)t->data; }

#define TRY(x) do { int _rc = (x); if (_rc) { rc = _rc; goto done; } } while (0)

/* forward.rs:451-516 with gdn_layer :518-632 and attention_layer :634-755. */
int zgo_forward_token(zgo_session* s, uint32_t token, float* logits) {
    zgo_model* m = s->m;
    const zgo_geometry* g = &m->g;
    int rc = ZGO_OK;
    size_t H = g->hidden, F = g->ffn, V = g->vocab;
    size_t gh = g->gdn_heads, gd = g->gdn_dim, width = gh * gd;
    size_t nq = g->q_heads, nkv = g->kv_heads, hd = g->head_dim;
    if (token >= V) return ZGO_E_MALFORMED;
    if ((uint32_t)s->position >= g->max_context) return ZGO_E_LIMIT;
    size_t big = width * 3 > nq * hd * 2 ? width * 3 : nq * hd * 2;
    if (F > big) big = F;
    float* x = (float*)malloc(sizeof(float) * H);
    float* nrm = (float*)malloc(sizeof(float) * H);
    float* attn = (float*)malloc(sizeof(float) * H);
    float* t1 = (float*)malloc(sizeof(float) * big);
    float* t2 = (float*)malloc(sizeof(float) * big);
    float* t3 = (float*)malloc(sizeof(float) * big);
    float* t4 = (float*)malloc(sizeof(float) * big);
    float* t5 = (float*)malloc(sizeof(float) * big);
    float* probs = NULL;
    /* embedding: lib.rs:740-752 -> cpu/src/source.rs:214-222 */
    {
        uint64_t be, bb;
        zgo_block_geometry(m->embd->ggml_type, &be, &bb);
        size_t rowb = H / be * bb;
        TRY(zgo_dequantize(m->embd->ggml_type, m->embd->data + (size_t)token * rowb, rowb, H, x));
    }
    for (unsigned i = 0; i < g->layers; ++i) {
        layer_w* L = &m->layers[i];
        TRY(zgo_rms_norm(x, vec(L->attn_norm), H, g->eps, nrm));
        if (!L->full) {
            float *qkv = t1, *z = t2, *raw = t3, *mixed = t4, *core = t5;
            float alpha[64], beta_p[64], gain[64], beta_c[64];
            TRY(project(m, L->qkv, nrm, qkv));
            TRY(project(m, L->gate, nrm, z));
            TRY(project(m, L->alpha, nrm, alpha));
            TRY(project(m, L->beta, nrm, beta_p));
            TRY(zgo_gdn_conv_step(qkv, vec(L->conv), s->conv[i], raw, width * 3));
            TRY(zgo_silu(raw, NULL, width * 3, mixed));
            float scale = 1.0f / sqrtf((float)gd);
            TRY(zgo_gdn_coefficients(alpha, beta_p, vec(L->ssm_dt), vec(L->ssm_a), gh, scale, gain,
                                     beta_c, NULL, NULL));
            float sc[512];
            for (size_t d = 0; d < gd; ++d) sc[d] = 1.0f / sqrtf((float)gd);
            /* q,k two-stage L2 in place over mixed[0 : 2*width] */
            TRY(zgo_grouped_rms_norm(mixed, sc, gd, gh * 2, g->eps / (float)gd, raw));
            const float* q = raw;
            const float* k = raw + width;
            const float* v = mixed + width * 2;
            for (size_t h = 0; h < gh; ++h)
                TRY(zgo_gdn_recurrent_step(s->rec[i] + h * gd * gd, q + h * gd, k + h * gd, v + h * gd,
                                           gain[h], beta_c[h], scale, core + h * gd, gd));
            TRY(zgo_grouped_rms_norm(core, vec(L->ssm_norm), gd, gh, g->eps, t3));
            TRY(zgo_silu(z, t3, width, t4));
            TRY(project(m, L->ssm_out, t4, attn));
        } else {
            float *qp = t1, *kp = t2, *vp = t3;
            TRY(project(m, L->wq, nrm, qp));
            TRY(project(m, L->wk, nrm, kp));
            TRY(project(m, L->wv, nrm, vp));
            float* rq = t4;
            float* gates = t5;
            for (size_t h = 0; h < nq; ++h) {
                memcpy(rq + h * hd, qp + h * hd * 2, sizeof(float) * hd);
                memcpy(gates + h * hd, qp + h * hd * 2 + hd, sizeof(float) * hd);
            }
            float* qn = qp; /* reuse after copy */
            TRY(zgo_grouped_rms_norm(rq, vec(L->q_norm), hd, nq, g->eps, qn));
            float kn[4096];
            TRY(zgo_grouped_rms_norm(kp, vec(L->k_norm), hd, nkv, g->eps, kn));
            float theta_scale = powf(10000000.0f, -2.0f / 64.0f);
            TRY(zgo_rope_kv(qn, kn, hd, nq, nkv, 64, (size_t)s->position, theta_scale));
            size_t T = (size_t)s->position + 1;
            memcpy(s->keys[i] + (size_t)s->position * kvw(m), kn, sizeof(float) * kvw(m));
            memcpy(s->values[i] + (size_t)s->position * kvw(m), vp, sizeof(float) * kvw(m));
            if (s->kv_bf16) {
                float* kr = s->keys[i] + (size_t)s->position * kvw(m);
                float* vr = s->values[i] + (size_t)s->position * kvw(m);
                for (size_t e = 0; e < kvw(m); ++e) {
                    kr[e] = bf16_round(kr[e]);
                    vr[e] = bf16_round(vr[e]);
                }
            }
            float* scores = (float*)malloc(sizeof(float) * nq * T);
            probs = (float*)malloc(sizeof(float) * nq * T);
            int r2 = zgo_attention_qk(qn, s->keys[i], T, hd, nq, nkv, 1.0f / sqrtf((float)hd), NULL, scores);
            if (!r2) r2 = zgo_attention_softmax(scores, nq, T, NULL, probs, NULL);
            free(scores);
            if (!r2) r2 = zgo_attention_value(probs, s->values[i], T, hd, nq, nkv, (T + 255) / 256 * 256, rq);
            free(probs);
            probs = NULL;
            TRY(r2);
            TRY(zgo_binary(1, rq, gates, nq * hd, kp));
            TRY(project(m, L->wo, kp, attn));
        }
        TRY(zgo_binary(0, x, attn, H, x));
        TRY(zgo_rms_norm(x, vec(L->post_norm), H, g->eps, nrm));
        TRY(project(m, L->ffn_gate, nrm, t1));
        TRY(project(m, L->ffn_up, nrm, t2));
        TRY(zgo_silu(t1, t2, F, t3));
        TRY(project(m, L->ffn_down, t3, attn));
        TRY(zgo_binary(0, x, attn, H, x));
        if (!finite_all(x, H)) { rc = ZGO_E_MALFORMED; goto done; }
    }
    s->position += 1;
    if (logits) {
        TRY(zgo_rms_norm(x, vec(m->out_norm), H, g->eps, nrm));
        TRY(zgo_matvec(m->embd->ggml_type, m->embd->data, m->embd->nbytes, V, H, nrm, logits, m->threads));
    }
done:
    free(x); free(nrm); free(attn); free(t1); free(t2); free(t3); free(t4); free(t5); free(probs);
    return rc;
}

size_t zgo_state_floats(const zgo_session* s) {
    const zgo_model* m = s->m;
    size_t n = 0;
    for (unsigned i = 0; i < m->g.layers; ++i) {
        if (m->layers[i].full) n += 2 * (size_t)s->position * kvw(m);
        else n += conv_ch(m) * 3 + (size_t)m->g.gdn_heads * m->g.gdn_dim * m->g.gdn_dim;
    }
    return n;
}

/* lib.rs:112-150 domain order. */
int zgo_state_export(const zgo_session* s, float* out, size_t n) {
    if (n != zgo_state_floats(s)) return ZGO_E_MALFORMED;
    const zgo_model* m = s->m;
    size_t at = 0;
    for (unsigned i = 0; i < m->g.layers; ++i) {
        if (m->layers[i].full) {
            size_t k = (size_t)s->position * kvw(m);
            memcpy(out + at, s->keys[i], sizeof(float) * k); at += k;
            memcpy(out + at, s->values[i], sizeof(float) * k); at += k;
        } else {
            size_t c = conv_ch(m) * 3, r = (size_t)m->g.gdn_heads * m->g.gdn_dim * m->g.gdn_dim;
            memcpy(out + at, s->conv[i], sizeof(float) * c); at += c;
            memcpy(out + at, s->rec[i], sizeof(float) * r); at += r;
        }
    }
    return ZGO_OK;
}

int zgo_state_import(zgo_session* s, const float* in, size_t n, int position) {
    int saved = s->position;
    s->position = position;
    if (position < 0 || (unsigned)position > s->m->g.max_context || n != zgo_state_floats(s)) {
        s->position = saved;
        return ZGO_E_MALFORMED;
    }
    const zgo_model* m = s->m;
    size_t at = 0;
    for (unsigned i = 0; i < m->g.layers; ++i) {
        if (m->layers[i].full) {
            size_t k = (size_t)position * kvw(m);
            memcpy(s->keys[i], in + at, sizeof(float) * k); at += k;
            memcpy(s->values[i], in + at, sizeof(float) * k); at += k;
        } else {
            size_t c = conv_ch(m) * 3, r = (size_t)m->g.gdn_heads * m->g.gdn_dim * m->g.gdn_dim;
            memcpy(s->conv[i], in + at, sizeof(float) * c); at += c;
            memcpy(s->rec[i], in + at, sizeof(float) * r); at += r;
        }
    }
    return ZGO_OK;
}
