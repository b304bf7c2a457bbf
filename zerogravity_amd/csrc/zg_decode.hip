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
//     codes [8][nbp] words (word l of block b at l * nbp + b, nbp = K/32
//     rounded up to 4), scales [K/32].
//   Q8_1 (quantization.rs:37-61, Q4_1 pairing): as Q8_0 (codes [8][nb8],
//     nb8 = K/32 rounded up to 8), plus per block s = f16(sum of codes *
//     unrounded d) in `extra`.
//   Q8_K (quantization.rs:66-92, Q6_K pairing): per 256-block (one
//     wavefront) the first element of largest magnitude gives the signed
//     max, inv = -127/max, d = 1/inv in `extra` [K/256], codes as Q8_0 laid
//     out lane-major (word w of block sb at (w%8)*(K/32) + 8sb + w/8), and
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
                // (word w of block sb: lane w % 8, slot w / 8) are adjacent
                const int w = (k >> 2) & 63, sb = k >> 8;
                codes[(size_t)(w & 7) * (K >> 5) + sb * 8 + (w >> 3)] = (int)word;
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
                // lane-major: word l * nb8 + block (nb8 = blocks rounded to
                // 8), so that two 16-byte reads serve an 8-block chunk
                const int nb8 = ((K >> 5) + 7) & ~7;
                codes[(size_t)l * nb8 + (k >> 5)] = (int)word;
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
                // lane-major: word l * nbp + block (nbp = blocks rounded to
                // 4), so that one 16-byte read serves four blocks
                const int nbp = ((K >> 5) + 3) & ~3;
                codes[(size_t)l * nbp + (k >> 5)] = (int)word;
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

// ============================================================= Q4_K GEMV

// Lanes: `lpr` per row, chunk c = sub + i*lpr (i < CH) is the group pair
// (2p, 2p+1) of block c/4: elements 64c .. 64c+63; the per-group epilogue
// is gemv_q4k_kernel's.  Weight byte e of the chunk holds element e of the
// low group (low nibble) and of the high group (high nibble), so a weight
// dword masked to its low or high nibbles meets the activation record's
// byte dwords lane for lane in one signed and one unsigned 4-way dot.  The
// workgroup codes the activation into LDS once (its weight loads for the
// first row group are already in flight), each lane copies its chunk
// records to registers.
template <int CH, int MT, int J, int RG, int PRO, int EPI>
__global__ __launch_bounds__(256) void fused_q4k_kernel(FusedGemvArgs a, int lpr_log2) {
    extern __shared__ uint32_t lds_q4[];
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int sub = lane & (lpr - 1);
    const int rsub = lane >> lpr_log2;
    const int rpw = 64 >> lpr_log2;
    const int K = a.K, N = a.N;
    const int nchunk = K >> 6, nbk = K >> 8;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * 4;
    const int m0 = blockIdx.y * MT;
    const int p = sub & 3;
    const uint8_t* qs = (const uint8_t*)a.qs;
    const v4u* hdr = (const v4u*)a.hdr;

    // row of lane group rsub in row group rg; with EPI_GLU a row group holds
    // rpw/2 (gate j, up j) pairs: even groups gate row j, odd groups up row
    // N/2 + j
    auto row_of = [&](int rg) {
        if (EPI == EPI_GLU) {
            const int j = rg * (rpw >> 1) + (rsub >> 1);
            return (rsub & 1) ? (N >> 1) + j : j;
        }
        return rg * rpw + rsub;
    };
    auto row_ok = [&](int rg) {
        if (EPI == EPI_GLU) return rg * (rpw >> 1) + (rsub >> 1) < (N >> 1);
        return rg * rpw + rsub < N;
    };
    // RG consecutive row groups per wave, all their loads issued together.
    // The loads are unconditional: a row past N reads row 0 (its sums are
    // never stored) and a chunk past the row end reads the row's last chunk
    // (its activation record is zero, so it adds exactly nothing).  Branches
    // around the loads would join with register copies that wait for them.
    v4i w0[RG][CH], w1[RG][CH];
    v4u h[RG][CH];
    auto load_rows = [&](int rg0) {
#pragma unroll
        for (int r = 0; r < RG; ++r) {
            const int row = row_ok(rg0 + r) ? row_of(rg0 + r) : 0;
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int c = min(sub + i * lpr, nchunk - 1);
                const uint8_t* base = qs + (size_t)row * (K >> 1) + (size_t)c * 32;
                w0[r][i] = load_nt(base);
                w1[r][i] = load_nt(base + 16);
                h[r][i] = hdr[(size_t)row * nbk + (c >> 2)];
            }
        }
    };
    // activation row 0's loads go first, then the weights', so that its
    // coding does not wait for the weights
    ProIn<J> pin;
    wg_prologue_load<PRO, J>(a, m0, m0 < a.M, pin);
    load_rows(wave * RG);

    wg_prologue_code<PRO, kCodecQ4K, J>(a, m0 < a.M, pin, lds_q4, nullptr, nullptr);
#pragma unroll
    for (int m = 1; m < MT; ++m)
        wg_prologue<PRO, kCodecQ4K, J>(a, m0 + m, m0 + m < a.M, lds_q4 + (size_t)m * nchunk * kRecWords, nullptr,
                                    nullptr);

    int xl0[MT][CH][8], xl1[MT][CH][8], xh0[MT][CH][8], xh1[MT][CH][8];
    float xs_lo[MT][CH], xs_hi[MT][CH], sx_lo[MT][CH], sx_hi[MT][CH];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = sub + i * lpr;
            if (c < nchunk) {
                const v4u* r = (const v4u*)(lds_q4 + ((size_t)m * nchunk + c) * kRecWords);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v4u r0 = r[j], r1 = r[2 + j], r2 = r[4 + j], r3 = r[6 + j];
                    xl0[m][i][4 * j + 0] = r0.x; xl0[m][i][4 * j + 1] = r0.y; xl0[m][i][4 * j + 2] = r0.z; xl0[m][i][4 * j + 3] = r0.w;
                    xl1[m][i][4 * j + 0] = r1.x; xl1[m][i][4 * j + 1] = r1.y; xl1[m][i][4 * j + 2] = r1.z; xl1[m][i][4 * j + 3] = r1.w;
                    xh0[m][i][4 * j + 0] = r2.x; xh0[m][i][4 * j + 1] = r2.y; xh0[m][i][4 * j + 2] = r2.z; xh0[m][i][4 * j + 3] = r2.w;
                    xh1[m][i][4 * j + 0] = r3.x; xh1[m][i][4 * j + 1] = r3.y; xh1[m][i][4 * j + 2] = r3.z; xh1[m][i][4 * j + 3] = r3.w;
                }
                const v4u mt = r[8];
                xs_lo[m][i] = __uint_as_float(mt.x);
                xs_hi[m][i] = __uint_as_float(mt.y);
                sx_lo[m][i] = __uint_as_float(mt.z);
                sx_hi[m][i] = __uint_as_float(mt.w);
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) xl0[m][i][q] = xl1[m][i][q] = xh0[m][i][q] = xh1[m][i][q] = 0;
                xs_lo[m][i] = xs_hi[m][i] = sx_lo[m][i] = sx_hi[m][i] = 0.0f;
            }
        }

    bool first = true;
    for (int rg0 = wave * RG; rg0 * rpw < N; rg0 += nwaves * RG) {  // (GLU: rg0 * rpw/2 < N/2, the same)
        if (!first) load_rows(rg0);
        first = false;
#pragma unroll
        for (int r = 0; r < RG; ++r) {
            const int row = row_of(rg0 + r);
            const bool rok = row_ok(rg0 + r);
            float acc[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const uint32_t ww[8] = {(uint32_t)w0[r][i].x, (uint32_t)w0[r][i].y, (uint32_t)w0[r][i].z,
                                        (uint32_t)w0[r][i].w, (uint32_t)w1[r][i].x, (uint32_t)w1[r][i].y,
                                        (uint32_t)w1[r][i].z, (uint32_t)w1[r][i].w};
                // sum of nibble * xq over each group, exactly: 256 * (nibbles .
                // signed high bytes) + (nibbles . unsigned low bytes)
                int ilo_h[MT], ihi_h[MT];
                uint32_t ilo_l[MT], ihi_l[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    ilo_h[m] = ihi_h[m] = 0;
                    ilo_l[m] = ihi_l[m] = 0u;
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t d = ww[q];
                    const uint32_t wl = d & 0x0f0f0f0fu, wh = (d >> 4) & 0x0f0f0f0fu;
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        ilo_h[m] = __builtin_amdgcn_sdot4((int)wl, xl0[m][i][q], ilo_h[m], false);
                        ilo_l[m] = __builtin_amdgcn_udot4(wl, (uint32_t)xl1[m][i][q], ilo_l[m], false);
                        ihi_h[m] = __builtin_amdgcn_sdot4((int)wh, xh0[m][i][q], ihi_h[m], false);
                        ihi_l[m] = __builtin_amdgcn_udot4(wh, (uint32_t)xh1[m][i][q], ihi_l[m], false);
                    }
                }
                int ilo[MT], ihi[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    ilo[m] = ilo_h[m] * 256 + (int)ilo_l[m];
                    ihi[m] = ihi_h[m] * 256 + (int)ihi_l[m];
                }
                uint32_t sc0, mn0, sc1, mn1;
                q4k_dev_scale_min(h[r][i], 2 * p, sc0, mn0);
                q4k_dev_scale_min(h[r][i], 2 * p + 1, sc1, mn1);
                const float d = f16_to_f32((uint16_t)(h[r][i].x & 0xffffu));
                const float dmin = f16_to_f32((uint16_t)(h[r][i].x >> 16));
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
            for (int m = 0; m < MT; ++m) acc[m] = group_sum_last(acc[m], lpr_log2);
            if (EPI == EPI_GLU) {
                // the gate sum sits in the last lane of the group before
                float gv[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) gv[m] = __shfl(acc[m], lane >= lpr ? lane - lpr : lane, 64);
                if (rok && (rsub & 1) && sub == lpr - 1) {
                    const int j = row - (N >> 1);
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        if (m0 + m < a.M) a.y[(size_t)(m0 + m) * a.ldy + j] = acc[m] * ggml_silu(gv[m]);
                }
            } else if (rok && sub == lpr - 1) {
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    if (m0 + m < a.M) epilogue(a, m0 + m, row, acc[m], EPI);
            }
        }
    }
}

// ============================================================= Q8_0 GEMV

// The workgroup codes MT activation rows into LDS (wg_prologue), then runs
// gemv_q8_0_kernel's row loop: the bit-exact reference order.  A wave's
// tiles stream in chunks of QC through two register buffers, the next
// chunk's loads issued before the current one is consumed; activation row
// 0's loads go out before the first chunk's and its coding overlaps them (a
// wave's loads complete in issue order).  Loads are unconditional: a tile
// past the row end reads the last one and is not consumed.
template <int MT, int J, int PRO, int EPI>
__global__ __launch_bounds__(256) void fused_q8_kernel(FusedGemvArgs a) {
    constexpr int QC = 8;
    extern __shared__ int lds_f8[];
    const int K = a.K, N = a.N;
    const int nb = K >> 5, nbc = (nb + 3) >> 2, nbp = nbc * 4;
    int* codes = lds_f8;                                 // [MT][8][nbp] words
    float* scales = (float*)(lds_f8 + MT * 8 * nbp);   // [MT][nbp]
    const int m0 = blockIdx.y * MT;
    const v4i* qs = (const v4i*)a.qs;
    const uint16_t* hdr = (const uint16_t*)a.hdr;
    const int lane = threadIdx.x & 63;
    const int rl = lane >> 3, l = lane & 7;
    const int groups = (N + 7) >> 3;
    const int nwaves = gridDim.x * 4;
    struct Chunk {
        v4i w[QC];
        uint2 h[QC];
    };
    auto load_chunk = [&](int R, int c0, Chunk& ck) {
        const int row = min(R * 8 + rl, N - 1);
        const uint16_t* hrow = hdr + (size_t)row * nbc * 4;
        const v4i* tile = qs + (size_t)min(R, groups - 1) * nbc * 64 + lane;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const int c = min(c0 + i, nbc - 1);
            ck.w[i] = load_nt(tile + (size_t)c * 64);
            ck.h[i] = *(const uint2*)(hrow + 4 * c);
        }
    };
    float acc[MT];
    auto consume = [&](const Chunk& ck, int c0) {
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const int c = c0 + i;
            if (c >= nbc) break;  // uniform
            const int ww[4] = {ck.w[i].x, ck.w[i].y, ck.w[i].z, ck.w[i].w};
            const uint32_t hw[4] = {ck.h[i].x & 0xffffu, ck.h[i].x >> 16, ck.h[i].y & 0xffffu, ck.h[i].y >> 16};
            v4i cw[MT];
            v4f sw[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                cw[m] = *(const v4i*)(codes + (size_t)(m * 8 + l) * nbp + 4 * c);
                sw[m] = *(const v4f*)(scales + (size_t)m * nbp + 4 * c);
            }
#pragma unroll
            for (int bi = 0; bi < 4; ++bi) {
                const int b = 4 * c + bi;
                if (b < nb) {
                    const float wd = f16_to_f32((uint16_t)hw[bi]);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const int xc = bi == 0 ? cw[m].x : bi == 1 ? cw[m].y : bi == 2 ? cw[m].z : cw[m].w;
                        const float xs = bi == 0 ? sw[m].x : bi == 1 ? sw[m].y : bi == 2 ? sw[m].z : sw[m].w;
                        const int pair = __builtin_amdgcn_sdot4(ww[bi], xc, 0, false);
                        const float scale = wd * xs;
                        acc[m] = fmaf((float)pair, scale, acc[m]);
                    }
                }
            }
        }
    };
    ProIn<J> pin;
    wg_prologue_load<PRO, J>(a, m0, m0 < a.M, pin);
    const int R0 = blockIdx.x * 4 + (threadIdx.x >> 6);
    Chunk ca, cb;
    load_chunk(R0, 0, ca);
    wg_prologue_code<PRO, kCodecQ8, J>(a, m0 < a.M, pin, nullptr, codes, scales);
#pragma unroll
    for (int m = 1; m < MT; ++m)
        wg_prologue<PRO, kCodecQ8, J>(a, m0 + m, m0 + m < a.M, nullptr, codes + (size_t)m * 8 * nbp,
                                   scales + (size_t)m * nbp);
    for (int R = R0; R < groups; R += nwaves) {
        if (R != R0) load_chunk(R, 0, ca);
        const int row = R * 8 + rl;
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int c0 = 0; c0 < nbc; c0 += 2 * QC) {
            if (c0 + QC < nbc) load_chunk(R, c0 + QC, cb);
            consume(ca, c0);
            if (c0 + QC >= nbc) break;
            if (c0 + 2 * QC < nbc) load_chunk(R, c0 + 2 * QC, ca);
            consume(cb, c0 + QC);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = group8_tree_last(acc[m]);  // the reference's lane tree, in lane 7
        if (row < N && l == 7) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m0 + m < a.M) epilogue(a, m0 + m, row, acc[m], EPI);
        }
    }
}

// ============================================== batched rows: f16 MFMA

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

// One workgroup per activation row (rows M..Mpad-1 zero): the prologue
// values of wg_prologue, rounded once to f16, into xh in the MFMA A-operand
// order of 32-row tiles: element (m, k) of tile mt = m/32 sits at
// ((mt*(K/256) + k/256)*16 + (k%256)/16)*64 + (k%16)/8*32 + m%32, times 8,
// plus k%8, so that lane l of the MFMA kernel loads step s of its K block
// as 16 contiguous bytes and a wave-instruction reads 1 KB contiguous.
template <int PRO, int JMAX>
__global__ __launch_bounds__(256) void act16_kernel(FusedGemvArgs a, _Float16* __restrict__ xh) {
    __shared__ double red[4];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, K = a.K;
    const bool valid = m < a.M;
    v4f v[JMAX], w[JMAX];
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
        const int k = 4 * tid + 1024 * j;
        v[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        w[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (valid && k < K) {
            v[j] = *(const v4f*)(a.x + (size_t)m * a.ldx + k);
            if (PRO == PRO_RMS) w[j] = *(const v4f*)(a.gamma + k);
            if (PRO == PRO_GATED || PRO == PRO_SILU_MUL) w[j] = *(const v4f*)(a.x2 + (size_t)m * a.ldx2 + k);
        }
    }
    if (PRO == PRO_RMS && a.rsplits > 0) {
        // the residual the previous (split-K) GEMM left pending: x += sum of
        // its partial tiles, split 0 first, written back as the new x
        const size_t mpad = (size_t)gridDim.x;
#pragma unroll
        for (int j = 0; j < JMAX; ++j) {
            const int k = 4 * tid + 1024 * j;
            if (valid && k < K) {
                v4f acc = *(const v4f*)(a.rparts + (size_t)m * K + k);
                for (int z = 1; z < a.rsplits; ++z) acc = acc + *(const v4f*)(a.rparts + ((size_t)z * mpad + m) * K + k);
                v[j] = v[j] + acc;
                *(v4f*)(a.xw + (size_t)m * a.ldx + k) = v[j];
                if (!finite_f32(v[j].x) || !finite_f32(v[j].y) || !finite_f32(v[j].z) || !finite_f32(v[j].w))
                    atomicOr(a.status, 1);
            }
        }
    }
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
        if (1024 * j >= K) break;
        float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        const float o[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
        if (PRO == PRO_RMS) {
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = (e[t] * inv) * o[t];
        } else if (PRO == PRO_GATED) {
            double s = 0.0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float q = e[t] * e[t];
                s += (double)q;
            }
            s = group_sum_last<32>(s);
            s = __shfl(s, (lane & 32) | 31, 64);
            const float gi = rms_inv(s, a.group, a.eps);
            const v4f g = k < K ? *(const v4f*)(a.gamma + (k & (a.group - 1))) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            const float gg[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = ((e[t] * gi) * gg[t]) * ggml_silu(o[t]);
        } else if (PRO == PRO_SILU_MUL) {
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = o[t] * ggml_silu(e[t]);
        }
        if (k < K) {
            typedef _Float16 h4v __attribute__((ext_vector_type(4)));
            h4v hv4;
#pragma unroll
            for (int t = 0; t < 4; ++t) hv4[t] = valid ? (_Float16)e[t] : (_Float16)0.0f;
            const size_t lane_t = (size_t)((k & 15) >> 3) * 32 + (m & 31);
            const size_t at = a.xh_rows ? (size_t)m * K + k
                                        : ((((size_t)(m >> 5) * (K >> 8) + (k >> 8)) * 16 + ((k & 255) >> 4)) * 64 +
                                           lane_t) * 8 + (k & 7);
            *(h4v*)(xh + at) = hv4;
        }
    }
}

// Y[m][n] = sum_k X[m][k] W[n][k] over 32-row activation blocks on v_mfma_f32_32x32x16_f16:
// A = X tile (32 rows m x 16 k), B = dequantized weights (16 k x 32 rows n),
// so D[i = m][j = n] and the lanes of a row store adjacent outputs.  Lane l
// holds A[m = l%32][k = 8*(l/32) + e] and B[k = 8*(l/32) + e][n = l%32]
// (e < 8); D register r is row m = (r%4) + 8*(r/4) + 4*(l/32), column
// n = l%32.  Per 256-element Q4_K block a lane uses the 8-byte pieces
// 32*c4 + 16*half + 8*(l/32) of its weight row: K step s (16 per block)
// uses piece (s/4, s%2), nibble (s/2)&1, group s/2.  Weights, headers and
// activations come in tile order (ensure_mfma_tiles, act16_kernel): each
// wave-instruction reads one contiguous run.  Weights are
// dequantized on packed f16: the nibble q becomes the f16 1024 + q by a
// byte permute, 1024 is subtracted exactly, and w = fma(q, scale, -min)
// with the group's scale and min rounded once to f16 (one rounding of the
// weight, against the reference's f32 q*scale - min then rounded to f16:
// they differ by the f16 rounding of scale and min).  Activations arrive in
// f16.  A wave owns NT tiles of 32 weight rows for 32 activation rows, so
// every activation load feeds NT MFMAs.
template <int EPI, int KS, int NT>
__global__ __launch_bounds__(64 * KS) void mfma_q4k_kernel(FusedGemvArgs a, const _Float16* __restrict__ xh) {
    // KS waves share the NT output tiles and split their K blocks (wave w
    // takes blocks w, w+KS, ...); the partial tiles are summed in a fixed
    // order through LDS, so the result does not depend on timing.
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    __shared__ float red[KS][16][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, hsel = lane >> 5, r32 = lane & 31;
    const int m0 = blockIdx.y * 32;
    const int K = a.K, N = a.N, nbk = K >> 8;
    bool nv[NT];
    int nbase[NT];
    const v4u* qtile[NT];
    const v4u* htile[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        // EPI_GLU (NT = 2): gate tile x and the up tile N/64 tiles later
        const int tile = EPI == EPI_GLU ? blockIdx.x + t * (N >> 6) : blockIdx.x * NT + t;
        nbase[t] = tile * 32;
        nv[t] = nbase[t] + r32 < N;
        const int tt = min(tile, (N - 1) >> 5);  // tiles past the end read the last one (results dropped)
        qtile[t] = (const v4u*)a.qs + (size_t)tt * nbk * 256 + lane;
        htile[t] = (const v4u*)a.hdr + (size_t)tt * nbk * 32 + r32;
    }
    const h8v* xtile = (const h8v*)xh + (size_t)blockIdx.y * nbk * 1024 + lane;
    f16v acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f16v{};
    // K blocks of this workgroup: all, or its 1/gridDim.z share (split-K)
    const int per = (nbk + gridDim.z - 1) / gridDim.z;
    const int kb0 = blockIdx.z * per, kb1 = min(nbk, kb0 + per);
    for (int kb = kb0 + wv; kb < kb1; kb += KS) {
        uint2 pc[NT][4][2];
        v4u hd[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const v4u q = qtile[t][((size_t)kb * 4 + c4) * 64];
                pc[t][c4][0] = make_uint2(q.x, q.y);
                pc[t][c4][1] = make_uint2(q.z, q.w);
            }
            hd[t] = htile[t][(size_t)kb * 32];
        }
        h8v xa[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) xa[s] = xtile[((size_t)kb * 16 + s) * 64];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float d = f16_to_f32((uint16_t)(hd[t].x & 0xffffu));
            const float dmin = f16_to_f32((uint16_t)(hd[t].x >> 16));
            h2v sc2[8], nm2[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                uint32_t sc, mn;
                q4k_dev_scale_min(hd[t], g, sc, mn);
                const _Float16 sh = (_Float16)(d * (float)sc), mh = (_Float16)(dmin * (float)mn);
                sc2[g] = h2v{sh, sh};
                nm2[g] = h2v{-mh, -mh};
            }
            const h2v bias = h2v{(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int g = s >> 1, nib = (s >> 1) & 1;
                const uint2 pw = pc[t][s >> 2][s & 1];
                const uint32_t w0 = (nib ? (pw.x >> 4) : pw.x) & 0x0f0f0f0fu;
                const uint32_t w1 = (nib ? (pw.y >> 4) : pw.y) & 0x0f0f0f0fu;
                // bytes (q, 0x64) pairs: the f16 bit patterns of 1024 + q
                const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
                const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
                const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
                const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
                const h2v e0 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p0) - bias, sc2[g], nm2[g]);
                const h2v e1 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p1) - bias, sc2[g], nm2[g]);
                const h2v e2 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p2) - bias, sc2[g], nm2[g]);
                const h2v e3 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p3) - bias, sc2[g], nm2[g]);
                h8v wb = h8v{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
                if (!nv[t]) wb = h8v{};
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[s], wb, acc[t], 0, 0, 0);
            }
        }
    }
    float vg[16 / KS];  // EPI_GLU: the gate tile's sums
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wv][r][lane] = acc[t][r];
        __syncthreads();
        // wave w finishes registers r = w, w+KS, ... of every lane
#pragma unroll
        for (int i = 0; i < 16 / KS; ++i) {
            const int r = wv + KS * i;
            float v;
            if (KS == 4) {
                v = (red[0][r][lane] + red[1][r][lane]) + (red[2][r][lane] + red[3][r][lane]);
            } else {
                v = ((red[0][r][lane] + red[1][r][lane]) + (red[2][r][lane] + red[3][r][lane])) +
                    ((red[4][r][lane] + red[5][r][lane]) + (red[6][r][lane] + red[7][r][lane]));
            }
            const int m = m0 + (r & 3) + 8 * (r >> 2) + 4 * hsel;
            if (EPI == EPI_GLU) {
                if (t == 0) {
                    vg[i] = v;
                } else if (nv[t]) {
                    // up * silu(gate), rounded to f16 into the down
                    // projection's activation tiles (K2 = N/2 columns)
                    const int j = nbase[0] + r32, nbk2 = (N >> 1) >> 8;
                    const size_t at = ((((size_t)(m >> 5) * nbk2 + (j >> 8)) * 16 + ((j & 255) >> 4)) * 64 +
                                       ((j & 15) >> 3) * 32 + (m & 31)) * 8 + (j & 7);
                    ((_Float16*)a.xh_out)[at] = (_Float16)(m < a.M ? v * ggml_silu(vg[i]) : 0.0f);
                }
            } else if (gridDim.z > 1) {
                if (nv[t]) a.parts[((size_t)blockIdx.z * 32 * gridDim.y + m) * N + nbase[t] + r32] = v;
            } else if (nv[t] && m < a.M) {
                epilogue(a, m, nbase[t] + r32, v, EPI);
            }
        }
        __syncthreads();
    }
}

// The same product for prompt-sized M (>= 1024 rows).  A workgroup of 4
// waves covers MB activation blocks of 32 rows and 4*NT weight tiles (NT per
// wave, K not split): each 256-element K block of the MB activation tiles
// is staged once in LDS for the four waves (the next block's loads in
// flight meanwhile), and every dequantized weight step feeds MB MFMAs.
// Weights, headers, activations, the dequantization and the epilogues
// (store, residual add, SwiGLU with NT = 2: gate tile x, up tile x + N/64)
// are those of mfma_q4k_kernel.
template <int EPI, int NT, int MB>
__global__ __launch_bounds__(256) void mfma_q4k_wide_kernel(FusedGemvArgs a, const _Float16* __restrict__ xh) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    __shared__ h8v xs[MB * 1024];  // MB activation tiles of one K block (16 KB each)
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hsel = lane >> 5, r32 = lane & 31;
    const int K = a.K, N = a.N, nbk = K >> 8;
    const int mblk0 = blockIdx.y * MB;
    bool nv[NT];
    int nbase[NT];
    const v4u* qtile[NT];
    const v4u* htile[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tile = EPI == EPI_GLU ? blockIdx.x * 4 + wv + t * (N >> 6) : (blockIdx.x * 4 + wv) * NT + t;
        nbase[t] = tile * 32;
        nv[t] = nbase[t] + r32 < N;
        const int tt = min(tile, (N - 1) >> 5);
        qtile[t] = (const v4u*)a.qs + (size_t)tt * nbk * 256 + lane;
        htile[t] = (const v4u*)a.hdr + (size_t)tt * nbk * 32 + r32;
    }
    const h8v* xg = (const h8v*)xh;
    h8v stage[MB][4];
    auto load_stage = [&](int kb) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) stage[mb][i] = xg[((size_t)(mblk0 + mb) * nbk + kb) * 1024 + tid + 256 * i];
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) xs[mb * 1024 + tid + 256 * i] = stage[mb][i];
    };
    uint2 pc[NT][4][2];
    v4u hd[NT];
    auto load_w = [&](int kb) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const v4u q = qtile[t][((size_t)kb * 4 + c4) * 64];
                pc[t][c4][0] = make_uint2(q.x, q.y);
                pc[t][c4][1] = make_uint2(q.z, q.w);
            }
            hd[t] = htile[t][(size_t)kb * 32];
        }
    };
    f16v acc[NT][MB];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f16v{};
    load_stage(0);
    load_w(0);
    store_stage();
    __syncthreads();
    for (int kb = 0; kb < nbk; ++kb) {
        uint2 pcc[NT][4][2];
        v4u hdc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            hdc[t] = hd[t];
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                pcc[t][c4][0] = pc[t][c4][0];
                pcc[t][c4][1] = pc[t][c4][1];
            }
        }
        if (kb + 1 < nbk) {
            load_stage(kb + 1);
            load_w(kb + 1);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float d = f16_to_f32((uint16_t)(hdc[t].x & 0xffffu));
            const float dmin = f16_to_f32((uint16_t)(hdc[t].x >> 16));
            h2v sc2[8], nm2[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                uint32_t sc, mn;
                q4k_dev_scale_min(hdc[t], g, sc, mn);
                const _Float16 sh = (_Float16)(d * (float)sc), mh = (_Float16)(dmin * (float)mn);
                sc2[g] = h2v{sh, sh};
                nm2[g] = h2v{-mh, -mh};
            }
            const h2v bias = h2v{(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
            for (int st = 0; st < 16; ++st) {
                const int g = st >> 1, nib = (st >> 1) & 1;
                const uint2 pw = pcc[t][st >> 2][st & 1];
                const uint32_t w0 = (nib ? (pw.x >> 4) : pw.x) & 0x0f0f0f0fu;
                const uint32_t w1 = (nib ? (pw.y >> 4) : pw.y) & 0x0f0f0f0fu;
                const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
                const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
                const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
                const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
                const h2v e0 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p0) - bias, sc2[g], nm2[g]);
                const h2v e1 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p1) - bias, sc2[g], nm2[g]);
                const h2v e2 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p2) - bias, sc2[g], nm2[g]);
                const h2v e3 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p3) - bias, sc2[g], nm2[g]);
                h8v wb = h8v{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
                if (!nv[t]) wb = h8v{};
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[t][mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xs[mb * 1024 + st * 64 + lane], wb, acc[t][mb],
                                                                         0, 0, 0);
            }
        }
        __syncthreads();  // every wave is done with this K block's tiles
        if (kb + 1 < nbk) {
            store_stage();
            __syncthreads();
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int mrow0 = (mblk0 + mb) * 32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mrow0 + (r & 3) + 8 * (r >> 2) + 4 * hsel;
            if (EPI == EPI_GLU) {
                if (nv[1]) {
                    const int j = nbase[0] + r32, nbk2 = (N >> 1) >> 8;
                    const size_t at = ((((size_t)(m >> 5) * nbk2 + (j >> 8)) * 16 + ((j & 255) >> 4)) * 64 +
                                       ((j & 15) >> 3) * 32 + (m & 31)) * 8 + (j & 7);
                    ((_Float16*)a.xh_out)[at] = (_Float16)(m < a.M ? acc[1][mb][r] * ggml_silu(acc[0][mb][r]) : 0.0f);
                }
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (nv[t] && m < a.M) epilogue(a, m, nbase[t] + r32, acc[t][mb][r], EPI);
            }
        }
    }
}

size_t batched_scratch_bytes(size_t M, size_t K) { return ((M + 31) / 32) * 32 * K * 2; }

int batched_splits(size_t N, size_t K) {
    // few 32-row tiles leave most CUs idle: split K over workgroups of 4
    // waves, one block per wave
    const size_t tiles = (N + 31) / 32, nbk = K / 256;
    if (tiles >= 128 || nbk < 8) return 1;
    return (int)std::min<size_t>(8, nbk / 4);
}

// Grid (tiles, K/256), 256 threads: Q4_K payload and headers of 32-row tile
// `tile`, block kb, into the MFMA operand order: thread (c4, lane) writes
// the 16 bytes lane l uses for pieces (c4, 0) and (c4, 1), the 8 bytes at
// 32*c4 + 8*(l/32) and 32*c4 + 16 + 8*(l/32) of row 32*tile + l%32; rows
// past N are zero (d = dmin = 0, so they dequantize to 0).
__global__ __launch_bounds__(256) void mfma_tile_q4k_kernel(const uint8_t* __restrict__ qs, const v4u* __restrict__ hdr,
                                                            int N, int K, v4u* __restrict__ qs_t,
                                                            v4u* __restrict__ hdr_t) {
    const int tile = blockIdx.x, kb = blockIdx.y, nbk = K >> 8;
    const int tid = threadIdx.x, c4 = tid >> 6, lane = tid & 63;
    const int row = tile * 32 + (lane & 31), hsel = lane >> 5;
    v4u out = v4u{0u, 0u, 0u, 0u};
    if (row < N) {
        const uint8_t* b = qs + (size_t)row * (K >> 1) + (size_t)kb * 128 + 32 * c4 + 8 * hsel;
        const uint2 p0 = *(const uint2*)b, p1 = *(const uint2*)(b + 16);
        out = v4u{p0.x, p0.y, p1.x, p1.y};
    }
    qs_t[(((size_t)tile * nbk + kb) * 4 + c4) * 64 + lane] = out;
    if (tid < 32) {
        const int r = tile * 32 + tid;
        hdr_t[((size_t)tile * nbk + kb) * 32 + tid] = r < N ? hdr[(size_t)r * nbk + kb] : v4u{0u, 0u, 0u, 0u};
    }
}

hipError_t ensure_mfma_tiles(DeviceWeight& w, hipStream_t s) {
    if (w.type != kQ4_K || w.K % 256 || w.N == 0) return hipErrorInvalidValue;
    if (w.qs_t) return hipSuccess;
    const size_t tiles = (w.N + 31) / 32, nbk = w.K / 256;
    void *q = nullptr, *h = nullptr;
    hipError_t e = hipMalloc(&q, tiles * nbk * 4096);
    if (e == hipSuccess) e = hipMalloc(&h, tiles * nbk * 512);
    if (e != hipSuccess) {
        if (q) (void)hipFree(q);
        return e;
    }
    hipLaunchKernelGGL(mfma_tile_q4k_kernel, dim3((unsigned)tiles, (unsigned)nbk), dim3(256), 0, s,
                       (const uint8_t*)w.qs, (const v4u*)w.hdr, (int)w.N, (int)w.K, (v4u*)q, (v4u*)h);
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(q);
        (void)hipFree(h);
        return e;
    }
    w.qs_t = q;
    w.hdr_t = h;
    return hipSuccess;
}

template <int PRO>
static void launch_act16(const FusedGemvArgs& a, int mpad, _Float16* xh, hipStream_t s) {
    if (a.K <= 1024) hipLaunchKernelGGL((act16_kernel<PRO, 1>), dim3(mpad), dim3(256), 0, s, a, xh);
    else if (a.K <= 2048) hipLaunchKernelGGL((act16_kernel<PRO, 2>), dim3(mpad), dim3(256), 0, s, a, xh);
    else if (a.K <= 4096) hipLaunchKernelGGL((act16_kernel<PRO, 4>), dim3(mpad), dim3(256), 0, s, a, xh);
    else hipLaunchKernelGGL((act16_kernel<PRO, 8>), dim3(mpad), dim3(256), 0, s, a, xh);
}

// up * silu(gate) of the library gate/up GEMM's f16 rows [M][2F] (gate
// columns first), rounded to f16 row-major [M][F]: the down GEMM's operand
// (the EPI_GLU epilogue's arithmetic on f16-rounded gate and up)
__global__ void glu16_kernel(const _Float16* __restrict__ gu, size_t M, size_t F, _Float16* __restrict__ out) {
    typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i >= M * F) return;
    const size_t m = i / F, j = i % F;
    const h8v_t g = *(const h8v_t*)(gu + m * 2 * F + j);
    const h8v_t u = *(const h8v_t*)(gu + m * 2 * F + F + j);
    h8v_t o;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = (_Float16)((float)u[t] * ggml_silu((float)g[t]));
    *(h8v_t*)(out + i) = o;
}

// Prompt-sized M with the f16 weight present: hipBLASLt on row-major f16
// activations (the activation kernel's values in row order, or the previous
// gate/up GEMM's product), f32 accumulation; EPI_RESID adds into y (beta 1).
static hipError_t blas_batched(const DeviceWeight& w, FusedGemvArgs a, void* scratch, hipStream_t s) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const int mpad = (a.M + 31) / 32 * 32;
    const _Float16* xh = (const _Float16*)a.xh_in;
    if (!xh) {
        a.xh_rows = 1;
        switch (a.pro) {
        case PRO_RMS: launch_act16<PRO_RMS>(a, mpad, (_Float16*)scratch, s); break;
        case PRO_GATED: launch_act16<PRO_GATED>(a, mpad, (_Float16*)scratch, s); break;
        case PRO_SILU_MUL: launch_act16<PRO_SILU_MUL>(a, mpad, (_Float16*)scratch, s); break;
        case PRO_PLAIN: launch_act16<PRO_PLAIN>(a, mpad, (_Float16*)scratch, s); break;
        default: return hipErrorInvalidValue;
        }
        xh = (const _Float16*)scratch;
    }
    if (a.epi == EPI_GLU) {
        if (!a.xh_out || a.N % 16) return hipErrorInvalidValue;
        e = blas_gemm_f16(dev, a.M, a.N, a.K, xh, w.w16, a.y, false, (size_t)a.N, 0.0f, s);
        if (e != hipSuccess) return e;
        const size_t F = (size_t)a.N / 2, n8 = (size_t)a.M * F / 8;
        hipLaunchKernelGGL(glu16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, (const _Float16*)a.y,
                           (size_t)a.M, F, (_Float16*)a.xh_out);
        return hipGetLastError();
    }
    return blas_gemm_f16(dev, a.M, a.N, a.K, xh, w.w16, a.y, true, a.ldy, a.epi == EPI_RESID ? 1.0f : 0.0f, s);
}

hipError_t batched_gemv(const DeviceWeight& w, const FusedGemvArgs& args, void* scratch, hipStream_t s) {
    if (w.type != kQ4_K || w.K % 256 || w.K > 8192 || args.M <= 0 || args.M > 65535 * 32) return hipErrorInvalidValue;
    if (args.pro == PRO_GATED && args.group != 128) return hipErrorInvalidValue;
    if (w.w16 && args.M >= kBlasRows && !(args.epi == EPI_RESID && args.splits > 1 && args.parts)) {
        FusedGemvArgs a = args;
        a.K = (int)w.K;
        a.N = (int)w.N;
        return blas_batched(w, a, scratch, s);
    }
    if (!w.qs_t || !w.hdr_t) return hipErrorNotReady;  // ensure_mfma_tiles first
    FusedGemvArgs a = args;
    a.qs = w.qs_t;
    a.hdr = w.hdr_t;
    a.K = (int)w.K;
    a.N = (int)w.N;
    const int mpad = (a.M + 31) / 32 * 32;
    _Float16* xh = (_Float16*)scratch;
    if (a.xh_in) {
        xh = (_Float16*)a.xh_in;  // prepared by the previous GEMM's EPI_GLU
    } else {
        switch (a.pro) {
        case PRO_RMS: launch_act16<PRO_RMS>(a, mpad, xh, s); break;
        case PRO_GATED: launch_act16<PRO_GATED>(a, mpad, xh, s); break;
        case PRO_SILU_MUL: launch_act16<PRO_SILU_MUL>(a, mpad, xh, s); break;
        case PRO_PLAIN: launch_act16<PRO_PLAIN>(a, mpad, xh, s); break;
        default: return hipErrorInvalidValue;
        }
    }
    // prompt-sized M (>= 1024 rows; below, the K-split kernel keeps more
    // workgroups busy): the LDS-staged variant, MB activation blocks per
    // workgroup (MB divides the block count)
    const int mblocks = mpad / 32;
    const bool no_split = !(a.epi == EPI_RESID && a.splits > 1 && a.parts);
    if (a.M >= 1024 && no_split) {
        const int mb = mblocks % 4 == 0 ? 4 : (mblocks % 2 == 0 ? 2 : 1);
        const int tiles = (a.N + 31) / 32;
        if (a.epi == EPI_GLU) {
            if (!batched_glu_supported(w.type, w.K, w.N) || !a.xh_out) return hipErrorInvalidValue;
            dim3 g((unsigned)((a.N / 64 + 3) / 4), (unsigned)(mblocks / mb), 1u);
            if (mb == 4) hipLaunchKernelGGL((mfma_q4k_wide_kernel<EPI_GLU, 2, 4>), g, dim3(256), 0, s, a, (const _Float16*)xh);
            else if (mb == 2) hipLaunchKernelGGL((mfma_q4k_wide_kernel<EPI_GLU, 2, 2>), g, dim3(256), 0, s, a, (const _Float16*)xh);
            else hipLaunchKernelGGL((mfma_q4k_wide_kernel<EPI_GLU, 2, 1>), g, dim3(256), 0, s, a, (const _Float16*)xh);
            return hipGetLastError();
        }
        // one weight tile per wave (two per wave, which halves the LDS
        // traffic per MFMA, cost occupancy and measured 1-3% slower)
        dim3 g((unsigned)((tiles + 3) / 4), (unsigned)(mblocks / mb), 1u);
#define ZG_MW(E, MBV) hipLaunchKernelGGL((mfma_q4k_wide_kernel<E, 1, MBV>), g, dim3(256), 0, s, a, (const _Float16*)xh)
#define ZG_MWE(E)                 \
    if (mb == 4) ZG_MW(E, 4);      \
    else if (mb == 2) ZG_MW(E, 2); \
    else ZG_MW(E, 1);
        if (a.epi == EPI_RESID) {
            ZG_MWE(EPI_RESID)
        } else {
            ZG_MWE(EPI_STORE)
        }
#undef ZG_MWE
#undef ZG_MW
        return hipGetLastError();
    }
    if (a.epi == EPI_GLU) {
        if (!batched_glu_supported(w.type, w.K, w.N) || !a.xh_out) return hipErrorInvalidValue;
        dim3 g((unsigned)(a.N / 64), (unsigned)(mpad / 32), 1u);
        if (a.N / 64 >= 512) hipLaunchKernelGGL((mfma_q4k_kernel<EPI_GLU, 4, 2>), g, dim3(256), 0, s, a, (const _Float16*)xh);
        else hipLaunchKernelGGL((mfma_q4k_kernel<EPI_GLU, 8, 2>), g, dim3(512), 0, s, a, (const _Float16*)xh);
        return hipGetLastError();
    }
    // NT tiles of 32 weight rows per workgroup (each activation load feeds
    // NT MFMAs) while that still leaves >= 192 workgroups; K split over 8
    // waves when the workgroups are few, else over 4
    const int tiles = (a.N + 31) / 32;
    const int nt = tiles / 4 >= 192 ? 4 : (tiles / 2 >= 192 ? 2 : 1);
    const int splits = a.epi == EPI_RESID && a.splits > 1 && a.parts ? a.splits : 1;
    dim3 g((unsigned)((tiles + nt - 1) / nt), (unsigned)(mpad / 32), (unsigned)splits);
    const bool wide = (tiles + nt - 1) / nt >= 512 || splits > 1;
#define ZG_MQ(E, KSV, NTV) hipLaunchKernelGGL((mfma_q4k_kernel<E, KSV, NTV>), g, dim3(64 * KSV), 0, s, a, (const _Float16*)xh)
#define ZG_MQN(E, KSV)            \
    if (nt == 4) ZG_MQ(E, KSV, 4);      \
    else if (nt == 2) ZG_MQ(E, KSV, 2); \
    else ZG_MQ(E, KSV, 1);
    if (a.epi == EPI_RESID) {
        if (wide) {
            ZG_MQN(EPI_RESID, 4)
        } else {
            ZG_MQN(EPI_RESID, 8)
        }
    } else {
        if (wide) {
            ZG_MQN(EPI_STORE, 4)
        } else {
            ZG_MQN(EPI_STORE, 8)
        }
    }
#undef ZG_MQN
#undef ZG_MQ
    return hipGetLastError();
}

// ============================================================ dispatch

// ====================================================== Q4_1, Q6_K, F32

// Q4_1 x Q8_1 (cpu/src/source/quantization.rs:198-227): lane l of a row's 8
// lanes takes elements 4l..4l+3 of every block, lane = fma(int dot,
// d_w * d_a, lane); the zero points accumulate apart (summs = summs +
// m_w * s_a) and join after the reference's lane tree.
template <int MT, int J, int PRO, int EPI>
__global__ __launch_bounds__(256) void fused_q41_kernel(FusedGemvArgs a) {
    // 8-block chunks stream QC at a time through two register buffers, the
    // next group's loads issued before the current one is consumed;
    // activation row 0's loads go out first and its coding overlaps them (a
    // wave's loads complete in issue order).  Loads are unconditional: a
    // chunk past the row end reads the last one and is not consumed.
    constexpr int QC = 4;
    extern __shared__ int lds_f41[];
    const int K = a.K, N = a.N;
    const int nb = K >> 5, nbc8 = (nb + 7) >> 3, nb8 = nbc8 * 8;
    int* codes = lds_f41;                                // [MT][8][nb8] words
    float* scales = (float*)(lds_f41 + MT * 8 * nb8);    // [MT][nb8]
    float* sums = scales + MT * nb8;                     // [MT][nb8]
    const int m0 = blockIdx.y * MT;
    const v4i* qs = (const v4i*)a.qs;
    const uint32_t* hdr = (const uint32_t*)a.hdr;
    const int lane = threadIdx.x & 63;
    const int rl = lane >> 3, l = lane & 7;
    const int groups = (N + 7) >> 3;
    const int nwaves = gridDim.x * 4;
    struct Chunk {
        v4i w[QC];
        v4u h0[QC], h1[QC];
    };
    auto load_chunk = [&](int R, int c0, Chunk& ck) {
        const int Rc = min(R, groups - 1);
        const uint32_t* hrow = hdr + (size_t)min(Rc * 8 + rl, N - 1) * nbc8 * 8;
        const v4i* tile = qs + (size_t)Rc * nbc8 * 64 + lane;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const int c = min(c0 + i, nbc8 - 1);
            ck.w[i] = load_nt(tile + (size_t)c * 64);
            ck.h0[i] = *(const v4u*)(hrow + 8 * c);
            ck.h1[i] = *(const v4u*)(hrow + 8 * c + 4);
        }
    };
    float acc[MT], summs[MT];
    auto consume = [&](const Chunk& ck, int c0) {
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const int c = c0 + i;
            if (c >= nbc8) break;  // uniform
            const uint32_t ww[4] = {(uint32_t)ck.w[i].x, (uint32_t)ck.w[i].y, (uint32_t)ck.w[i].z,
                                    (uint32_t)ck.w[i].w};
            const uint32_t hw[8] = {ck.h0[i].x, ck.h0[i].y, ck.h0[i].z, ck.h0[i].w,
                                    ck.h1[i].x, ck.h1[i].y, ck.h1[i].z, ck.h1[i].w};
            int xc[MT][8];
            float xs[MT][8], xu[MT][8];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const v4i* cp = (const v4i*)(codes + (size_t)(m * 8 + l) * nb8 + 8 * c);
                const v4f* sp = (const v4f*)(scales + (size_t)m * nb8 + 8 * c);
                const v4f* up = (const v4f*)(sums + (size_t)m * nb8 + 8 * c);
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const v4i cv = cp[hh];
                    const v4f sv = sp[hh], uv = up[hh];
                    xc[m][4 * hh] = cv.x; xc[m][4 * hh + 1] = cv.y; xc[m][4 * hh + 2] = cv.z; xc[m][4 * hh + 3] = cv.w;
                    xs[m][4 * hh] = sv.x; xs[m][4 * hh + 1] = sv.y; xs[m][4 * hh + 2] = sv.z; xs[m][4 * hh + 3] = sv.w;
                    xu[m][4 * hh] = uv.x; xu[m][4 * hh + 1] = uv.y; xu[m][4 * hh + 2] = uv.z; xu[m][4 * hh + 3] = uv.w;
                }
            }
#pragma unroll
            for (int bi = 0; bi < 8; ++bi) {
                const int b = 8 * c + bi;
                if (b < nb) {
                    const uint32_t q = (ww[bi >> 1] >> (16 * (bi & 1))) & 0xffffu;
                    const int w8 = (int)((q & 0xfu) | ((q & 0xf0u) << 4) | ((q & 0xf00u) << 8) | ((q & 0xf000u) << 12));
                    const float d0 = f16_to_f32((uint16_t)(hw[bi] & 0xffffu));
                    const float mw = f16_to_f32((uint16_t)(hw[bi] >> 16));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const int partial = __builtin_amdgcn_sdot4(w8, xc[m][bi], 0, false);
                        const float ms = mw * xu[m][bi];
                        summs[m] = summs[m] + ms;
                        const float scale = d0 * xs[m][bi];
                        acc[m] = fmaf((float)partial, scale, acc[m]);
                    }
                }
            }
        }
    };
    ProIn<J> pin;
    wg_prologue_load<PRO, J>(a, m0, m0 < a.M, pin);
    const int R0 = blockIdx.x * 4 + (threadIdx.x >> 6);
    Chunk ca, cb;
    load_chunk(R0, 0, ca);
    wg_prologue_code<PRO, kCodecQ81, J>(a, m0 < a.M, pin, nullptr, codes, scales, sums);
#pragma unroll
    for (int m = 1; m < MT; ++m)
        wg_prologue<PRO, kCodecQ81, J>(a, m0 + m, m0 + m < a.M, nullptr, codes + (size_t)m * 8 * nb8,
                                       scales + (size_t)m * nb8, sums + (size_t)m * nb8);
    for (int R = R0; R < groups; R += nwaves) {
        if (R != R0) load_chunk(R, 0, ca);
        const int row = R * 8 + rl;
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = summs[m] = 0.0f;
        for (int c0 = 0; c0 < nbc8; c0 += 2 * QC) {
            if (c0 + QC < nbc8) load_chunk(R, c0 + QC, cb);
            consume(ca, c0);
            if (c0 + QC >= nbc8) break;
            if (c0 + 2 * QC < nbc8) load_chunk(R, c0 + 2 * QC, ca);
            consume(cb, c0 + QC);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = group8_tree_last(acc[m]);
        if (row < N && l == 7) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m0 + m < a.M) epilogue(a, m0 + m, row, acc[m] + summs[m], EPI);
        }
    }
}

__device__ __forceinline__ int sbyte(const v4u& v, int idx) {
    const int q = idx >> 2;
    const uint32_t d = q == 0 ? v.x : (q == 1 ? v.y : (q == 2 ? v.z : v.w));
    return (int)(int8_t)(d >> (8 * (idx & 3)));
}

// Q6_K x Q8_K (quantization.rs:228-285): lane L of a row's 8 lanes holds
// every element at position 4L..4L+3 of its 32-group.  Per superblock its
// int32 sum is sum(code * local scale * q8) (4-element dot products, one
// local scale each) minus 32 * (bsum * scale) over the contiguous 16-groups
// 2L and 2L+1; lane = fma((float)int, d_a * d_w, lane); the Q8_0 lane tree.
template <int MT, int J, int PRO, int EPI>
__global__ __launch_bounds__(256) void fused_q6k_kernel(FusedGemvArgs a) {
    // superblocks stream in chunks of QS through two register buffers, the
    // next chunk's loads issued before the current one is consumed;
    // activation row 0's loads go out first and its coding overlaps the
    // first chunk's (a wave's loads complete in issue order).  Loads are
    // unconditional: a superblock past the row end reads the last one and
    // is not consumed.
    constexpr int QS = 4;
    extern __shared__ int lds_f6[];
    const int K = a.K, N = a.N, nsb = K >> 8;
    int* codes = lds_f6;                                 // [MT][K/4] words
    float* dk = (float*)(lds_f6 + MT * (K >> 2));        // [MT][nsb]
    int* bs = (int*)(dk + MT * nsb);                     // [MT][K/16]
    const int m0 = blockIdx.y * MT;
    const uint32_t* qa = (const uint32_t*)a.qs;
    const uint32_t* qb = qa + q6k_b_offset((size_t)N, (size_t)K);
    const uint8_t* scl = (const uint8_t*)a.hdr;
    const float* dw = (const float*)(scl + (size_t)N * nsb * 16);
    const int lane = threadIdx.x & 63;
    const int rl = lane >> 3, l = lane & 7;
    const int groups = (N + 7) >> 3;
    const int nwaves = gridDim.x * 4;
    struct Chunk {
        v4u A[QS], S[QS];
        uint2 B[QS];
        float wd[QS];
    };
    auto load_chunk = [&](int R, int sb0, Chunk& ck) {
        const int row = min(R, groups - 1) * 8 + rl;  // tile rows past N exist (8-row tiles)
        const size_t rr = (size_t)min(row, N - 1);
#pragma unroll
        for (int i = 0; i < QS; ++i) {
            const int sb = min(sb0 + i, nsb - 1);
            ck.A[i] = *(const v4u*)(qa + q6k_a_index((size_t)row, (size_t)sb, l, (size_t)nsb));
            ck.B[i] = *(const uint2*)(qb + q6k_b_index((size_t)row, (size_t)sb, l, (size_t)nsb));
            ck.S[i] = *(const v4u*)(scl + (rr * nsb + sb) * 16);
            ck.wd[i] = dw[rr * nsb + sb];
        }
    };
    float acc[MT];
    auto consume = [&](const Chunk& ck, int sb0) {
#pragma unroll
        for (int i = 0; i < QS; ++i) {
            const int sb = sb0 + i;
            if (sb >= nsb) break;  // uniform
            const uint32_t av[4] = {ck.A[i].x, ck.A[i].y, ck.A[i].z, ck.A[i].w};
            const uint32_t bv[2] = {ck.B[i].x, ck.B[i].y};
            int code4[2][4], sub[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t nib = (av[h * 2 + (g & 1)] >> (g >= 2 ? 4 : 0)) & 0x0f0f0f0fu;
                    const uint32_t hi = ((bv[h] >> (2 * g)) & 0x03030303u) << 4;
                    code4[h][g] = (int)(nib | hi);
                    sub[h][g] = sbyte(ck.S[i], h * 8 + g * 2 + (l >> 2));
                }
            const int so0 = sbyte(ck.S[i], 2 * l), so1 = sbyte(ck.S[i], 2 * l + 1);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int* cl = codes + m * (K >> 2) + (size_t)l * (K >> 5) + sb * 8;
                const v4i c0 = *(const v4i*)cl, c1 = *(const v4i*)(cl + 4);
                const int cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                int iacc = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        iacc += sub[h][g] * __builtin_amdgcn_sdot4(code4[h][g], cw[h * 4 + g], 0, false);
                const int* bm = bs + m * (K >> 4) + sb * 16;
                iacc -= 32 * (bm[2 * l] * so0 + bm[2 * l + 1] * so1);
                const float scale = dk[m * nsb + sb] * ck.wd[i];
                acc[m] = fmaf((float)iacc, scale, acc[m]);
            }
        }
    };
    ProIn<J> pin;
    wg_prologue_load<PRO, J>(a, m0, m0 < a.M, pin);
    const int R0 = blockIdx.x * 4 + (threadIdx.x >> 6);
    Chunk ca, cb;
    load_chunk(R0, 0, ca);
    wg_prologue_code<PRO, kCodecQ8K, J>(a, m0 < a.M, pin, nullptr, codes, nullptr, dk, bs);
#pragma unroll
    for (int m = 1; m < MT; ++m)
        wg_prologue<PRO, kCodecQ8K, J>(a, m0 + m, m0 + m < a.M, nullptr, codes + m * (K >> 2), nullptr,
                                       dk + m * nsb, bs + m * (K >> 4));
    for (int R = R0; R < groups; R += nwaves) {
        if (R != R0) load_chunk(R, 0, ca);
        const int row = R * 8 + rl;
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int sb0 = 0; sb0 < nsb; sb0 += 2 * QS) {
            if (sb0 + QS < nsb) load_chunk(R, sb0 + QS, cb);
            consume(ca, sb0);
            if (sb0 + QS >= nsb) break;
            if (sb0 + 2 * QS < nsb) load_chunk(R, sb0 + 2 * QS, ca);
            consume(cb, sb0 + QS);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = group8_tree_last(acc[m]);
        if (row < N && l == 7) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m0 + m < a.M) epilogue(a, m0 + m, row, acc[m], EPI);
        }
    }
}

// F32 rows (cpu/src/source.rs:325-366): 32 lanes per row, lane t holds the
// accumulator of positions t mod 32 (the reference's accum[t / 8][t % 8]),
// fma over the 32-element steps in order; the tree (a[t] + a[t+16]) +
// (a[t+8] + a[t+24]), then lanes t, t+4, then (h0 + h1) + (h2 + h3) is the
// XOR tree 16, 8, 4, 1, 2; the tail past the last full step is added
// serially (product, then sum).
template <int MT, int J, int PRO, int EPI>
__global__ __launch_bounds__(256) void fused_f32_kernel(FusedGemvArgs a) {
    extern __shared__ int lds_ff[];
    const int K = a.K, N = a.N;
    float* xs = (float*)lds_ff;  // [MT][K]
    const int m0 = blockIdx.y * MT;
#pragma unroll
    for (int m = 0; m < MT; ++m)
        wg_prologue<PRO, kCodecF32, J>(a, m0 + m, m0 + m < a.M, nullptr, (int*)(xs + (size_t)m * K), nullptr);
    const float* W = (const float*)a.qs;
    const int lane = threadIdx.x & 63, t = lane & 31;
    const int np = K & ~31;
    const int pairs = (N + 1) >> 1;
    const int nwaves = gridDim.x * 4;
    for (int P = blockIdx.x * 4 + (threadIdx.x >> 6); P < pairs; P += nwaves) {
        const int row = P * 2 + (lane >> 5);
        const size_t rr = (size_t)(row < N ? row : N - 1);
        const float* wr = W + rr * K;
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int base = 0; base < np; base += 32) {
            const float w = wr[base + t];
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[m] = fmaf(w, xs[(size_t)m * K + base + t], acc[m]);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[m];
            v = v + __shfl_xor(v, 16, 64);
            v = v + __shfl_xor(v, 8, 64);
            v = v + __shfl_xor(v, 4, 64);
            v = v + __shfl_xor(v, 1, 64);
            v = v + __shfl_xor(v, 2, 64);
            acc[m] = v;
        }
        if (row < N && t == 0) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m0 + m >= a.M) continue;
                float r = acc[m];
                for (int i = np; i < K; ++i) {
                    const float p = wr[i] * xs[(size_t)m * K + i];
                    r = r + p;
                }
                epilogue(a, m0 + m, row, r, EPI);
            }
        }
    }
}

template <int PRO, int EPI>
static hipError_t launch_codec(const FusedGemvArgs& a, int type, hipStream_t s) {
    const int K = a.K;
    const int mt = type == kF32 ? 1 : (a.M == 1 ? 1 : (a.M == 2 ? 2 : 4));
    size_t per;
    if (type == kQ4_1) per = (size_t)((K / 32 + 7) / 8 * 8) * 40;  // codes 8 words + scale + sum per block
    else if (type == kQ6_K) per = (size_t)K + (size_t)(K / 256) * 4 + (size_t)(K / 16) * 4;
    else per = (size_t)K * 4;
    const size_t lds = per * mt;
    const size_t units = type == kF32 ? ((size_t)a.N + 1) / 2 : ((size_t)a.N + 7) / 8;
    const unsigned wgs = (unsigned)std::min<size_t>((units + 3) / 4, 256 * 8);
    dim3 g(wgs, (unsigned)((a.M + mt - 1) / mt));
#define ZG_FC(KER, T, JJ) hipLaunchKernelGGL((KER<T, JJ, PRO, EPI>), g, dim3(256), lds, s, a)
#define ZG_FCJ(KER, JJ)                 \
    if (mt == 1) ZG_FC(KER, 1, JJ);      \
    else if (mt == 2) ZG_FC(KER, 2, JJ); \
    else ZG_FC(KER, 4, JJ);
#define ZG_FCK(KER)          \
    if (K <= 1024) {         \
        ZG_FCJ(KER, 1)       \
    } else if (K <= 2048) {  \
        ZG_FCJ(KER, 2)       \
    } else if (K <= 4096) {  \
        ZG_FCJ(KER, 4)       \
    } else {                 \
        ZG_FCJ(KER, 8)       \
    }
    if (type == kQ4_1) {
        ZG_FCK(fused_q41_kernel)
    } else if (type == kQ6_K) {
        ZG_FCK(fused_q6k_kernel)
    } else {
        ZG_FCK(fused_f32_kernel)
    }
#undef ZG_FCK
#undef ZG_FCJ
#undef ZG_FC
    return hipGetLastError();
}

template <int PRO, int EPI>
static hipError_t launch_q4k(const FusedGemvArgs& a, hipStream_t s) {
    // lpr = 2^l lanes per row, ch 64-element chunks per lane: the pair with
    // the fewest idle chunk slots (ch * lpr - nchunk), fewer chunks per lane
    // on a tie (K = 6144: 32 lanes x 3 chunks, not 64 x 2 with a quarter
    // idle); activation slabs J = ceil(K / 1024) rounded to 2, 4, 8
    const int nchunk = a.K / 64;
    int l = -1, ch = 0;
    for (int t = 6; t >= 2; --t) {
        const int c = (nchunk + (1 << t) - 1) >> t;
        if (c > 3) break;
        if (l < 0 || c * (1 << t) - nchunk < ch * (1 << l) - nchunk) {
            l = t;
            ch = c;
        }
    }
    if (l < 0 || a.K > 8192) return hipErrorInvalidValue;
    int mt = a.M == 1 ? 1 : (a.M == 2 ? 2 : 4);
    while (mt > 1 && ch * mt > 4) mt >>= 1;
    // B=1: up to 4 row groups per wave so that ~4096 waves cover the matrix
    // (fewer workgroups repeating the prologue, more loads in flight per
    // wave; measured best against ~2048 waves and one group per wave)
    const size_t rpw = 64u >> l, groups = (a.N + rpw - 1) / rpw;
    int rg = 1;
    if (mt == 1) {
        while (rg < 4 && groups > (size_t)4096 * rg) rg *= 2;
    }
    const size_t waves = (groups + rg - 1) / rg;
    const unsigned wgs = (unsigned)std::min<size_t>((waves + 3) / 4, 256 * 8);
    dim3 g(wgs, (unsigned)((a.M + mt - 1) / mt));
    const size_t lds = (size_t)mt * nchunk * kRecWords * 4;
#define ZG_F4(C, T, JJ, R) hipLaunchKernelGGL((fused_q4k_kernel<C, T, JJ, R, PRO, EPI>), g, dim3(256), lds, s, a, l)
#define ZG_F4R(C, JJ)                \
    if (rg == 1) ZG_F4(C, 1, JJ, 1);      \
    else if (rg == 2) ZG_F4(C, 1, JJ, 2); \
    else ZG_F4(C, 1, JJ, 4);
    if (ch == 3) {
        if (a.K <= 4096) {
            ZG_F4R(3, 4)
        } else {
            ZG_F4R(3, 8)
        }
    } else if (ch == 2) {
        if (mt == 1) {
            ZG_F4R(2, 8)
        } else {
            ZG_F4(2, 2, 8, 1);
        }
    } else if (a.K <= 2048) {
        if (mt == 1) {
            ZG_F4R(1, 2)
        } else if (mt == 2) {
            ZG_F4(1, 2, 2, 1);
        } else {
            ZG_F4(1, 4, 2, 1);
        }
    } else {
        if (mt == 1) {
            ZG_F4R(1, 4)
        } else if (mt == 2) {
            ZG_F4(1, 2, 4, 1);
        } else {
            ZG_F4(1, 4, 4, 1);
        }
    }
#undef ZG_F4R
#undef ZG_F4
    return hipGetLastError();
}

template <int PRO, int EPI>
static hipError_t launch_q8(const FusedGemvArgs& a, hipStream_t s) {
    const int K = a.K;
    int mt = a.M == 1 ? 1 : (a.M == 2 ? 2 : 4);
    auto lds = [&](int t) { return (size_t)t * ((K / 32 + 3) / 4 * 4) * 36; };  // codes 8 words + scale per block
    const size_t groups = (a.N + 7) / 8;
    const unsigned wgs = (unsigned)std::min<size_t>((groups + 3) / 4, 256 * 8);
    dim3 g(wgs, (unsigned)((a.M + mt - 1) / mt));
#define ZG_F8(T, JJ) hipLaunchKernelGGL((fused_q8_kernel<T, JJ, PRO, EPI>), g, dim3(256), lds(T), s, a)
#define ZG_F8J(JJ)                  \
    if (mt == 1) ZG_F8(1, JJ);      \
    else if (mt == 2) ZG_F8(2, JJ); \
    else ZG_F8(4, JJ);
    if (K <= 1024) {
        ZG_F8J(1)
    } else if (K <= 2048) {
        ZG_F8J(2)
    } else if (K <= 4096) {
        ZG_F8J(4)
    } else {
        ZG_F8J(8)
    }
#undef ZG_F8J
#undef ZG_F8
    return hipGetLastError();
}

template <int PRO>
static hipError_t launch_pro(const FusedGemvArgs& a, int type, hipStream_t s) {
    if (a.epi == EPI_GLU) {
        if constexpr (PRO == PRO_RMS) {
            if (type == kQ4_K) return launch_q4k<PRO_RMS, EPI_GLU>(a, s);
        }
        return hipErrorInvalidValue;
    }
    if (type == kQ4_K) return a.epi == EPI_RESID ? launch_q4k<PRO, EPI_RESID>(a, s) : launch_q4k<PRO, EPI_STORE>(a, s);
    if (type == kQ8_0) return a.epi == EPI_RESID ? launch_q8<PRO, EPI_RESID>(a, s) : launch_q8<PRO, EPI_STORE>(a, s);
    if (type == kQ4_1 || type == kQ6_K || type == kF32)
        return a.epi == EPI_RESID ? launch_codec<PRO, EPI_RESID>(a, type, s) : launch_codec<PRO, EPI_STORE>(a, type, s);
    return hipErrorInvalidValue;
}

bool fused_glu_supported(int type, size_t K, size_t N) {
    // a row group must hold whole (gate, up) pairs: 64 lanes over <= 32
    // lanes per row (K <= 2048), rpw even
    return type == kQ4_K && K % 256 == 0 && K <= 2048 && N % 2 == 0 && N > 0;
}

bool batched_glu_supported(int type, size_t K, size_t N) {
    return type == kQ4_K && K % 256 == 0 && K <= 8192 && N % 64 == 0 && (N / 2) % 256 == 0;
}

bool fused_gemv_supported(int type, size_t K, size_t N, int pro) {
    if (N == 0 || K == 0 || N > (1u << 30)) return false;
    if (pro == PRO_GATED && (K % 128 || K / 128 > 256 || 256 % (K / 128))) return false;
    if (K > 8192) return false;  // prologue slabs
    if (type == kQ4_K || type == kQ6_K) return K % 256 == 0;
    if (type == kQ8_0 || type == kQ4_1) return K % 32 == 0;
    if (type == kF32) return K % 4 == 0;
    return false;
}

hipError_t fused_gemv(const DeviceWeight& w, const FusedGemvArgs& args, hipStream_t s) {
    if (!fused_gemv_supported(w.type, w.K, w.N, args.pro) || args.M <= 0) return hipErrorInvalidValue;
    if (args.pro == PRO_GATED && args.group != 128) return hipErrorInvalidValue;  // 32 lanes x 4 per group
    if (args.epi == EPI_GLU && !fused_glu_supported(w.type, w.K, w.N)) return hipErrorInvalidValue;
    FusedGemvArgs a = args;
    a.qs = w.qs;
    a.hdr = w.hdr;
    a.K = (int)w.K;
    a.N = (int)w.N;
    switch (a.pro) {
    case PRO_RMS: return launch_pro<PRO_RMS>(a, w.type, s);
    case PRO_GATED: return launch_pro<PRO_GATED>(a, w.type, s);
    case PRO_SILU_MUL: return launch_pro<PRO_SILU_MUL>(a, w.type, s);
    case PRO_PLAIN: return launch_pro<PRO_PLAIN>(a, w.type, s);
    default: return hipErrorInvalidValue;
    }
}

// ============================================================ GDN decode

// Grid (H * 4, B), 256 threads: workgroup (h, quarter) owns value columns
// quarter*32 .. +31 of head h.  The causal conv keeps a 4-slot ring per
// channel: the token at position p is written to slot p%4 while the taps
// x[p-3], x[p-2], x[p-1] are read from the other three slots, so the
// workgroups of one head that all read the q/k channels never race with the
// one (quarter 0) that writes them.  conv: cpu/src/ops/gdn.rs:7-44 (left to
// right, no FMA) + SiLU (forward.rs:548); L2, gates and recurrence as
// gdn_recurrent_kernel<true>.
// HEAD: one workgroup of 4 x 256 threads per (head, row) -- quarter q is
// threads 256q.. -- sharing the conv, norms and gates, and finishing with
// the gated RMSNorm of the head's output into the next GEMM's f16 tiles.
template <bool HEAD>
__global__ __launch_bounds__(HEAD ? 1024 : 256) void gdn_decode_kernel(GdnDecodeArgs a) {
    constexpr int D = 128;
    __shared__ float qk[2 * D];
    __shared__ float vv[HEAD ? D : 32];
    __shared__ float gates[2];
    __shared__ float ob[HEAD ? D : 1];
    const int h = HEAD ? blockIdx.x : blockIdx.x >> 2, b = blockIdx.y;
    const int quarter = HEAD ? (int)(threadIdx.x >> 8) : (int)(blockIdx.x & 3);
    const int tid = threadIdx.x & 255;
    const int W = a.H * D;
    const int lane = tid & 63, wv = tid >> 6;
    const int jl = wv * 8 + (lane >> 3);  // column within the quarter
    const int j = quarter * 32 + jl;
    const int s = lane & 7;
    const float* xin = a.proj + (size_t)b * a.proj_stride;
    float* ring = a.ring + (size_t)b * 3 * W * 4;
    // The conv and gate inputs are requested first, then this thread's 16
    // state values (the bulk of the traffic): a wave's loads complete in
    // issue order, so the conv, norms and gates wait only for their own
    // inputs while the state is in flight.  HEAD: threads 0..255 own the q/k
    // channels and 256..383 the value channels, one each; else every thread
    // owns q/k channel tid and threads < 32 also value channel
    // quarter*32 + tid.  Loads are unconditional (clamped in range) and each
    // sum is used on two paths, so that none moves behind the state loads.
    struct ConvIn {
        v4f r, w;
        float x;
    };
    auto conv_load = [&](int ch) {
        ConvIn c;
        c.r = *(const v4f*)(ring + (size_t)ch * 4);
        c.w = *(const v4f*)(a.conv_w + (size_t)ch * 4);
        c.x = xin[ch];
        return c;
    };
    const int ch_qk = tid < D ? h * D + tid : W + h * D + (tid - D);
    const int vc = HEAD ? max(0, min((int)threadIdx.x - 256, D - 1)) : quarter * 32 + (tid & 31);
    const int ch_v = 2 * W + h * D + vc;
    const int ch_a = HEAD && threadIdx.x >= 256 ? ch_v : ch_qk;
    const ConvIn in_a = conv_load(ch_a);
    ConvIn in_v;
    if constexpr (!HEAD) in_v = conv_load(ch_v);
    const float g_a = xin[4 * W + h], g_b = xin[4 * W + a.H + h], g_dt = a.dt[h], g_sa = a.ssm_a[h];
    // HEAD: wave 0's gated-norm inputs, requested now so that the tail does
    // not wait for them (loads are not moved across the barriers below)
    v4f tail_g = v4f{0.0f, 0.0f, 0.0f, 0.0f}, tail_z = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (HEAD && threadIdx.x < 64) {
        const int t = threadIdx.x & 31;
        tail_g = *(const v4f*)(a.norm + 4 * t);
        tail_z = *(const v4f*)(xin + 3 * W + h * D + 4 * t);
    }
    float* col = a.state + (((size_t)b * a.H + h) * D + j) * D + 4 * s;
    v4f sv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) sv[c] = *(const v4f*)(col + 32 * c);
    const int p = a.pos[b];
    const int s0 = (p + 1) & 3, s1 = (p + 2) & 3, s2 = (p + 3) & 3, sw = p & 3;
    auto conv = [&](const ConvIn& c) {
        const float hv[4] = {c.r.x, c.r.y, c.r.z, c.r.w};
        const float t0 = hv[s0] * c.w.x;
        const float t1 = hv[s1] * c.w.y;
        const float t2 = hv[s2] * c.w.z;
        const float t3 = c.x * c.w.w;
        float acc = t0 + t1;
        acc = acc + t2;
        acc = acc + t3;
        return acc;
    };
    if constexpr (HEAD) {
        const float cv = conv(in_a);
        if (threadIdx.x < 256) {
            qk[threadIdx.x] = ggml_silu(cv);
            ring[(size_t)ch_qk * 4 + sw] = in_a.x;
        } else if (threadIdx.x < 256 + D) {
            vv[vc] = ggml_silu(cv);
            ring[(size_t)ch_v * 4 + sw] = in_a.x;
        }
    } else {
        qk[tid] = ggml_silu(conv(in_a));
        if (quarter == 0) ring[(size_t)ch_qk * 4 + sw] = in_a.x;
        if (tid < 32) {
            vv[tid] = ggml_silu(conv(in_v));
            ring[(size_t)ch_v * 4 + sw] = in_v.x;
        }
    }
    // the head's gates (f64-evaluated transcendentals) once per workgroup,
    // by the wave without value channels
    if (tid == 192 && (!HEAD || quarter == 0)) {
        float gn, bt, sp, gr;
        gdn_coef(g_a, g_b, g_dt, g_sa, gn, bt, sp, gr);
        gates[0] = gn;
        gates[1] = bt;
    }
    lds_barrier();  // the state loads stay in flight

    float q[4][4], k[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            q[c][t] = qk[32 * c + 4 * s + t];
            k[c][t] = qk[D + 32 * c + 4 * s + t];
        }
    // two-stage L2 (forward.rs:564-576)
    double sq = 0.0, sk = 0.0;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float a2 = q[c][t] * q[c][t];
            const float b2 = k[c][t] * k[c][t];
            sq += (double)a2;
            sk += (double)b2;
        }
    sq = group8_sum_all(sq);
    sk = group8_sum_all(sk);
    const float dsq = 1.0f / sqrtf((float)D);
    const float eps_d = a.eps / (float)D;
    const float iq = 1.0f / sqrtf((float)(sq / (double)D) + eps_d);
    const float ik = 1.0f / sqrtf((float)(sk / (double)D) + eps_d);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float tq = q[c][t] * iq;
            q[c][t] = tq * dsq;
            const float tk = k[c][t] * ik;
            k[c][t] = tk * dsq;
        }
    const float gain = gates[0], beta = gates[1];
    const float vj = vv[HEAD ? j : jl];
    float cv[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const v4f v = sv[c];
        cv[c][0] = v.x * gain; cv[c][1] = v.y * gain; cv[c][2] = v.z * gain; cv[c][3] = v.w * gain;
    }
    const float prev = column_dot(cv, k);
    const float delta = (vj - prev) * beta;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) cv[c][t] = fmaf(k[c][t], delta, cv[c][t]);
    const float o = column_dot(cv, q);
#pragma unroll
    for (int c = 0; c < 4; ++c) *(v4f*)(col + 32 * c) = v4f{cv[c][0], cv[c][1], cv[c][2], cv[c][3]};
    if (s == 0) a.core[(size_t)b * W + h * D + j] = o * a.scale;
    if constexpr (HEAD) {
        // gated RMSNorm of the head (forward.rs:586-594) in act16_kernel's
        // arithmetic: 32 lanes of wave 0, elements 4t..4t+3 each, f64 sum of
        // f32 squares over the group, then ((e * inv) * gamma) * silu(z)
        if (s == 0) ob[j] = o * a.scale;
        __syncthreads();
        if (threadIdx.x < 64) {  // the whole wave runs the 32-lane tree; lanes 32.. repeat the group
            const int t = threadIdx.x & 31;
            float e[4];
            double sq = 0.0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                e[i] = ob[4 * t + i];
                const float q2 = e[i] * e[i];
                sq += (double)q2;
            }
            sq = group_sum_last<32>(sq);
            sq = __shfl(sq, ((int)threadIdx.x & 32) | 31, 64);
            const float gi = rms_inv(sq, D, a.eps);
            const float gg[4] = {tail_g.x, tail_g.y, tail_g.z, tail_g.w};
            const float zz[4] = {tail_z.x, tail_z.y, tail_z.z, tail_z.w};
            typedef _Float16 h4v __attribute__((ext_vector_type(4)));
            h4v hv4;
#pragma unroll
            for (int i = 0; i < 4; ++i) hv4[i] = (_Float16)(((e[i] * gi) * gg[i]) * ggml_silu(zz[i]));
            const int k = h * D + 4 * t, m = b;
            const size_t lane_t = (size_t)((k & 15) >> 3) * 32 + (m & 31);
            const size_t at = ((((size_t)(m >> 5) * (W >> 8) + (k >> 8)) * 16 + ((k & 255) >> 4)) * 64 + lane_t) * 8 + (k & 7);
            if (threadIdx.x < 32) *(h4v*)((_Float16*)a.xh + at) = hv4;
        }
    }
}

hipError_t gdn_decode(const GdnDecodeArgs& a, size_t B, hipStream_t s) {
    if (a.H <= 0 || B == 0) return hipErrorInvalidValue;
    if (a.xh) {
        if (!a.norm || (a.H * 128) % 256) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gdn_decode_kernel<true>, dim3((unsigned)a.H, (unsigned)B), dim3(1024), 0, s, a);
    } else {
        hipLaunchKernelGGL(gdn_decode_kernel<false>, dim3((unsigned)(a.H * 4), (unsigned)B), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

// ===================================================== attention decode

template <typename KV>
__device__ __forceinline__ float kv_ld(const KV* p);
template <>
__device__ __forceinline__ float kv_ld<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float kv_ld<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }
template <typename KV>
__device__ __forceinline__ KV kv_st(float v);
template <>
__device__ __forceinline__ float kv_st<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t kv_st<uint16_t>(float v) {
    uint32_t b = __float_as_uint(v);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}
template <typename KV>
__device__ __forceinline__ void kv_ld4(const KV* p, float (&o)[4]);
template <>
__device__ __forceinline__ void kv_ld4<float>(const float* p, float (&o)[4]) {
    const v4f v = *(const v4f*)p;
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
template <>
__device__ __forceinline__ void kv_ld4<uint16_t>(const uint16_t* p, float (&o)[4]) {
    const uint2 v = *(const uint2*)p;
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
}

// Four consecutive cache elements kept in their storage form until used.
template <typename KV>
struct KVPack;
template <>
struct KVPack<float> {
    v4f v;
    __device__ __forceinline__ void load(const float* p) { v = *(const v4f*)p; }
    __device__ __forceinline__ void zero() { v = v4f{0.0f, 0.0f, 0.0f, 0.0f}; }
    __device__ __forceinline__ void unpack(float (&o)[4]) const {
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
};
template <>
struct KVPack<uint16_t> {
    uint2 v;
    __device__ __forceinline__ void load(const uint16_t* p) { v = *(const uint2*)p; }
    __device__ __forceinline__ void zero() { v = make_uint2(0u, 0u); }
    __device__ __forceinline__ void unpack(float (&o)[4]) const {
        o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
    }
};

// RoPE of one 256-wide head held in LDS, lanes < 32 of a wave
// (lib.rs:1552-1577: pairs (i, i+32), angle starts at the position and is
// multiplied by theta_scale per pair, FMA form).
__device__ __forceinline__ void head_rope(float* hv, const float* sn, const float* cs, int lane) {
    if (lane < 32) {
        const float a = hv[lane], bb = hv[lane + 32];
        hv[lane] = fmaf(a, cs[lane], -(bb * sn[lane]));
        hv[lane + 32] = fmaf(a, sn[lane], bb * cs[lane]);
    }
}

// Grid (nblk, kv_heads, B).  Each workgroup: (1) issues the key loads of its
// first token block, (2) normalises (forward.rs:680-695) and ropes
// (lib.rs:1552-1577) the G query heads of its kv head and the new key (one
// head per wave, redundant across workgroups: ~1 KB of work), (3) appends
// K/V at the row's position if it owns that token block, (4) scores its token
// blocks blockIdx.x, +nblk, ... in the reference's 32-accumulator dot order
// (see attn_qk_kernel), the position's own token from its copy of the stored
// key.
template <typename KV, int G>
__global__ __launch_bounds__(256) void attn_decode_qk_kernel(AttnDecodeArgs a) {
    constexpr int D = 256;
    __shared__ float hv[G + 1][D];
    __shared__ float rsin[32], rcos[32];
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int p = a.pos[b], T = p + 1;
    const int nblk = gridDim.x;
    const int s = tid & 7;
    const float* proj = a.proj + (size_t)b * a.proj_stride;
    const int QD2 = a.nq * 2 * D;
    KV* kc = (KV*)a.kcache + (size_t)b * a.cache_row_stride + (size_t)kvh * D;
    KV* vc = (KV*)a.vcache + (size_t)b * a.cache_row_stride + (size_t)kvh * D;
    const size_t tstep = (size_t)a.nkv * D;

    KVPack<KV> kn[8];  // keys of the next token block, loaded ahead
    // bounded by the cache size, not by the position, so the first loads do
    // not wait for it; tokens at or past the position are replaced or
    // dropped where they are used
    auto load_keys = [&](int tb) {
        const int t = min(tb * 32 + (tid >> 3), a.max_ctx - 1);
#pragma unroll
        for (int c = 0; c < 8; ++c) kn[c].load(kc + (size_t)t * tstep + 32 * c + 4 * s);
    };
    // q heads (tasks 0..G-1) and the key (task G): wave w takes tasks w,
    // w+4.  Their loads are issued before the first token block's keys (a
    // wave's loads complete in issue order, so the normalisation waits only
    // for its own inputs); a task past G loads task G's rows and is dropped.
    constexpr int NR = G / 4 + 1;
    float tv[NR][4], tg[NR][4];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int task = min(4 * i + wv, G);
        const float* src = task < G ? proj + (size_t)(kvh * G + task) * 2 * D : proj + QD2 + (size_t)kvh * D;
        const float* gamma = task < G ? a.qnorm : a.knorm;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            tv[i][r] = src[lane + 64 * r];
            tg[i][r] = gamma[lane + 64 * r];
        }
    }
    load_keys(blockIdx.x);

    // rotation angles of this position, shared by every head
    if (tid < 32) {
        float angle = (float)p;
        for (int t = 0; t < tid; ++t) angle *= a.theta_scale;
        rsin[tid] = cr_sinf(angle);
        rcos[tid] = cr_cosf(angle);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int task = 4 * i + wv;
        if (task <= G) {
            const float* v = tv[i];
            const float* gm = tg[i];
            double sq = 0.0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float q = v[r] * v[r];
                sq += (double)q;
            }
            sq = wave_sum_xor<double>(sq, 64);
            const float inv = rms_inv(sq, D, a.eps);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float t = v[r] * inv;
                hv[task][lane + 64 * r] = t * gm[r];
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int task0 = 0; task0 <= G; task0 += 4) {
        const int task = task0 + wv;
        if (task <= G) head_rope(hv[task], rsin, rcos, lane);
    }
    __syncthreads();
    {
        const KV st = kv_st<KV>(hv[G][tid]);
        if (((p >> 5) % nblk) == (int)blockIdx.x) {
            const float* vsrc = proj + QD2 + (size_t)a.nkv * D + (size_t)kvh * D;
            kc[(size_t)p * tstep + tid] = st;
            vc[(size_t)p * tstep + tid] = kv_st<KV>(vsrc[tid]);
        }
        __syncthreads();
        hv[G][tid] = kv_ld<KV>(&st);
        __syncthreads();
    }
    float qv[G][8][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[g][c][e] = hv[g][32 * c + 4 * s + e];
    float* sb = a.scores + (size_t)b * a.score_stride + (size_t)kvh * G * a.head_stride;
    for (int tb = blockIdx.x; tb * 32 < T; tb += nblk) {
        KVPack<KV> cur[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) cur[c] = kn[c];
        if ((tb + nblk) * 32 < T) load_keys(tb + nblk);
        const int t = tb * 32 + (tid >> 3);
        float kk[8][4];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (t == p) {
#pragma unroll
                for (int e = 0; e < 4; ++e) kk[c][e] = hv[G][32 * c + 4 * s + e];
            } else {
                cur[c].unpack(kk[c]);
            }
        }
        float acc[G][4];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[g][e] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[g][e] = fmaf(qv[g][c][e], kk[c][e], acc[g][e]);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[g][e] = group8_tree_last(acc[g][e]);
        if (t < T && s == 7) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float dot = (acc[g][0] + acc[g][1]) + (acc[g][2] + acc[g][3]);
                sb[(size_t)g * a.head_stride + t] = dot * a.scale;
            }
        }
    }

}

// Softmax statistics of one head's T scores (lib.rs:1352-1387) by a
// workgroup of 256 threads: max, GGML exp, 8-wide f32 partials summed in
// f64, inv = (float)(1/sum).  Thread t owns 8-element blocks t, t+256, ...
// of each 4096-token span.  Returns {max, inv} to every thread and the f64
// sum (for the degenerate check).
//
// One span's scores in registers, -inf past T; loads bounded by the cache
// size, not by T, so they are issued before T is known, without branches.
__device__ __forceinline__ void softmax_span_load(const float* row, int base, int T, int max_ctx, float (&e)[2][8]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int at = base + 8 * (tid + 256 * r) + i;
            const float sv = row[min(at, max_ctx - 1)];
            e[r][i] = at < T ? sv : -INFINITY;
        }
}

// Statistics of a row that fits one span (T <= 4096), from its registers;
// x returns GGML exp(score - max) per element, zero past T.
__device__ __forceinline__ void softmax_span_stats(const float (&e)[2][8], int T, float& m_out, float& inv_out,
                                                   double& total_out, float (&x)[2][8]) {
    __shared__ float wmax[4];
    __shared__ double wsum[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, e[r][i]);
    m = wave_max(m);
    if (lane == 0) wmax[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    double sum = 0.0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[r][i] = 8 * (tid + 256 * r) + i < T ? ggml_exp(e[r][i] - m) : 0.0f;
        if (8 * (tid + 256 * r) < T) {
            const float partial =
                ((x[r][0] + x[r][4]) + (x[r][2] + x[r][6])) + ((x[r][1] + x[r][5]) + (x[r][3] + x[r][7]));
            sum += (double)partial;
        }
    }
    sum = wave_sum_xor<double>(sum, 64);
    if (lane == 0) wsum[wv] = sum;
    __syncthreads();
    const double total = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    m_out = m;
    inv_out = (float)(1.0 / total);
    total_out = total;
}

__device__ __forceinline__ void softmax_stats(const float* row, int T, int max_ctx, float& m_out, float& inv_out,
                                              double& total_out) {
    if (T <= 4096) {  // one span: each score loaded once
        float e[2][8], x[2][8];
        softmax_span_load(row, 0, T, max_ctx, e);
        softmax_span_stats(e, T, m_out, inv_out, total_out, x);
        return;
    }
    __shared__ float wmax[4];
    __shared__ double wsum[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float m = -INFINITY;
    double sum = 0.0;
    for (int pass = 0; pass < 2; ++pass) {
        for (int base = 0; base < T; base += 4096) {
            float e[2][8];
            softmax_span_load(row, base, T, max_ctx, e);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                if (pass == 0) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) m = fmaxf(m, e[r][i]);
                } else if (base + 8 * (tid + 256 * r) < T) {
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) x[i] = base + 8 * (tid + 256 * r) + i < T ? ggml_exp(e[r][i] - m) : 0.0f;
                    const float partial = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
                    sum += (double)partial;
                }
            }
        }
        if (pass == 0) {
            m = wave_max(m);
            if (lane == 0) wmax[wv] = m;
            __syncthreads();
            m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        }
    }
    sum = wave_sum_xor<double>(sum, 64);
    if (lane == 0) wsum[wv] = sum;
    __syncthreads();
    const double total = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    m_out = m;
    inv_out = (float)(1.0 / total);
    total_out = total;
}

// Grid (q_heads, B): the statistics of one head, stored as {max, inv} for
// the value kernel (batches of 8 rows and more).
__global__ __launch_bounds__(256) void attn_decode_stats_kernel(AttnDecodeArgs a) {
    const int h = blockIdx.x, b = blockIdx.y;
    const int T = a.pos[b] + 1;
    const float* row = a.scores + (size_t)b * a.score_stride + (size_t)h * a.head_stride;
    float m, inv;
    double total;
    softmax_stats(row, T, a.max_ctx, m, inv, total);
    if (threadIdx.x == 0) {
        a.stats[((size_t)b * a.nq + h) * 2] = m;
        a.stats[((size_t)b * a.nq + h) * 2 + 1] = inv;
        if (!(total >= 1.0) || !(total < INFINITY)) atomicOr(a.status, 8);
    }
}

// CPT consecutive cache elements as f32 (CPT = 1, 2 or 4).
template <typename KV, int CPT>
__device__ __forceinline__ void kv_ldn(const KV* p, float (&o)[CPT]) {
    if constexpr (CPT == 4) {
        kv_ld4<KV>(p, o);
    } else if constexpr (sizeof(KV) == 4) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) o[c] = ((const float*)p)[c];
    } else if constexpr (CPT == 2) {
        const uint32_t v = *(const uint32_t*)p;
        o[0] = __uint_as_float(v << 16);
        o[1] = __uint_as_float(v & 0xffff0000u);
    } else {
        o[0] = __uint_as_float((uint32_t)*(const uint16_t*)p << 16);
    }
}

// Grid (256 / (8 CPT), q_heads / HG, B): the value sum of attn_pv_kernel
// (32 FMA chains over tokens per channel, lib.rs:1276-1305) for HG query
// heads (sharing one kv head) over 8 CPT channels per workgroup.  Lane =
// channel-group * 8 + chain % 8, wave = chain / 8: a thread runs chain `a`
// for CPT adjacent channels.  Per tile of 32 NV tokens every value and score
// load is issued at once (bounded by the cache, not the position, so they
// do not wait for it), p = GGML exp(score - max) * inv is staged in LDS as
// [token][heads], and the chains advance in token order; the fixed tree and
// the sigmoid output gate (forward.rs:751) finish.  The LDS barriers do not
// wait for the value loads, which only the chains consume.  Few heads and
// channels per workgroup spread a single row over many workgroups.
template <typename KV, int HG, int CPT, int NV, bool FS>
__global__ __launch_bounds__(256) void attn_decode_pv_kernel(AttnDecodeArgs a) {
    constexpr int D = 256, TT = 32 * NV, CB = 8 * CPT, NS = HG * TT / 256, HP = HG == 3 ? 4 : HG;
    __shared__ float pt[TT * HP];
    __shared__ float red[HG][CB][33];
    // XCD-aware order: workgroup L (dispatch order) runs on XCD L % 8, so the
    // logical ids are dealt to give each XCD a contiguous range, in which the
    // heads of one kv head vary fastest (HG == 1), then the channel groups:
    // the workgroups that share V's cache lines (adjacent channel groups, the
    // heads of a kv head) then share one XCD's L2 and each line is fetched
    // once, not once per XCD.
    const unsigned nx = gridDim.x, ny = gridDim.y, nwg = nx * ny * gridDim.z;
    const unsigned lin = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const unsigned q = nwg % 8 ? lin : (lin % 8) * (nwg / 8) + lin / 8;
    int cgx, h0, b;
    if constexpr (HG == 1) {
        const unsigned G = (unsigned)(a.nq / a.nkv);
        const unsigned g = q % G, r = q / G;
        cgx = (int)(r % nx);
        const unsigned r2 = r / nx;
        h0 = (int)((r2 % (unsigned)a.nkv) * G + g);
        b = (int)(r2 / (unsigned)a.nkv);
    } else {
        cgx = (int)(q % nx);
        h0 = (int)((q / nx) % ny) * HG;
        b = (int)(q / (nx * ny));
    }
    const int kvh = h0 / (a.nq / a.nkv);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int T = a.pos[b] + 1;
    const float* sb = a.scores + (size_t)b * a.score_stride + (size_t)h0 * a.head_stride;
    float gate = 0.0f;
    if (tid < HG * CB) {
        const int g = tid / CB, c = tid % CB;
        gate = a.proj[(size_t)b * a.proj_stride + (size_t)(h0 + g) * 2 * D + D + cgx * CB + c];
    }
    const int cq = lane >> 3, ai = wv * 8 + (lane & 7);
    const int j0 = cgx * CB + cq * CPT;
    const KV* vb = (const KV*)a.vcache + (size_t)b * a.cache_row_stride + (size_t)kvh * D + j0;
    const size_t vstep = (size_t)a.nkv * D;
    const int tmax = a.max_ctx - 1;
    float acc[HG][CPT];
#pragma unroll
    for (int g = 0; g < HG; ++g)
#pragma unroll
        for (int c = 0; c < CPT; ++c) acc[g][c] = 0.0f;
    // unconditional loads (no branches: a load in a branch is followed by a
    // wait there), token indices clamped to the last token, so that rows
    // past the position reread a line already in cache; their values are
    // masked where they are used
    auto load_values = [&](int t0, float (&vv)[NV][CPT]) {
        const KV* vt = vb + (size_t)(t0 + ai) * vstep;
        if (t0 + TT <= T) {
#pragma unroll
            for (int n = 0; n < NV; ++n) kv_ldn<KV, CPT>(vt + (size_t)(32 * n) * vstep, vv[n]);
        } else {
#pragma unroll
            for (int n = 0; n < NV; ++n) kv_ldn<KV, CPT>(vb + (size_t)min(t0 + ai + 32 * n, T - 1) * vstep, vv[n]);
        }
    };
    // the chains over one tile, its probabilities staged in pt
    auto run_chains = [&](int t0, const float (&vv)[NV][CPT]) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int tt = ai + 32 * n;
            const bool live = t0 + tt < T;  // a select, not a branch: past T the chain is unchanged
            float p4[HP];
            if constexpr (HP == 4) {
                const v4f q = *(const v4f*)&pt[tt * 4];
                p4[0] = q.x; p4[1] = q.y; p4[2] = q.z; p4[3] = q.w;
            } else {
#pragma unroll
                for (int g = 0; g < HP; ++g) p4[g] = pt[tt * HP + g];
            }
#pragma unroll
            for (int g = 0; g < HG; ++g)
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    const float f = fmaf(vv[n][c], p4[g], acc[g][c]);
                    acc[g][c] = live ? f : acc[g][c];
                }
        }
    };
    float mx[HG], inv[HG];
    bool tiled = true;
    float gate_s = 0.0f;
    if constexpr (FS) {
        // small batches: the head's statistics computed here (the same
        // arithmetic as attn_decode_stats_kernel, so the same values) instead
        // of a launch
        static_assert(HG == 1, "fused statistics are per head");
        static_assert(TT <= 4096, "one tile within one statistics span");
        double total;
        if (T <= TT) {
            // one tile: each score loaded once for the statistics and the
            // probabilities, the values issued right behind the scores so
            // that their latency overlaps the statistics
            float e[2][8], x[2][8], vv[NV][CPT];
            softmax_span_load(sb, 0, T, a.max_ctx, e);
            load_values(0, vv);
            // the output gate (an f64 exp) while the scores and values are
            // in flight (the gate was loaded first)
            gate_s = source_sigmoid(gate);
            softmax_span_stats(e, T, mx[0], inv[0], total, x);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int tt = 8 * (tid + 256 * r) + i;
                    if (tt < TT) pt[tt] = x[r][i] * inv[0];
                }
            lds_barrier();
            run_chains(0, vv);
            tiled = false;
        } else {
            softmax_stats(sb, T, a.max_ctx, mx[0], inv[0], total);
        }
        if (cgx == 0 && tid == 0 && (!(total >= 1.0) || !(total < INFINITY))) atomicOr(a.status, 8);
    } else {
#pragma unroll
        for (int g = 0; g < HG; ++g) {
            mx[g] = a.stats[((size_t)b * a.nq + h0 + g) * 2];
            inv[g] = a.stats[((size_t)b * a.nq + h0 + g) * 2 + 1];
        }
    }
    for (int t0 = 0; tiled && t0 < T; t0 += TT) {
        float vv[NV][CPT];
        load_values(t0, vv);
        float sv[NS];
#pragma unroll
        for (int r = 0; r < NS; ++r) {
            const int i = tid + 256 * r, g = i / TT, t = t0 + i % TT;
            sv[r] = sb[(size_t)g * a.head_stride + min(t, tmax)];
        }
#pragma unroll
        for (int r = 0; r < NS; ++r) {
            const int i = tid + 256 * r, g = i / TT, tt = i % TT;
            pt[tt * HP + g] = t0 + tt < T ? ggml_exp(sv[r] - mx[g]) * inv[g] : 0.0f;
        }
        lds_barrier();
        run_chains(t0, vv);
        lds_barrier();
    }
#pragma unroll
    for (int g = 0; g < HG; ++g)
#pragma unroll
        for (int c = 0; c < CPT; ++c) red[g][cq * CPT + c][ai] = acc[g][c];
    __syncthreads();
    if (tid < HG * CB) {
        const int g = tid / CB, c = tid % CB;
        const float* r = red[g][c];
        float comb[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) comb[l] = (r[l] + r[16 + l]) + (r[8 + l] + r[24 + l]);
        const float h0s = comb[0] + comb[4], h1 = comb[1] + comb[5], h2 = comb[2] + comb[6], h3 = comb[3] + comb[7];
        float v = (h0s + h1) + (h2 + h3);
        v = v * (tiled ? source_sigmoid(gate) : gate_s);
        a.out[(size_t)b * a.out_stride + (size_t)(h0 + g) * D + cgx * CB + c] = v;
        if (a.xh) {
            const int k = (h0 + g) * D + cgx * CB + c, m = b, K = a.nq * D;
            const size_t lane_t = (size_t)((k & 15) >> 3) * 32 + (m & 31);
            const size_t at = ((((size_t)(m >> 5) * (K >> 8) + (k >> 8)) * 16 + ((k & 255) >> 4)) * 64 + lane_t) * 8 + (k & 7);
            ((_Float16*)a.xh)[at] = (_Float16)v;
        }
    }
}

template <typename KV, int G>
static void launch_attn(const AttnDecodeArgs& a, size_t B, hipStream_t s) {
    // token blocks per (row, kv head): 64 at batch 1, fewer as rows add
    // parallelism (each workgroup then pipelines several blocks)
    const size_t want = B >= 8 ? 8 : 64 / B;
    const unsigned nblk = (unsigned)std::min<size_t>((a.max_ctx + 31) / 32, want);
    hipLaunchKernelGGL((attn_decode_qk_kernel<KV, G>), dim3(nblk, a.nkv, (unsigned)B), dim3(256), 0, s, a);
    // batch < 8: one head and 8 channels per workgroup (a row over 32 x nq
    // workgroups, each token tile in one burst), the softmax statistics
    // folded in; rows in numbers: a statistics launch, then the kv head's G
    // heads and 32 channels per workgroup
    if (B >= 8) {
        hipLaunchKernelGGL(attn_decode_stats_kernel, dim3(a.nq, (unsigned)B), dim3(256), 0, s, a);
        hipLaunchKernelGGL((attn_decode_pv_kernel<KV, G, 4, 16, false>), dim3(256 / 32, a.nq / G, (unsigned)B), dim3(256),
                           0, s, a);
    } else {
        // one tile of 72 x 32 tokens when it covers the whole cache (fewer
        // clamped loads past the position than the 96 x 32 tile), else 96
        if (a.max_ctx <= 72 * 32)
            hipLaunchKernelGGL((attn_decode_pv_kernel<KV, 1, 1, 72, true>), dim3(256 / 8, a.nq, (unsigned)B), dim3(256), 0,
                               s, a);
        else
            hipLaunchKernelGGL((attn_decode_pv_kernel<KV, 1, 1, 96, true>), dim3(256 / 8, a.nq, (unsigned)B), dim3(256), 0,
                               s, a);
    }
}

hipError_t attn_decode(const AttnDecodeArgs& a, size_t B, hipStream_t s) {
    if (a.nkv <= 0 || a.nq % a.nkv || B == 0 || a.max_ctx <= 0) return hipErrorInvalidValue;
    const int G = a.nq / a.nkv;
#define ZG_AT(KV)                                              \
    switch (G) {                                               \
    case 1: launch_attn<KV, 1>(a, B, s); break;                \
    case 2: launch_attn<KV, 2>(a, B, s); break;                \
    case 3: launch_attn<KV, 3>(a, B, s); break;                \
    case 4: launch_attn<KV, 4>(a, B, s); break;                \
    default: return hipErrorInvalidValue;                      \
    }
    if (a.kv_bf16) {
        ZG_AT(uint16_t)
    } else {
        ZG_AT(float)
    }
#undef ZG_AT
    return hipGetLastError();
}

// ================================================== greedy + position

// Greedy id per row (core/src/numerics.rs:126-140: first maximum wins,
// nonfinite is an error -> status bit 2) in two launches: kArgBlocks
// partial (max, first index) pairs per row, then one wave per row reduces
// them, writes the id and, when asked, moves the row's position on.
constexpr int kArgBlocks = 64;

__device__ __forceinline__ void argmax_merge(float& best, int& bi, float ov, int oi) {
    if (ov > best || (ov == best && oi < bi)) {
        best = ov;
        bi = oi;
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits, int V, size_t ld,
                                                             int* __restrict__ status, float* __restrict__ pmax,
                                                             int* __restrict__ pidx) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int blk = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int per = ((V + kArgBlocks - 1) / kArgBlocks + 3) & ~3;
    const int lo = blk * per, hi = min(V, lo + per);
    const float* row = logits + (size_t)b * ld;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    bool bad = false;
    for (int i0 = lo; i0 < hi; i0 += 256 * 4) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = i0 + tid + 256 * r;
            v[r] = i < hi ? row[i] : -INFINITY;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = i0 + tid + 256 * r;
            if (i < hi) {
                if (!finite_f32(v[r])) bad = true;
                argmax_merge(best, bi, v[r], i);
            }
        }
    }
    if (bad) atomicOr(status, 4);
    for (int off = 32; off > 0; off >>= 1) argmax_merge(best, bi, __shfl_xor(best, off, 64), __shfl_xor(bi, off, 64));
    if (lane == 0) {
        sv[wv] = best;
        si[wv] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) argmax_merge(best, bi, sv[w], si[w]);
        pmax[b * kArgBlocks + blk] = best;
        pidx[b * kArgBlocks + blk] = bi;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pmax, const int* __restrict__ pidx,
                                                          uint32_t* __restrict__ greedy, int* __restrict__ pos,
                                                          int* __restrict__ ntok, int advance) {
    const int b = blockIdx.x, lane = threadIdx.x;
    float m = lane < kArgBlocks ? pmax[b * kArgBlocks + lane] : -INFINITY;
    int mi = lane < kArgBlocks ? pidx[b * kArgBlocks + lane] : 0x7fffffff;
    for (int off = 32; off > 0; off >>= 1) argmax_merge(m, mi, __shfl_xor(m, off, 64), __shfl_xor(mi, off, 64));
    if (lane == 0) {
        greedy[b] = mi == 0x7fffffff ? 0u : (uint32_t)mi;
        if (advance) {
            const int np = pos[b] + 1;
            pos[b] = np;
            ntok[b] = np + 1;
        }
    }
}

hipError_t argmax_step(const float* logits, size_t V, size_t ld, size_t B, uint32_t* greedy, int* status, float* pmax,
                       int* pidx, unsigned* tickets, int* pos, int* ntok, int advance, hipStream_t s) {
    (void)tickets;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks, (unsigned)B), dim3(256), 0, s, logits, (int)V, ld, status,
                       pmax, pidx);
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)B), dim3(64), 0, s, pmax, pidx, greedy, pos, ntok, advance);
    return hipGetLastError();
}

size_t argmax_partials(size_t B) { return B * kArgBlocks; }

}  // namespace zg
