// Batched-row (B > 4) decode projections on f16 MFMA and the prompt-sized GEMMs.
#include "zg_decode_common.hpp"

namespace zg {

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
            for (int t = 0; t < 4; ++t) {
                hv4[t] = valid ? (_Float16)e[t] : (_Float16)0.0f;
                // past the f16 range: status bit 4 (the f32 paths carry it)
                if (a.status && valid && !(fabsf(e[t]) <= 65504.0f)) atomicOr(a.status, 16);
            }
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
    __shared__ float inv_s[32];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, hsel = lane >> 5, r32 = lane & 31;
    const int m0 = blockIdx.y * 32;
    const int K = a.K, N = a.N, nbk = K >> 8;
    // an RMS projection on tiles a residual projection left (rms_ss_in):
    // its per-tile sums of squares for the 32 rows are requested now (TPR
    // adjacent threads per row, 8 each) and reduced after the main loop
    constexpr int TPR = KS >= 8 ? 16 : 8;
    const int srow = threadIdx.x / TPR, ssub = threadIdx.x % TPR;
    double ssv[8];
    if (a.rms_ss_in) {
        const int n = a.rms_ss_n;
        const double* ss = a.rms_ss_in + (size_t)(m0 + min(srow, 31)) * n;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int c = ssub + q * TPR;
            const double x = ss[min(c, n - 1)];
            ssv[q] = c < n && srow < 32 ? x : 0.0;
        }
    }
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
    if (a.rms_ss_in) {  // (rms_ss_n <= 8 * TPR; the first barrier below orders inv_s)
        double tot = 0.0;
#pragma unroll
        for (int q = 0; q < 8; ++q) tot += ssv[q];
        tot = group_sum_last<TPR>(tot);
        if (srow < 32 && ssub == TPR - 1) inv_s[srow] = rms_inv(tot, K, a.eps);
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
            if (a.rms_ss_in) v *= inv_s[m - m0];
            if (EPI == EPI_RESID && a.rms_tiles_out) {
                // the residual finished here, then the next RMS projection's
                // A tile element (m, n): f16(x_new * gamma) (its 1/rms is
                // applied after its dot), and this tile's f64 sum of the f32
                // squares of x_new per row (lanes of one half share a row)
                const int n = nbase[t] + r32;
                const bool live = nv[t] && m < a.M;
                float xn = 0.0f;
                if (live) {
                    float* p = a.y + (size_t)m * a.ldy + n;
                    xn = *p + v;  // source_binary Add, lib.rs:1258-1271
                    *p = xn;
                    if (!finite_f32(xn)) atomicOr(a.status, 1);
                }
                if (nv[t]) {
                    const float tv = live ? xn * a.rms_gamma[n] : 0.0f;
                    if (!(fabsf(tv) <= 65504.0f)) atomicOr(a.status, 16);
                    const size_t at = ((((size_t)(m >> 5) * (N >> 8) + (n >> 8)) * 16 + ((n & 255) >> 4)) * 64 +
                                       ((n & 15) >> 3) * 32 + (m & 31)) * 8 + (n & 7);
                    a.rms_tiles_out[at] = (_Float16)tv;
                }
                const float sq = xn * xn;
                const double tot = group_sum_last<32>((double)sq);
                if (r32 == 31 && nbase[t] < N) a.rms_ss_out[(size_t)m * (N >> 5) + (nbase[t] >> 5)] = tot;
                continue;
            }
            if (EPI == EPI_GLU) {
                if (t == 0) {
                    vg[i] = v;
                } else if (nv[t]) {
                    // up * silu(gate), rounded to f16 into the down
                    // projection's activation tiles (K2 = N/2 columns)
                    const int j = nbase[0] + r32, nbk2 = (N >> 1) >> 8;
                    const size_t at = ((((size_t)(m >> 5) * nbk2 + (j >> 8)) * 16 + ((j & 255) >> 4)) * 64 +
                                       ((j & 15) >> 3) * 32 + (m & 31)) * 8 + (j & 7);
                    const float pr = m < a.M ? v * ggml_silu(vg[i]) : 0.0f;
                    if (a.status && !(fabsf(pr) <= 65504.0f)) atomicOr(a.status, 16);
                    ((_Float16*)a.xh_out)[at] = (_Float16)pr;
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
        const uint8_t* b = qs + q4k_chunk_offset(row, 4 * kb + c4, K) + 8 * hsel;
        const uint2 p0 = *(const uint2*)b, p1 = *(const uint2*)(b + 256);
        out = v4u{p0.x, p0.y, p1.x, p1.y};
    }
    qs_t[(((size_t)tile * nbk + kb) * 4 + c4) * 64 + lane] = out;
    if (tid < 32) {
        const int r = tile * 32 + tid;
        hdr_t[((size_t)tile * nbk + kb) * 32 + tid] = r < N ? hdr[q4k_hdr_index(r, kb, nbk)] : v4u{0u, 0u, 0u, 0u};
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

hipError_t batched_gemv(const DeviceWeight& w, const FusedGemvArgs& args, void* scratch, hipStream_t s) {
    if (w.type != kQ4_K || w.K % 256 || w.K > 8192 || args.M <= 0 || args.M > 65535 * 32) return hipErrorInvalidValue;
    if (args.pro == PRO_GATED && args.group != 128) return hipErrorInvalidValue;
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
    if ((a.rms_tiles_out || a.rms_ss_in) && a.splits > 1) return hipErrorInvalidValue;
    if (a.rms_ss_in && a.rms_ss_n > 64) return hipErrorInvalidValue;  // 8 sums per thread, 8+ threads per row
    // prompt-sized M: the register-blocked GEMM (zg_gemm.hip)
    const bool no_split = !(a.epi == EPI_RESID && a.splits > 1 && a.parts);
    if (a.M >= kGemmRows && no_split && !a.rms_tiles_out && !a.rms_ss_in &&
        prompt_gemm_supported(w.type, w.K, w.N, a.epi))
        return prompt_gemm(w, args, xh, s);
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


}  // namespace zg
