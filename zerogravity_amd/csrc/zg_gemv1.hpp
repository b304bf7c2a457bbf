#pragma once
// Decode GEMV of one activation row (B = 1) against Q4_K weights on the
// int8 matrix cores (v_mfma_i32_16x16x64_i8).
//
// Why the matrix cores at B = 1: without packed FP32 the chip retires about
// 39 T VALU lane-ops/s, only ~2.8 per weight at the HBM rate, and an f32
// dequant-dot needs about that many (measured: VALU-bound LM head).  Here
// the VALU only unpacks nibbles (3 ops per 8 weights) and applies the group
// scales; the products run on the MFMA pipe.
//
// Activation: each wave of the workgroup owns 512 elements of K (K / 512
// waves) and codes them per 32-group to int16, c = rint(b * 32639 / amax),
// split into signed bytes c = 256 h + l (h, l in [-128, 127]); the group's
// scale amax / 32639 and its f32 sum go to LDS.  b is the prologue value
// without the RMS factor: RMSNorm's 1 / rms multiplies the row sums at the
// end and the gated norm's per-head factor multiplies the group scales, so
// the coding needs no cross-wave reduction.
//
// Tile: 16 weight rows (8 gate + 8 up with EPI_GLU).  Lane l = (j = l % 16,
// s = l / 16) of wave w reads 16 bytes at byte 64 (4w + u) + 16 s of row j
// for units u = 0..3 (a unit is 128 elements, 64 bytes; the weight layout
// puts the 64 lanes' pieces side by side): the B operand of
// MFMA (u, nibble n) is the low (n = 0) or high (n = 1) nibbles of those
// bytes, the elements 64 (s / 2) + 32 n + 16 (s % 2) + [0, 16) of the unit.
// The A operand of MFMA (u, n) holds in row 4u + 2 hh + x (hh = the unit's
// chunk half, x = 0 high bytes, 1 low bytes) the codes of the same elements
// where the lane's k-slice s lies in half hh, zero elsewhere; rows of other
// units are zero, so the four MFMAs of a nibble accumulate into one D whose
// lane (j, s) holds unit s's four partial sums for row j:
//   D = {h.q half 0, l.q half 0, h.q half 1, l.q half 1}.
// Each lane then applies its unit's four group scales (Q4_K d * sc, dmin * mn
// from the row's block header, and the activation group scales), the four
// lanes of a row are summed, and the waves' partials are added in wave
// order through LDS.  The weights of the next tile are requested before the
// cross-wave sum.
//
// Per group of 32 this forms scale * (sum of q * a) - min * (sum of a): the
// reference's serial f32 sum of (q * scale - min) * a (cpu/src/source.rs:
// 431-459) regrouped, with a coded to 16 bits per group (relative step
// 1 / 32639 of the group's largest magnitude).
#include "zg_decode_common.hpp"

namespace zg {

constexpr int kGemv1MaxK = 8192;

__device__ __forceinline__ v4i g1_mfma(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <int W, int PRO, int EPI, int R>
__global__ __launch_bounds__(64 * W) void gemv1_q4k_kernel(FusedGemvArgs a) {
    static_assert(R == 16 || (R == 8 && EPI != EPI_GLU), "16-row tiles, or 8-row tiles without the GLU pairing");
    constexpr int K = 512 * W, nbk = K / 256;
    // R = 8: lanes j < 8 carry units 4w, 4w+1 and lanes j >= 8 units 4w+2,
    // 4w+3 of the same 8 rows (g = j / 8 picks the pair); U MFMAs per nibble
    constexpr int U = R == 16 ? 4 : 2;
    __shared__ __align__(16) int8_t cod[W][2][512];  // per wave: high bytes, low bytes, element order
    __shared__ float gmeta[W][16][2];                // per wave group: {scale, sum}
    __shared__ float part[2][W][16];
    __shared__ double ssq[W];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j = lane & 15, s = lane >> 4;
    const int nout = EPI == EPI_GLU ? (a.N >> 1) : a.N;
    constexpr int TR = EPI == EPI_GLU ? 8 : R;  // outputs per tile
    const int ntiles = (nout + TR - 1) / TR;
    // the GDN input projection's gate tiles go to the first workgroups, whose
    // weights arrive first, so the gates' f64 transcendentals end before the
    // last workgroups do (gate_dt); otherwise tiles in order
    const int tshift = (EPI == EPI_STORE && a.gate_dt) ? a.gate_row / TR : 0;
    auto tile_of = [&](int k) { return tshift ? (k + tshift) % ntiles : k; };
    const uint8_t* qs = (const uint8_t*)a.qs;
    const v4u* hdr = (const v4u*)a.hdr;

    auto row_of = [&](int t) {
        if (EPI == EPI_GLU) {
            const int o = min(t * 8 + (j & 7), nout - 1);
            return j < 8 ? o : nout + o;  // up rows follow the N/2 gate rows
        }
        return min(t * R + (R == 16 ? j : (j & 7)), nout - 1);  // past the end: re-read the last row, never stored
    };
    // the unit (of the wave's four) whose partial sums the lane's D rows
    // hold: s for R = 16; (s >> 1) + 2 (s & 1) for R = 8, valid on the lanes
    // whose pair g = j >> 3 is s & 1
    const int ue = R == 16 ? s : (s >> 1) + 2 * (s & 1);
    const bool lane_valid = R == 16 || (s & 1) == (j >> 3);
    v4u nib[U], hl;
    // piece s of units 4w .. 4w+3 (R = 8: of units 4w + 2g, 4w + 2g + 1) of
    // the lane's row: in the 16-row tile layout (q4k_chunk_offset) a wave
    // instruction reads 1 KB contiguously (R = 8: eight 128-byte runs)
    auto load_tile = [&](int t) {
        const size_t row = (size_t)row_of(t);
        const int u0 = 4 * w + (R == 16 ? 0 : 2 * (j >> 3));
        const uint8_t* rp = qs + (((row >> 4) * (K / 128) + u0) * 64 + (row & 15) + 16 * s) * 16;
#pragma unroll
        for (int u = 0; u < U; ++u) nib[u] = (v4u)load_nt(rp + 1024 * u);
        hl = hdr[q4k_hdr_index(row, (4 * w + ue) >> 1, nbk)];  // the block of unit ue
    };

    // ---- activation loads (issued first: a wave's loads complete in order)
    const int e = 512 * w + 8 * lane;
    v4f xv[2], ov[2], gv[2];
    if (PRO == PRO_EMBED_RMS) {
        // the token's embedding row: the weights go first (they do not
        // depend on the token), then this lane's 8 elements (one 8-byte
        // half-chunk piece and the block header) and gamma
        const uint32_t t = *a.tok;
        load_tile(tile_of(blockIdx.x));
        const bool ok = t < (uint32_t)a.emb_rows;
        const size_t row = ok ? t : 0;
        const uint8_t* eq = (const uint8_t*)a.emb_qs + q4k_chunk_offset(row, e >> 6, K) + ((e & 31) >= 16 ? 256 : 0) +
                            (e & 15);
        const uint2 nb = *(const uint2*)eq;
        const v4u eh = ((const v4u*)a.emb_hdr)[q4k_hdr_index(row, e >> 8, nbk)];
#pragma unroll
        for (int q = 0; q < 2; ++q) ov[q] = *(const v4f*)(a.gamma + e + 4 * q);
        uint32_t sc, mn;
        q4k_dev_scale_min(eh, (e & 255) >> 5, sc, mn);
        const float d = f16_to_f32((uint16_t)(eh.x & 0xffffu)), dm = f16_to_f32((uint16_t)(eh.x >> 16));
        const float scale = d * (float)sc, mnf = dm * (float)mn;
        const int sh = (e >> 5) & 1 ? 4 : 0;  // the high group's elements sit in the high nibbles
        float xe[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t byte = ((q < 4 ? nb.x : nb.y) >> (8 * (q & 3))) & 0xffu;
            xe[q] = ok ? scale * (float)((byte >> sh) & 15u) - mnf : 0.0f;
        }
        xv[0] = v4f{xe[0], xe[1], xe[2], xe[3]};
        xv[1] = v4f{xe[4], xe[5], xe[6], xe[7]};
        if (blockIdx.x == 0) {
            *(v4f*)(a.x_out + e) = xv[0];
            *(v4f*)(a.x_out + e + 4) = xv[1];
            if (!ok && tid == 0) atomicOr(a.status, 2);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            xv[q] = *(const v4f*)(a.x + e + 4 * q);
            if (PRO == PRO_RMS) ov[q] = *(const v4f*)(a.gamma + e + 4 * q);
            if (PRO == PRO_GATED || PRO == PRO_SILU_MUL || PRO == PRO_GATED_PRE) ov[q] = *(const v4f*)(a.x2 + e + 4 * q);
            if (PRO == PRO_GATED) gv[q] = *(const v4f*)(a.gamma + ((e + 4 * q) & (a.group - 1)));
        }
        __builtin_amdgcn_sched_barrier(0);
        load_tile(tile_of(blockIdx.x));
    }
    // a residual projection's outputs of the first tile, requested now (the
    // add at the end then waits on no further load); a wave's loads
    // complete in order, and the prologue waits only for the activation
    float ypre = 0.0f;
    if (EPI == EPI_RESID && w == 0 && lane < TR) {
        const int o = min((int)blockIdx.x * TR + j, nout - 1);
        ypre = a.y[o];
    }

    // ---- prologue values b (zg_decode_common.hpp's operations, without the
    // RMS factors)
    float b[8];
    double sq = 0.0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const float xe[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
        const float oe[4] = {ov[q].x, ov[q].y, ov[q].z, ov[q].w};
        const float ge[4] = {gv[q].x, gv[q].y, gv[q].z, gv[q].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float v = xe[t];
            if (PRO == PRO_RMS || PRO == PRO_GATED || PRO == PRO_GATED_PRE || PRO == PRO_EMBED_RMS) {
                const float sqr = v * v;
                sq += (double)sqr;
            }
            if (PRO == PRO_RMS || PRO == PRO_EMBED_RMS) v = v * oe[t];
            else if (PRO == PRO_GATED) v = (v * ge[t]) * ggml_silu(oe[t]);
            else if (PRO == PRO_SILU_MUL) v = oe[t] * ggml_silu(v);
            else if (PRO == PRO_GATED_PRE) v = oe[t];  // (x * gamma) * silu(z), formed by the producer
            b[4 * q + t] = v;
        }
    }
    float fold = 1.0f;
    if (PRO == PRO_GATED || PRO == PRO_GATED_PRE) {
        // per head of 128 elements: 16 lanes
        double hs = sq;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) hs += __shfl_xor(hs, o, 64);
        fold = rms_inv(hs, a.group, a.eps);
    }
    if (PRO == PRO_RMS || PRO == PRO_EMBED_RMS) {
        const double ws = group_sum_last<64>(sq);
        if (lane == 63) ssq[w] = ws;
    }
    // group of 32 = 4 lanes: largest magnitude and sum
    float amax = 0.0f, gsum = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        amax = fmaxf(amax, fabsf(b[t]));
        gsum += b[t];
    }
    amax = fmaxf(amax, dpp_f<kDppXor1>(amax));
    amax = fmaxf(amax, dpp_f<kDppXor2>(amax));
    gsum += dpp_f<kDppXor1>(gsum);
    gsum += dpp_f<kDppXor2>(gsum);
    const float qi = amax == 0.0f ? 0.0f : 32639.0f / amax;
    uint32_t hw[2] = {0u, 0u}, lw[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        int c = (int)rintf(b[t] * qi);
        c = min(max(c, -32639), 32639);
        const int hb = (c + 128) >> 8, lb = c - 256 * hb;
        hw[t >> 2] |= ((uint32_t)hb & 0xffu) << (8 * (t & 3));
        lw[t >> 2] |= ((uint32_t)lb & 0xffu) << (8 * (t & 3));
    }
    *(uint2*)&cod[w][0][8 * lane] = make_uint2(hw[0], hw[1]);
    *(uint2*)&cod[w][1][8 * lane] = make_uint2(lw[0], lw[1]);
    if ((lane & 3) == 0) {
        gmeta[w][lane >> 2][0] = (amax / 32639.0f) * fold;
        gmeta[w][lane >> 2][1] = gsum * fold;
    }
    // this wave's LDS writes complete before its own reads below
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // ---- A operands.  R = 16: unit u = j / 4 in rows 4u..4u+3 of MFMA u.
    // R = 8: MFMA u carries in rows 8u..8u+3 unit u (for the columns of
    // pair 0) and in rows 8u+4..8u+7 unit u + 2 (pair 1); the products of
    // a row with the other pair's columns are never read.
    v4i A[U][2];
    {
        const int ua = R == 16 ? (j >> 2) : (j >> 3) + 2 * ((j >> 2) & 1);  // the unit of A row j
        const int ma = R == 16 ? (j >> 2) : (j >> 3);                        // the MFMA that carries it
        const bool mine = ((j >> 1) & 1) == (s >> 1);
        const int8_t* src = cod[w][j & 1] + 128 * ua + 64 * (s >> 1) + 16 * (s & 1);
        const v4i z = {0, 0, 0, 0};
        const v4i v0 = mine ? *(const v4i*)src : z;
        const v4i v1 = mine ? *(const v4i*)(src + 32) : z;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            A[u][0] = ma == u ? v0 : z;
            A[u][1] = ma == u ? v1 : z;
        }
    }
    // the lane's epilogue groups: G = 4 ue + 2 hh + n of this wave
    float gsc[4], gsm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        gsc[q] = gmeta[w][4 * ue + q][0];
        gsm[q] = gmeta[w][4 * ue + q][1];
    }

    int pb = 0;
    float inv = 1.0f;
    bool first = true;
    float best = -INFINITY;  // greedy partial (wave 0, lanes < 16)
    int bi = 0x7fffffff;
    bool bad = false;
    for (int k = blockIdx.x; k < ntiles; k += gridDim.x) {
        const int t = tile_of(k);
        v4i D[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const v4i lo = (v4i)(nib[u] & 0x0f0f0f0fu);
            const v4i hi = (v4i)((nib[u] >> 4) & 0x0f0f0f0fu);
            D[0] = g1_mfma(A[u][0], lo, D[0]);
            D[1] = g1_mfma(A[u][1], hi, D[1]);
        }
        const v4u h = hl;
        const float d = f16_to_f32((uint16_t)(h.x & 0xffffu)), dm = f16_to_f32((uint16_t)(h.x >> 16));
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int dot = 256 * D[n][2 * hh] + D[n][2 * hh + 1];
                uint32_t sc, mn;
                q4k_dev_scale_min(h, 4 * (ue & 1) + 2 * hh + n, sc, mn);
                const int q = 2 * hh + n;
                acc += (d * (float)sc) * (gsc[q] * (float)dot) - (dm * (float)mn) * gsm[q];
            }
        const int next = k + gridDim.x;
        if (next < ntiles) load_tile(tile_of(next));
        if (R == 8) {
            // row r's four units sit on lanes (r, 0), (r, 2), (r + 8, 1),
            // (r + 8, 3): the others add zero
            acc = lane_valid ? acc : 0.0f;
            acc += __shfl_xor(acc, 8, 64);
        }
        acc += __shfl_xor(acc, 16, 64);
        acc += __shfl_xor(acc, 32, 64);
        if (lane < R) part[pb][w][j] = acc;
        lds_barrier();
        if (w == 0 && lane < R) {
            if ((PRO == PRO_RMS || PRO == PRO_EMBED_RMS) && first) {
                double tot = 0.0;
#pragma unroll
                for (int q = 0; q < W; ++q) tot += ssq[q];
                inv = rms_inv(tot, K, a.eps);
            }
            float v = 0.0f;
#pragma unroll
            for (int q = 0; q < W; ++q) v += part[pb][q][j];
            v *= inv;
            if (EPI == EPI_GLU) {
                const float up = __shfl_xor(v, 8, 16);
                const int o = t * 8 + j;
                if (j < 8 && o < nout) a.y[o] = up * ggml_silu(v);
            } else {
                const int o = t * R + j;
                if (EPI == EPI_STORE && a.gate_dt && o >= a.gate_row && o < a.gate_row + 2 * a.gate_heads) {
                    // the GDN gates from this output (alpha or the beta projection)
                    const int g = o - a.gate_row;
                    v = g < a.gate_heads ? gdn_gain(v, a.gate_dt[g], a.gate_a[g])
                                         : source_sigmoid(v);
                }
                if (o < nout) {
                    if (EPI == EPI_RESID && first) {
                        const float nv = ypre + v;  // source_binary Add, lib.rs:1258-1271
                        a.y[o] = nv;
                        if (!finite_f32(nv)) atomicOr(a.status, 1);
                    } else {
                        epilogue(a, 0, o, v, EPI);
                    }
                    if (EPI == EPI_STORE && a.amax) {
                        bad |= !finite_f32(v);
                        if (v > best || (v == best && o < bi)) {
                            best = v;
                            bi = o;
                        }
                    }
                }
            }
        }
        first = false;
        pb ^= 1;
    }
    if (EPI == EPI_STORE && a.amax && w == 0) {
        // lanes >= R hold (-inf, none): the first largest value of the
        // workgroup's outputs
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (ov > best || (ov == best && oi < bi)) {
                best = ov;
                bi = oi;
            }
        }
        if (bad) atomicOr(a.status, 4);
        if (lane == 0) {
            a.amax[blockIdx.x] = best;
            a.aidx[blockIdx.x] = bi;
        }
    }
}

// Rows per tile: 8 where 16-row tiles would leave more than half of the
// 256 CUs without a workgroup (the N = 2048 projections), else 16.
inline int gemv1_tile_rows(int nout, int epi) { return epi != EPI_GLU && nout <= 2048 ? 8 : 16; }

// Workgroups of launch_gemv1_q4k for N outputs.
inline int gemv1_grid(int nout, int epi) {
    const int tr = epi == EPI_GLU ? 8 : gemv1_tile_rows(nout, epi);
    return std::min((nout + tr - 1) / tr, 2048);
}

// Grid: one workgroup per tile up to 2048, the rest in further passes of
// the same workgroups (the activation coded once per workgroup).
template <int PRO, int EPI>
hipError_t launch_gemv1_q4k(const FusedGemvArgs& a, hipStream_t s) {
    if (a.M != 1 || a.K % 512 || a.K > kGemv1MaxK || (EPI == EPI_GLU && a.N % 2)) return hipErrorInvalidValue;
    if ((PRO == PRO_GATED || PRO == PRO_GATED_PRE) && a.group != 128) return hipErrorInvalidValue;
    const int nout = EPI == EPI_GLU ? a.N / 2 : a.N;
    const dim3 g((unsigned)gemv1_grid(nout, EPI));
    constexpr int R8 = EPI == EPI_GLU ? 16 : 8;  // (GLU tiles stay at 16 rows)
    const bool r8 = gemv1_tile_rows(nout, EPI) == 8;
#define ZG_G1(WV)                                                                           \
    if (r8)                                                                                 \
        hipLaunchKernelGGL((gemv1_q4k_kernel<WV, PRO, EPI, R8>), g, dim3(64 * WV), 0, s, a); \
    else                                                                                    \
        hipLaunchKernelGGL((gemv1_q4k_kernel<WV, PRO, EPI, 16>), g, dim3(64 * WV), 0, s, a)
    switch (a.K / 512) {
    case 1: ZG_G1(1); break;
    case 2: ZG_G1(2); break;
    case 3: ZG_G1(3); break;
    case 4: ZG_G1(4); break;
    case 5: ZG_G1(5); break;
    case 6: ZG_G1(6); break;
    case 7: ZG_G1(7); break;
    case 8: ZG_G1(8); break;
    case 12: ZG_G1(12); break;
    case 16: ZG_G1(16); break;
    default: return hipErrorInvalidValue;
    }
#undef ZG_G1
    return hipGetLastError();
}

}  // namespace zg
