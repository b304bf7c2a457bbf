// Batched-row decode projections on f16 MFMA (Q4_K from 2 rows up, in the
// session step and zg_gemv_device) and the prompt-sized GEMMs.
#include "zg_decode_common.hpp"

namespace zg {

// ============================================== batched rows: f16 MFMA

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

// One workgroup per activation row (rows M..Mpad-1 zero): the prologue
// values of wg_prologue, rounded once to f16, into xh in the A-operand order
// of the kernel that consumes them (xh_tile_index: 16-row tiles for decode
// batches, else 32-row tiles), so that each lane of the MFMA kernel loads 16
// contiguous bytes and a wave-instruction reads 1 KB contiguous.
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
            const size_t at = a.xh_rows ? (size_t)m * K + k : xh_tile_index(m, k, K, a.M);
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
                    a.rms_tiles_out[xh_tile_index(m, n, N, a.M)] = (_Float16)tv;
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
                    const int j = nbase[0] + r32;
                    const float pr = m < a.M ? v * ggml_silu(vg[i]) : 0.0f;
                    if (a.status && !(fabsf(pr) <= 65504.0f)) atomicOr(a.status, 16);
                    ((_Float16*)a.xh_out)[xh_tile_index(m, j, N >> 1, a.M)] = (_Float16)pr;
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

// ====================================== decode batches: Q4_K 16-row tiles
//
// Y[m][n] = sum_k X[m][k] W[n][k] for a decode batch (M < kGemmRows, K a
// multiple of 1024 up to 6144) on v_mfma_f32_16x16x32_f16, reading the
// weights in their Q4_K 16-row tile layout (q4k_chunk_offset) directly.
//
// Rows n are dealt to the workgroups in balanced runs of 16-row tiles,
// 16 MBW activation rows per workgroup (blockIdx.y), about 256 workgroups in
// all (one per CU).  Every CU must take in its whole 16 MBW x K activation
// block besides its share of the weights, so the CUs stream evenly and all
// of a workgroup's loads are issued before its first product; with few
// tiles (N/16 <= 256) a workgroup takes one 16-row half (MBW = 1): twice the
// workgroups, each taking in half the activations, and the two halves of a
// tile, gridDim.x workgroups apart, run on one XCD (dispatch deals
// workgroups to the 8 XCDs in turn), where the second read of the weights
// can hit L2.  Eight waves split K: wave w holds the A operands of units
// [w*UPW, (w+1)*UPW) (a unit is 128 columns) for its row halves in
// registers and multiplies them with every tile of its run.  For a unit, lane l of the weight operand
// takes the 16-byte piece (row l%16, half h = (l/16)&1, run 2u + l/32) of
// the 1 KB unit block (one contiguous wave load); its low and high nibbles,
// bytes 0-7 and 8-15, give the four 8-element B operands i = 2 nib + sub,
// dequantised on packed f16 as the 32-row kernel does (the nibble q becomes
// 1024 + q by a byte permute, 1024 is subtracted exactly, w = fma(q, scale,
// -min) with the group's scale and min rounded once to f16).  The A
// operands hold the same columns in the same lanes (xh16_index).  D
// register r of lane l is (m = 4 (l/16) + r, n = l%16).  The eight waves'
// partial tiles are summed in wave order through LDS.
//
// SwiGLU (EPI_GLU): a tile is 8 gate rows j and their 8 up rows N/2 + j
// (lanes l%16 < 8 and >= 8), so each output pairs lanes l and l ^ 8.
// Residual (EPI_RESID) with rms_tiles_out: as the 32-row kernel, with the
// sums of squares per 16-column tile (rms_ss_out[m][N/16]).
// TMAX tiles per pass.  LOOP 0: one pass; 1: passes over a longer run,
// each pass's weights requested after the previous pass; 2 (UPW <= 2): the
// next pass's weights requested before the current pass is multiplied.
constexpr int kM16Waves = 8;
// Tiles per pass that keep a wave's operands in registers (512 threads:
// 256 registers a lane); the A operands weigh UPW * MBW.
constexpr int m16_tiles_per_pass(int upw, int loop, int mbw) {
    const int ue = (upw * mbw + 1) / 2;
    return ue >= 5 || (loop == 1 && ue >= 3) ? 1 : (ue == 4 ? 2 : 3);
}

template <int EPI, int UPW, int LOOP, int MBW>
__global__ __launch_bounds__(64 * kM16Waves) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma16_q4k_kernel(
    FusedGemvArgs a, const h8v* __restrict__ xh) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    constexpr int KW = kM16Waves, VR = EPI == EPI_GLU ? 8 : 16;
    constexpr int TMAX = m16_tiles_per_pass(UPW, LOOP, MBW);
    // block headers: one per block when a wave's units pair into blocks
    // (UPW even: units 2b, 2b+1 of block b), else one per unit
    constexpr int NH = UPW % 2 == 0 ? UPW / 2 : UPW;
    static_assert(MBW * TMAX <= KW, "a finishing wave per (tile, row half)");
    __shared__ v4f red[KW][MBW * TMAX][64];
    __shared__ float inv_s[16 * MBW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, L = lane >> 4, r16 = lane & 15;
    const int K = a.K, N = a.N, nunits = K >> 7, nbk = K >> 8;
    const int nout = EPI == EPI_GLU ? N >> 1 : N, nvt = (nout + VR - 1) / VR;
    const int t0 = (int)((long long)blockIdx.x * nvt / gridDim.x);
    const int t1 = (int)((long long)(blockIdx.x + 1) * nvt / gridDim.x);
    const int m0 = 16 * MBW * blockIdx.y, ub = w * UPW, h = L & 1, cp = L >> 1;
    const uint8_t* qs = (const uint8_t*)a.qs;
    const v4u* hdr = (const v4u*)a.hdr;

    // ---- loads, in the order of use: the producer's per-tile sums of
    // squares (TPR threads per row, SSV each: 128 per row at most), the A
    // operands, the weights
    constexpr int TPR = 32 / MBW, SSV = 4 * MBW;
    double ssv[SSV];
    const int srow = tid / TPR, ssub = tid % TPR;
    auto reduce_ss = [&]() {  // (the first barrier of a pass orders inv_s)
        double tot = 0.0;
#pragma unroll
        for (int q = 0; q < SSV; ++q) tot += ssv[q];
        tot = group_sum_last<TPR>(tot);
        if (ssub == TPR - 1) inv_s[srow] = rms_inv(tot, K, a.eps);
    };
    if (a.rms_ss_in) {
        const int n = a.rms_ss_n;
        const double* ss = a.rms_ss_in + (size_t)(m0 + srow) * n;
#pragma unroll
        for (int q = 0; q < SSV; ++q) {
            const int c = ssub + TPR * q;
            const double x = ss[min(c, n - 1)];
            ssv[q] = c < n ? x : 0.0;
        }
        if (UPW * MBW >= 10) reduce_ss();  // wide units: before the main loads hold their registers
    }
    // lane l carries activation row m0 + 16 mb + l % 16 (xh16_index): rows
    // past M are the tiles' zero padding, so those lanes take zeros without
    // a load (a 2-row batch reads an eighth of the block)
    h8v xa[UPW][MBW][4];
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) {
        const bool live = m0 + 16 * mb + r16 < a.M;
#pragma unroll
        for (int u = 0; u < UPW; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xa[u][mb][i] = h8v{0, 0, 0, 0, 0, 0, 0, 0};
                if (live) xa[u][mb][i] = xh[(((size_t)(MBW * blockIdx.y + mb) * nunits + ub + u) * 4 + i) * 64 + lane];
            }
    }
    auto wrow = [&](int vt) {
        if (EPI == EPI_GLU) {
            const int j = min(vt * 8 + (r16 & 7), nout - 1);
            return r16 < 8 ? j : nout + j;
        }
        return vt * 16 + r16;  // < 16 * nvt: inside the zero-padded last tile
    };
    // weights and headers stream (read once per step): non-temporal loads
    // keep the activation block, which every workgroup re-reads, in L2
    auto issue = [&](v4u (&wq)[UPW][TMAX], v4u (&hd)[NH][TMAX], int tb) {
#pragma unroll
        for (int t = 0; t < TMAX; ++t) {
            if (tb + t < t1) {
                const int row = wrow(tb + t);
                const size_t tile = (size_t)(row >> 4);
#pragma unroll
                for (int u = 0; u < UPW; ++u) {
                    if (NH == UPW || u % 2 == 0)
                        hd[NH == UPW ? u : u / 2][t] = __builtin_nontemporal_load(hdr + (tile * nbk + ((ub + u) >> 1)) * 16 + (row & 15));
                    wq[u][t] = __builtin_nontemporal_load((const v4u*)(qs + ((tile * nunits + ub + u) * 64 + (row & 15) + 16 * h + 32 * cp) * 16));
                }
            }
        }
    };
    // a residual projection's own outputs, requested up front: wave w adds
    // into (tile t0 + w/MBW, row half w%MBW) -- the single-pass shapes
    float yv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, gn = 0.0f;
    const bool ypre = EPI == EPI_RESID && LOOP == 0 && w < MBW * min(TMAX, t1 - t0);
    if (ypre) {
        const int n = (t0 + w / MBW) * 16 + r16;
        if (n < N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 16 * (w % MBW) + 4 * L + r;
                if (m < a.M) yv[r] = a.y[(size_t)m * a.ldy + n];
            }
            if (a.rms_tiles_out) gn = a.rms_gamma[n];
        }
    }
    v4u wA[UPW][TMAX], hA[NH][TMAX];
    issue(wA, hA, t0);
    __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first product

    if (a.rms_ss_in && UPW * MBW < 10) reduce_ss();

    const h2v bias = h2v{(_Float16)1024.0f, (_Float16)1024.0f};
    auto pass = [&](const v4u (&wq)[UPW][TMAX], const v4u (&hd)[NH][TMAX], int tb) {
        const int ntb = min(TMAX, t1 - tb);
        v4f acc[TMAX][MBW];
#pragma unroll
        for (int t = 0; t < TMAX; ++t)
#pragma unroll
            for (int mb = 0; mb < MBW; ++mb) acc[t][mb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < UPW; ++u) {
            const int gl = 2 * (2 * ((ub + u) & 1) + cp);  // low-nibble group of the lane's run in its block
#pragma unroll
            for (int t = 0; t < TMAX; ++t) {
                if (t < ntb) {
                    const v4u hh = hd[NH == UPW ? u : u / 2][t];
                    const float d = f16_to_f32((uint16_t)(hh.x & 0xffffu));
                    const float dm = f16_to_f32((uint16_t)(hh.x >> 16));
                    h2v sc2[2], nm2[2];
#pragma unroll
                    for (int nib = 0; nib < 2; ++nib) {
                        uint32_t sc, mn;
                        q4k_dev_scale_min(hh, gl + nib, sc, mn);
                        const _Float16 sh = (_Float16)(d * (float)sc), mh = (_Float16)(dm * (float)mn);
                        sc2[nib] = h2v{sh, sh};
                        nm2[nib] = h2v{-mh, -mh};
                    }
                    const v4u q = wq[u][t];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int nib = i >> 1, sub = i & 1;
                        const uint32_t d0 = sub ? q.z : q.x, d1 = sub ? q.w : q.y;
                        const uint32_t w0 = (nib ? (d0 >> 4) : d0) & 0x0f0f0f0fu;
                        const uint32_t w1 = (nib ? (d1 >> 4) : d1) & 0x0f0f0f0fu;
                        // bytes (q, 0x64) pairs: the f16 bit patterns of 1024 + q
                        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
                        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
                        const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
                        const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
                        const h2v e0 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p0) - bias, sc2[nib], nm2[nib]);
                        const h2v e1 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p1) - bias, sc2[nib], nm2[nib]);
                        const h2v e2 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p2) - bias, sc2[nib], nm2[nib]);
                        const h2v e3 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p3) - bias, sc2[nib], nm2[nib]);
                        const h8v wb = h8v{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
#pragma unroll
                        for (int mb = 0; mb < MBW; ++mb)
                            acc[t][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u][mb][i], wb, acc[t][mb], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TMAX; ++t)
#pragma unroll
            for (int mb = 0; mb < MBW; ++mb) red[w][MBW * t + mb][lane] = acc[t][mb];
        __syncthreads();
        // wave w finishes (tile t = w/MBW, row half w%MBW)
        if (w < MBW * ntb) {
            v4f v = red[0][w][lane];
#pragma unroll
            for (int q = 1; q < KW; ++q) v = v + red[q][w][lane];
            const int vt = tb + w / MBW, mh = 16 * (w % MBW);
            float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (a.rms_ss_in) vv[r] *= inv_s[mh + 4 * L + r];
            if (EPI == EPI_GLU) {
                const int j = vt * 8 + (r16 & 7);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float up = __shfl_xor(vv[r], 8, 16);  // the up row's sum (lane l ^ 8)
                    const int m = m0 + mh + 4 * L + r;
                    if (r16 < 8 && j < nout) {
                        // up * silu(gate), rounded to f16 into the down
                        // projection's activation tiles (K2 = N/2 columns)
                        const float pr = m < a.M ? up * ggml_silu(vv[r]) : 0.0f;
                        if (a.status && !(fabsf(pr) <= 65504.0f)) atomicOr(a.status, 16);
                        ((_Float16*)a.xh_out)[xh_tile_index(m, j, nout, a.M)] = (_Float16)pr;
                    }
                }
            } else if (EPI == EPI_RESID) {
                const int n = vt * 16 + r16;
                const bool nv = n < N;
                float g = gn;
                if (!ypre && nv && a.rms_tiles_out) g = a.rms_gamma[n];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + mh + 4 * L + r;
                    const bool live = nv && m < a.M;
                    float xn = 0.0f;
                    if (live) {
                        float* p = a.y + (size_t)m * a.ldy + n;
                        xn = (ypre ? yv[r] : *p) + vv[r];  // source_binary Add, lib.rs:1258-1271
                        *p = xn;
                        if (!finite_f32(xn)) atomicOr(a.status, 1);
                    }
                    if (a.rms_tiles_out) {
                        // the next RMS projection's A tile element (m, n):
                        // f16(x_new * gamma) (its 1/rms is applied after its
                        // dot), and this 16-column tile's f64 sum of the f32
                        // squares of x_new (the 16 lanes of a row)
                        if (nv) {
                            const float tv = live ? xn * g : 0.0f;
                            if (!(fabsf(tv) <= 65504.0f)) atomicOr(a.status, 16);
                            a.rms_tiles_out[xh_tile_index(m, n, N, a.M)] = (_Float16)tv;
                        }
                        const float sq = xn * xn;
                        const double tot = group_sum_last<16>((double)sq);
                        if (r16 == 15) a.rms_ss_out[(size_t)m * (N >> 4) + vt] = tot;
                    }
                }
            } else {
                const int n = vt * 16 + r16;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + mh + 4 * L + r;
                    if (n < N && m < a.M) a.y[(size_t)m * a.ldy + n] = vv[r];
                }
            }
        }
        __syncthreads();
    };
    if constexpr (LOOP == 0) {
        pass(wA, hA, t0);
    } else if constexpr (LOOP == 1) {
        for (int tb = t0; tb < t1; tb += TMAX) {
            if (tb > t0) {
                issue(wA, hA, tb);
                __builtin_amdgcn_sched_barrier(0);
            }
            pass(wA, hA, tb);
        }
    } else if constexpr (LOOP == 2) {
        static_assert(UPW <= 2, "two weight buffers fit the registers up to UPW = 2");
        v4u wB[UPW][TMAX], hB[NH][TMAX];
        for (int tb = t0; tb < t1; tb += 2 * TMAX) {
            const int tb2 = tb + TMAX;
            issue(wB, hB, tb2);
            __builtin_amdgcn_sched_barrier(0);
            pass(wA, hA, tb);
            if (tb2 >= t1) break;
            issue(wA, hA, tb2 + TMAX);
            __builtin_amdgcn_sched_barrier(0);
            pass(wB, hB, tb2);
        }
    } else {
        // LOOP 3: three buffers, the next two passes' weights in flight
        // while one is multiplied (long runs: a 151936-row LM head)
        static_assert(UPW <= 2, "three weight buffers fit the registers up to UPW = 2");
        v4u wB[UPW][TMAX], hB[NH][TMAX], wC[UPW][TMAX], hC[NH][TMAX];
        issue(wB, hB, t0 + TMAX);
        for (int tb = t0; tb < t1; tb += 3 * TMAX) {
            issue(wC, hC, tb + 2 * TMAX);
            __builtin_amdgcn_sched_barrier(0);
            pass(wA, hA, tb);
            if (tb + TMAX >= t1) break;
            issue(wA, hA, tb + 3 * TMAX);
            __builtin_amdgcn_sched_barrier(0);
            pass(wB, hB, tb + TMAX);
            if (tb + 2 * TMAX >= t1) break;
            issue(wB, hB, tb + 4 * TMAX);
            __builtin_amdgcn_sched_barrier(0);
            pass(wC, hC, tb + 2 * TMAX);
        }
    }
}

bool batched16_supported(size_t M, size_t K, size_t N, int epi) {
    // every shape of the 16-row layout: producers write it whenever
    // xh16_layout(M, K) holds, so this kernel must take them all
    if (!xh16_layout(M, K) || N == 0 || N > (1u << 30)) return false;
    return epi != EPI_GLU || (N % 16 == 0 && (N / 2) % 128 == 0);
}

template <int EPI, int MBW>
static hipError_t launch_mfma16_m(const FusedGemvArgs& a, const _Float16* xh, hipStream_t s) {
    const int upw = a.K / 1024, nout = EPI == EPI_GLU ? a.N / 2 : a.N, vr = EPI == EPI_GLU ? 8 : 16;
    const int gy = (a.M + 16 * MBW - 1) / (16 * MBW);
    const int nvt = (nout + vr - 1) / vr, G = std::min(nvt, std::max(1, 256 / gy)), per = (nvt + G - 1) / G;
    const int tmax = m16_tiles_per_pass(upw, 0, MBW);
    // one pass; passes with the next one's weights in flight; with the next
    // two (four or more passes of a plain store: the residual and SwiGLU
    // epilogues leave no room for a third buffer); one buffer where two do
    // not fit (UPW > 2)
    const int loop = per <= tmax ? 0 : (upw <= 2 ? (per >= 4 * tmax && EPI == EPI_STORE ? 3 : 2) : 1);
    const dim3 g((unsigned)G, (unsigned)gy);
    const h8v* x = (const h8v*)xh;
#define ZG_M16(U)                                                                                                  \
    case U:                                                                                                        \
        if (loop == 0) {                                                                                           \
            hipLaunchKernelGGL((mfma16_q4k_kernel<EPI, U, 0, MBW>), g, dim3(64 * kM16Waves), 0, s, a, x);          \
        } else if (loop == 1) {                                                                                    \
            hipLaunchKernelGGL((mfma16_q4k_kernel<EPI, U, 1, MBW>), g, dim3(64 * kM16Waves), 0, s, a, x);          \
        } else if (loop == 2) {                                                                                    \
            if constexpr (U <= 2)                                                                                  \
                hipLaunchKernelGGL((mfma16_q4k_kernel<EPI, U, 2, MBW>), g, dim3(64 * kM16Waves), 0, s, a, x);      \
        } else {                                                                                                   \
            if constexpr (U <= 2 && EPI == EPI_STORE)                                                              \
                hipLaunchKernelGGL((mfma16_q4k_kernel<EPI, U, 3, MBW>), g, dim3(64 * kM16Waves), 0, s, a, x);      \
        }                                                                                                          \
        break;
    switch (upw) {
        ZG_M16(1)
        ZG_M16(2)
        ZG_M16(3)
        ZG_M16(4)
        ZG_M16(5)
        ZG_M16(6)
    default: return hipErrorInvalidValue;
    }
#undef ZG_M16
    return hipGetLastError();
}

// One 16-row half per workgroup when the rows are few (M <= 16) or the
// tiles are (N/16 <= 256: the whole-block workgroups would leave CUs idle).
template <int EPI>
static hipError_t launch_mfma16(const FusedGemvArgs& a, const _Float16* xh, hipStream_t s) {
    const int nvt = EPI == EPI_GLU ? (a.N / 2 + 7) / 8 : (a.N + 15) / 16;
    if (a.M <= 16 || nvt <= 256) return launch_mfma16_m<EPI, 1>(a, xh, s);
    return launch_mfma16_m<EPI, 2>(a, xh, s);
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

// Prompt-sized rows in the 32-row tile layout (plain or RMSNorm prologue, no
// pending split-K residual): four rows per workgroup, thread t taking row
// t % 4 and the 8-column groups t / 4 + 64 i, so that the four rows' 16-byte
// runs of a group sit side by side in the tiles and a wave's stores fill
// whole 64-byte spans (one row per workgroup scattered 16-byte stores 512
// bytes apart).  Same arithmetic as act16_kernel: f64 sum of the f32
// squares per row (in a fixed order), (x * inv) * gamma, f16.
template <int PRO, int NG>
__global__ __launch_bounds__(256) void act16_rows_kernel(FusedGemvArgs a, _Float16* __restrict__ xh) {
    __shared__ double red[4][4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, r = tid & 3, gi = tid >> 2;
    const int m = blockIdx.x * 4 + r, K = a.K;
    const bool valid = m < a.M;
    v4f v[NG][2], w[NG][2];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int k = 8 * (gi + 64 * i);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v[i][h] = valid ? *(const v4f*)(a.x + (size_t)m * a.ldx + k + 4 * h) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (PRO == PRO_RMS) w[i][h] = *(const v4f*)(a.gamma + k + 4 * h);
        }
    }
    float inv = 1.0f;
    if (PRO == PRO_RMS) {
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < NG; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float q = v[i][h][e] * v[i][h][e];
                    s += (double)q;
                }
        // the 16 lanes of this row in the wave (lane bits 2..5), then the waves
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) s += __shfl_xor(s, o, 64);
        if (lane < 4) red[wv][lane] = s;
        __syncthreads();
        inv = rms_inv((red[0][r] + red[1][r]) + (red[2][r] + red[3][r]), K, a.eps);
    }
    bool over = false;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int k = 8 * (gi + 64 * i);
        typedef _Float16 h8v_ __attribute__((ext_vector_type(8)));
        h8v_ o8;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y = v[i][h][e];
                if (PRO == PRO_RMS) y = (y * inv) * w[i][h][e];
                over |= valid && !(fabsf(y) <= 65504.0f);
                o8[4 * h + e] = valid ? (_Float16)y : (_Float16)0.0f;
            }
        *(h8v_*)(xh + xh_tile_index(m, k, K, a.M)) = o8;
    }
    // past the f16 range: status bit 4 (the f32 paths carry it)
    if (over && a.status) atomicOr(a.status, 16);
}

template <int PRO>
static void launch_act16(const FusedGemvArgs& a, int mpad, _Float16* xh, hipStream_t s) {
    if ((PRO == PRO_RMS || PRO == PRO_PLAIN) && !a.xh_rows && a.rsplits <= 0 && !xh16_layout(a.M, a.K) &&
        a.K % 512 == 0) {
        switch (a.K / 512) {
        case 2: hipLaunchKernelGGL((act16_rows_kernel<PRO, 2>), dim3(mpad / 4), dim3(256), 0, s, a, xh); return;
        case 4: hipLaunchKernelGGL((act16_rows_kernel<PRO, 4>), dim3(mpad / 4), dim3(256), 0, s, a, xh); return;
        case 8: hipLaunchKernelGGL((act16_rows_kernel<PRO, 8>), dim3(mpad / 4), dim3(256), 0, s, a, xh); return;
        case 12: hipLaunchKernelGGL((act16_rows_kernel<PRO, 12>), dim3(mpad / 4), dim3(256), 0, s, a, xh); return;
        default: break;
        }
    }
    if (a.K <= 1024) hipLaunchKernelGGL((act16_kernel<PRO, 1>), dim3(mpad), dim3(256), 0, s, a, xh);
    else if (a.K <= 2048) hipLaunchKernelGGL((act16_kernel<PRO, 2>), dim3(mpad), dim3(256), 0, s, a, xh);
    else if (a.K <= 4096) hipLaunchKernelGGL((act16_kernel<PRO, 4>), dim3(mpad), dim3(256), 0, s, a, xh);
    else hipLaunchKernelGGL((act16_kernel<PRO, 8>), dim3(mpad), dim3(256), 0, s, a, xh);
}

hipError_t batched_gemv(const DeviceWeight& w, const FusedGemvArgs& args, void* scratch, hipStream_t s) {
    if (w.type == kQ8_0) return q8_rows_gemv(w, args, scratch, s);
    if (w.type == kQ6_K) return q6k_rows_gemv(w, args, scratch, s);
    if (w.type != kQ4_K || w.K % 256 || w.K > 8192 || args.M <= 0 || args.M > 65535 * 32) return hipErrorInvalidValue;
    if (args.pro == PRO_GATED && args.group != 128) return hipErrorInvalidValue;
    const bool m16 = batched16_supported((size_t)args.M, w.K, w.N, args.epi);
    if (!m16 && (!w.qs_t || !w.hdr_t)) return hipErrorNotReady;  // ensure_mfma_tiles first
    FusedGemvArgs a = args;
    a.qs = m16 ? w.qs : w.qs_t;  // the 16-row kernel reads the Q4_K tile layout itself
    a.hdr = m16 ? w.hdr : w.hdr_t;
    a.K = (int)w.K;
    a.N = (int)w.N;
    if (m16) {  // no split-K; the sums of squares fit 8 per thread
        if ((a.epi == EPI_RESID && a.splits > 1 && a.parts) || (a.rms_ss_in && a.rms_ss_n > 128) ||
            (a.rms_tiles_out && (a.epi != EPI_RESID || a.N % 128)) || (a.epi == EPI_GLU && !a.xh_out))
            return hipErrorInvalidValue;
    }
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
    if (m16) {
        switch (a.epi) {
        case EPI_GLU: return launch_mfma16<EPI_GLU>(a, xh, s);
        case EPI_RESID: return launch_mfma16<EPI_RESID>(a, xh, s);
        default: return launch_mfma16<EPI_STORE>(a, xh, s);
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
