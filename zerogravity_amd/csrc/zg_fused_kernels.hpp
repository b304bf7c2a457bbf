#pragma once
// Kernels of the fused decode GEMV (one launch per projection at B <= 4:
// the codecs other than Q4_K, and Q4_K at 2-4 rows through
// zg_gemv_device_fused; one Q4_K row takes the int8 GEMV, and 2+ Q4_K rows
// of zg_gemv_device and the session step the batched f16 kernels)
// and their launch templates; zg_fused_<prologue>.hip instantiate one
// prologue each so that the instantiations compile in parallel.
#include "zg_decode_common.hpp"
#include "zg_gemv1.hpp"

namespace zg {

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
                const uint8_t* base = qs + q4k_chunk_offset(row, c, K);
                w0[r][i] = load_nt(base);
                w1[r][i] = load_nt(base + 256);
                h[r][i] = hdr[q4k_hdr_index(row, c >> 2, nbk)];
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
    const int nb = K >> 5, nbc = (nb + 3) >> 2, nbp = nbc * 4, nbs = nbp + 4;
    int* codes = lds_f8;                                 // [MT][8][nbs] words (wg_prologue's Q8_0 layout)
    float* scales = (float*)(lds_f8 + MT * 8 * nbs);   // [MT][nbp]
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
                cw[m] = *(const v4i*)(codes + (size_t)(m * 8 + l) * nbs + 4 * c);
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
        wg_prologue<PRO, kCodecQ8, J>(a, m0 + m, m0 + m < a.M, nullptr, codes + (size_t)m * 8 * nbs,
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
    const int nb = K >> 5, nbc8 = (nb + 7) >> 3, nb8 = nbc8 * 8, nbs8 = nb8 + 4;
    int* codes = lds_f41;                                // [MT][8][nbs8] words (wg_prologue's Q8_1 layout)
    float* scales = (float*)(lds_f41 + MT * 8 * nbs8);   // [MT][nb8]
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
                const v4i* cp = (const v4i*)(codes + (size_t)(m * 8 + l) * nbs8 + 8 * c);
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
        wg_prologue<PRO, kCodecQ81, J>(a, m0 + m, m0 + m < a.M, nullptr, codes + (size_t)m * 8 * nbs8,
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
// STAGED: the MT activation rows come already coded (q6k_act_rows_kernel,
// the same prologue function) from a.staged, one row per ms + nsb + K/16
// words in the LDS layout below, instead of being coded per workgroup.
template <int MT, int J, int PRO, int EPI, bool STAGED = false>
__global__ __launch_bounds__(256) void fused_q6k_kernel(FusedGemvArgs a) {
    // superblocks stream in chunks of QS through two register buffers, the
    // next chunk's loads issued before the current one is consumed;
    // activation row 0's loads go out first and its coding overlaps the
    // first chunk's (a wave's loads complete in issue order).  Loads are
    // unconditional: a superblock past the row end reads the last one and
    // is not consumed.
    constexpr int QS = 4;
    extern __shared__ int lds_f6[];
    const int K = a.K, N = a.N, nsb = K >> 8, ls = (K >> 5) + 4, ms = 8 * ls;
    int* codes = lds_f6;                                 // [MT][8][K/32 + 4] words (wg_prologue's Q8_K layout)
    float* dk = (float*)(lds_f6 + MT * ms);              // [MT][nsb]
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
                const int* cl = codes + m * ms + (size_t)l * ls + sb * 8;
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
    const int R0 = blockIdx.x * 4 + (threadIdx.x >> 6);
    Chunk ca, cb;
    if constexpr (STAGED) {
        // the first chunk's weights go out first, then the rows' copy (rows
        // past M zero); the copy's words keep the LDS layout, so a row is
        // one contiguous run of rw words
        load_chunk(R0, 0, ca);
        const int rw = ms + nsb + (K >> 4);
        for (int i = threadIdx.x; i < MT * rw; i += blockDim.x) {
            const int m = i / rw, o = i - m * rw;
            const int v = m0 + m < a.M ? a.staged[(size_t)(m0 + m) * rw + o] : 0;
            if (o < ms) codes[m * ms + o] = v;
            else if (o < ms + nsb) ((int*)dk)[m * nsb + o - ms] = v;
            else bs[m * (K >> 4) + o - ms - nsb] = v;
        }
        __syncthreads();
    } else {
        ProIn<J> pin;
        wg_prologue_load<PRO, J>(a, m0, m0 < a.M, pin);
        load_chunk(R0, 0, ca);
        wg_prologue_code<PRO, kCodecQ8K, J>(a, m0 < a.M, pin, nullptr, codes, nullptr, dk, bs);
#pragma unroll
        for (int m = 1; m < MT; ++m)
            wg_prologue<PRO, kCodecQ8K, J>(a, m0 + m, m0 + m < a.M, nullptr, codes + m * ms, nullptr,
                                           dk + m * nsb, bs + m * (K >> 4));
    }
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
hipError_t launch_codec(const FusedGemvArgs& a, int type, hipStream_t s) {
    const int K = a.K;
    const int mt = type == kF32 ? 1 : (a.M == 1 ? 1 : (a.M == 2 ? 2 : 4));
    size_t per;
    // codes 8 words per block (lane rows padded by 4 words) + scale + sum per block
    if (type == kQ4_1) per = (size_t)(8 * ((K / 32 + 7) / 8 * 8 + 4) + 2 * ((K / 32 + 7) / 8 * 8)) * 4;
    else if (type == kQ6_K) per = (size_t)8 * (K / 32 + 4) * 4 + (size_t)(K / 256) * 4 + (size_t)(K / 16) * 4;
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
hipError_t launch_q4k(const FusedGemvArgs& a, hipStream_t s) {
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
hipError_t launch_q8(const FusedGemvArgs& a, hipStream_t s) {
    const int K = a.K;
    int mt = a.M == 1 ? 1 : (a.M == 2 ? 2 : 4);
    // codes 8 words per block (rows padded by 4 words) + a scale per block
    auto lds = [&](int t) { return (size_t)t * (8 * ((K / 32 + 3) / 4 * 4 + 4) + (K / 32 + 3) / 4 * 4) * 4; };
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

// One activation row of a Q4_K weight with K a multiple of 512 (K / 512 of
// 1..8, 12, 16) runs on the int8 matrix cores (zg_gemv1.hpp).
inline bool gemv1_fits(const FusedGemvArgs& a, int type) {
    const int wv = a.K / 512;
    return type == kQ4_K && a.M == 1 && a.K % 512 == 0 && (wv <= 8 || wv == 12 || wv == 16) &&
           ((a.pro != PRO_GATED && a.pro != PRO_GATED_PRE) || a.group == 128) && (a.epi != EPI_GLU || a.N % 2 == 0);
}

template <int PRO>
hipError_t launch_pro(const FusedGemvArgs& a, int type, hipStream_t s) {
    if constexpr (PRO == PRO_RMS) {
        if (a.emb_qs) {  // the activation is an embedding row (matrix-core GEMV only)
            if (!gemv1_fits(a, type) || a.epi != EPI_STORE) return hipErrorInvalidValue;
            return launch_gemv1_q4k<PRO_EMBED_RMS, EPI_STORE>(a, s);
        }
    }
    if (gemv1_fits(a, type)) {
        if (a.epi == EPI_GLU) {
            if constexpr (PRO == PRO_RMS) return launch_gemv1_q4k<PRO_RMS, EPI_GLU>(a, s);
            return hipErrorInvalidValue;
        }
        return a.epi == EPI_RESID ? launch_gemv1_q4k<PRO, EPI_RESID>(a, s) : launch_gemv1_q4k<PRO, EPI_STORE>(a, s);
    }
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

}  // namespace zg
