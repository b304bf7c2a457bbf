// Q8_0 projections of more than 4 activation rows: the weights streamed
// once for up to 16 rows per workgroup.
//
// Arithmetic (cpu/src/source/quantization.rs:171-196, as gemv_q8_0_kernel
// and fused_q8_kernel restate it): per (activation row m, output row n)
// eight f32 accumulators; accumulator l takes, block after block, the int32
// dot of block elements 4l..4l+3 with the activation codes, fused-multiply-
// added with scale = f16(w.d) * act.d, and the value is the tree
// ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)).  Lane (r8, l) of a wave is
// accumulator l of weight row 8 g + r8 for each of its R row groups g and
// each of the MT activation rows, so the per-(m, n) chain and the final
// tree are the reference's: bit-identical to the one-to-four-row kernels.
//
// Two launches.  q8_act_rows_kernel codes every activation row once (one
// workgroup per row, the fused kernels' own prologue function, so the codes
// and scales are theirs) into the prepared layout of act_prepare_for: int8
// codes [M][K], then per block the f16-rounded scale [M][K/32] at the next
// 256-byte boundary.  q8_rows_kernel stages MT rows of it into LDS (word l
// of block b at (m * 8 + l) * nbs + b, nbs = nbp + 4 so that the 8 words of
// a block fall in different banks: one 16-byte read gives a lane four
// blocks of its word) and streams its row groups' weight tiles through two
// register buffers, the next QC chunks requested before the current ones
// are multiplied.  Every activation word read from LDS serves R weight rows
// and every weight word MT activation rows: the fused kernels read all the
// weights again for each group of four rows.  q8_mfma_kernel forms the same
// per-word dots on the int8 matrix cores (below); launch_rows picks one of
// the two by shape.
//
// Q6_K beyond 4 rows takes the same two-launch form: q6k_act_rows_kernel
// codes each row once to Q8_K (the prologue function the fused Q6_K kernel
// runs per workgroup), and fused_q6k_kernel in its staged mode copies up to
// 16 coded rows per workgroup instead of coding them, so one weight stream
// serves them all with the kernel's own per-row arithmetic.
#include <type_traits>

#include "zg_fused_kernels.hpp"

namespace zg {

namespace {

constexpr int kQ8RowsQC = 2;  // 4-block chunks per register buffer

template <int PRO, int J>
__global__ __launch_bounds__(256) void q8_act_rows_kernel(FusedGemvArgs a, int8_t* __restrict__ aq,
                                                          float* __restrict__ ad) {
    extern __shared__ int lds_q8a[];
    const int K = a.K, nb = K >> 5, nbp = (nb + 3) & ~3, nbs = nbp + 4;
    int* codes = lds_q8a;                         // [8][nbs] words, the prologue's layout
    float* scales = (float*)(lds_q8a + 8 * nbs);  // [nbp]
    const int m = blockIdx.x;
    wg_prologue<PRO, kCodecQ8, J>(a, m, true, nullptr, codes, scales);  // ends with a barrier
    int* out = (int*)(aq + (size_t)m * K);
    for (int wd = threadIdx.x; wd < (K >> 2); wd += blockDim.x) out[wd] = codes[(wd & 7) * nbs + (wd >> 3)];
    for (int b = threadIdx.x; b < nb; b += blockDim.x) ad[(size_t)m * nb + b] = scales[b];
}

template <int MT, int R, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void q8_rows_kernel(
    FusedGemvArgs a, const int8_t* __restrict__ aq, const float* __restrict__ ad) {
    constexpr int QC = kQ8RowsQC;
    extern __shared__ int lds_q8r[];
    const int K = a.K, N = a.N, M = a.M;
    const int nb = K >> 5, nbc = (nb + 3) >> 2, nbp = nbc * 4, nbs = nbp + 4, kw = K >> 2;
    int* codes = lds_q8r;                               // [MT][8][nbs] words
    float* scales = (float*)(lds_q8r + MT * 8 * nbs);   // [MT][nbp]
    const int m0 = blockIdx.y * MT;
    const int lane = threadIdx.x & 63, r8 = lane >> 3, l = lane & 7;
    const int groups = (N + 7) >> 3, tasks = (groups + R - 1) / R;
    const int nwaves = gridDim.x * 4;
    const v4i* qs = (const v4i*)a.qs;
    const uint16_t* hdr = (const uint16_t*)a.hdr;

    struct Chunk {
        v4i w[QC][R];
        uint2 h[QC][R];
    };
    // row groups past the end re-read the last group, blocks past the end
    // the last chunk: loaded, never consumed
    auto load = [&](int T, int c0, Chunk& ck) {
#pragma unroll
        for (int q = 0; q < QC; ++q) {
            const int c = min(c0 + q, nbc - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int g = min(T * R + r, groups - 1);
                const int row = min(g * 8 + r8, N - 1);
                ck.w[q][r] = load_nt(qs + ((size_t)g * nbc + c) * 64 + lane);
                ck.h[q][r] = *(const uint2*)(hdr + (size_t)row * nbp + 4 * c);
            }
        }
    };
    const int T0 = blockIdx.x * 4 + (threadIdx.x >> 6);
    Chunk ca, cb;
    if (T0 < tasks) load(T0, 0, ca);
    __builtin_amdgcn_sched_barrier(0);

    // ---- stage the MT activation rows (zero past M) into LDS
    const int nq = MT * (kw >> 2);  // 16-byte pieces: words 4p .. 4p+3 of a row (one block half)
    for (int p = threadIdx.x; p < nq; p += blockDim.x) {
        const int m = p / (kw >> 2), wd = 4 * (p - m * (kw >> 2));
        v4i v = {0, 0, 0, 0};
        if (m0 + m < M) v = *(const v4i*)(aq + (size_t)(m0 + m) * K + 4 * wd);
        const int b = wd >> 3, l0 = wd & 7;
        int* dst = codes + (m * 8 + l0) * nbs + b;
        dst[0] = v.x;
        dst[nbs] = v.y;
        dst[2 * nbs] = v.z;
        dst[3 * nbs] = v.w;
    }
    for (int i = threadIdx.x; i < MT * nbp; i += blockDim.x) {
        const int m = i / nbp, b = i - m * nbp;
        scales[i] = (m0 + m < M && b < nb) ? ad[(size_t)(m0 + m) * nb + b] : 0.0f;
    }
    __syncthreads();

    float acc[R][MT];
    auto consume = [&](const Chunk& ck, int c0) {
#pragma unroll
        for (int q = 0; q < QC; ++q) {
            const int c = c0 + q;
            if (c >= nbc) break;  // uniform
            float wd[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wd[r][0] = f16_to_f32((uint16_t)(ck.h[q][r].x & 0xffffu));
                wd[r][1] = f16_to_f32((uint16_t)(ck.h[q][r].x >> 16));
                wd[r][2] = f16_to_f32((uint16_t)(ck.h[q][r].y & 0xffffu));
                wd[r][3] = f16_to_f32((uint16_t)(ck.h[q][r].y >> 16));
            }
            // a whole chunk runs unguarded; only a last chunk past nb checks
            // each block (uniform)
            const int nbi = min(4, nb - 4 * c);
            auto blocks = [&](auto full) {
                // row m + 1's codes and scales are requested before row m's
                // products, so the LDS latency hides behind them
                v4i cwn = *(const v4i*)(codes + l * nbs + 4 * c);
                v4f swn = *(const v4f*)(scales + 4 * c);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const v4i cw = cwn;
                    const v4f sw = swn;
                    if (m + 1 < MT) {
                        cwn = *(const v4i*)(codes + ((m + 1) * 8 + l) * nbs + 4 * c);
                        swn = *(const v4f*)(scales + (m + 1) * nbp + 4 * c);
                    }
                    const int xc[4] = {cw.x, cw.y, cw.z, cw.w};
                    const float xs[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
                    for (int bi = 0; bi < 4; ++bi) {
                        if (decltype(full)::value || bi < nbi) {
#pragma unroll
                            for (int r = 0; r < R; ++r) {
                                const int ww = bi == 0 ? ck.w[q][r].x
                                             : bi == 1 ? ck.w[q][r].y
                                             : bi == 2 ? ck.w[q][r].z
                                                       : ck.w[q][r].w;
                                const int pair = __builtin_amdgcn_sdot4(ww, xc[bi], 0, false);
                                const float scale = wd[r][bi] * xs[bi];
                                acc[r][m] = fmaf((float)pair, scale, acc[r][m]);
                            }
                        }
                    }
                }
            };
            if (nbi == 4) blocks(std::true_type{});
            else blocks(std::false_type{});
        }
    };

    for (int T = T0; T < tasks; T += nwaves) {
        if (T != T0) load(T, 0, ca);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
        for (int c0 = 0; c0 < nbc; c0 += 2 * QC) {
            if (c0 + QC < nbc) load(T, c0 + QC, cb);
            consume(ca, c0);
            if (c0 + QC >= nbc) break;
            if (c0 + 2 * QC < nbc) load(T, c0 + 2 * QC, ca);
            consume(cb, c0 + QC);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int g = T * R + r, row = g * 8 + r8;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float v = group8_tree_last(acc[r][m]);  // the reference's lane tree, in lane 7
                if (l == 7 && g < groups && row < N && m0 + m < M) epilogue(a, m0 + m, row, v, EPI);
            }
        }
    }
}

// The same products on the int8 matrix cores (v_mfma_i32_16x16x32_i8, one
// Q8_0 block per instruction).  A: row i = 8 mm + l is word l of activation
// row 2 p + mm (pair p): its codes at k = 4l .. 4l+3 and zeros elsewhere,
// so D[i][j] is exactly the int32 dot of word l with output row j's word l,
// the reference's per-lane dot.  B: lane (j, kq) holds the block's words
// 2kq and 2kq+1 of output row n0 + j; in the tile layout those are two
// adjacent 16-byte pieces carrying the chunk's four blocks (one 32-byte
// load, the tile's chunk read whole by the wave).  D: lane (j, kq) holds
// rows 4kq .. 4kq+3, i.e. activation row 2p + kq/2 and words
// l = 4(kq & 1) .. +3, which share one scale wd[n][b] * xs[m][b]: one
// product per four fmas instead of one per fma.  After the last block,
// lanes kq and kq ^ 1 (16 apart) add words l and l + 4, and the even lane
// forms ((s0 + s2) + (s1 + s3)): the reference's tree, so the result is
// q8_rows_kernel's bit for bit.
template <int MP, int R, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void q8_mfma_kernel(
    FusedGemvArgs a, const int8_t* __restrict__ aq, const float* __restrict__ ad) {
    constexpr int MT = 2 * MP;
    extern __shared__ int lds_q8m[];
    const int K = a.K, N = a.N, M = a.M;
    const int nb = K >> 5, nbc = (nb + 3) >> 2, nbp = nbc * 4, nbs = nbp + 4, kw = K >> 2;
    int* codes = lds_q8m;                              // [MT][8][nbs] words
    float* scales = (float*)(lds_q8m + MT * 8 * nbs);  // [MT][nbp]
    const int m0 = blockIdx.y * MT;
    const int lane = threadIdx.x & 63, j = lane & 15, kq = lane >> 4;
    const int tiles = (N + 15) >> 4, tasks = (tiles + R - 1) / R;
    const int nwaves = gridDim.x * 4;
    const v4i* qs = (const v4i*)a.qs;
    const uint16_t* hdr = (const uint16_t*)a.hdr;

    struct Chunk {
        v4i w0[R], w1[R];
        uint2 h[R];
    };
    // rows past N re-read row N - 1, chunks past the end the last one:
    // loaded, never consumed
    auto load = [&](int T, int c, Chunk& ck) {
        c = min(c, nbc - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(min(T * R + r, tiles - 1) * 16 + j, N - 1);
            const v4i* p = qs + ((size_t)(n >> 3) * nbc + c) * 64 + (n & 7) * 8 + 2 * kq;
            ck.w0[r] = load_nt(p);
            ck.w1[r] = load_nt(p + 1);
            ck.h[r] = *(const uint2*)(hdr + (size_t)n * nbp + 4 * c);
        }
    };
    const int T0 = blockIdx.x * 4 + (threadIdx.x >> 6);
    Chunk ca, cb;
    if (T0 < tasks) load(T0, 0, ca);
    __builtin_amdgcn_sched_barrier(0);

    // ---- stage the MT activation rows (zero past M) into LDS
    const int nq = MT * (kw >> 2);
    for (int p = threadIdx.x; p < nq; p += blockDim.x) {
        const int m = p / (kw >> 2), wd = 4 * (p - m * (kw >> 2));
        v4i v = {0, 0, 0, 0};
        if (m0 + m < M) v = *(const v4i*)(aq + (size_t)(m0 + m) * K + 4 * wd);
        const int b = wd >> 3, l0 = wd & 7;
        int* dst = codes + (m * 8 + l0) * nbs + b;
        dst[0] = v.x;
        dst[nbs] = v.y;
        dst[2 * nbs] = v.z;
        dst[3 * nbs] = v.w;
    }
    for (int i = threadIdx.x; i < MT * nbp; i += blockDim.x) {
        const int m = i / nbp, b = i - m * nbp;
        scales[i] = (m0 + m < M && b < nb) ? ad[(size_t)(m0 + m) * nb + b] : 0.0f;
    }
    __syncthreads();

    const int l = j & 7, mm = j >> 3;  // this lane's A row: word l of activation row 2p + mm
    const bool lo = l == 2 * kq, hi = l == 2 * kq + 1;
    float acc[MP][R][4];
    auto consume = [&](const Chunk& ck, int c) {
        const int nbi = min(4, nb - 4 * c);
        float wd[R][4];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wd[r][0] = f16_to_f32((uint16_t)(ck.h[r].x & 0xffffu));
            wd[r][1] = f16_to_f32((uint16_t)(ck.h[r].x >> 16));
            wd[r][2] = f16_to_f32((uint16_t)(ck.h[r].y & 0xffffu));
            wd[r][3] = f16_to_f32((uint16_t)(ck.h[r].y >> 16));
        }
        auto blocks = [&](auto full) {
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const v4i xv = *(const v4i*)(codes + ((2 * p + mm) * 8 + l) * nbs + 4 * c);
                const v4f sv = *(const v4f*)(scales + (2 * p + (kq >> 1)) * nbp + 4 * c);
                const int xw[4] = {xv.x, xv.y, xv.z, xv.w};
                const float xs[4] = {sv.x, sv.y, sv.z, sv.w};
                // the pair's four blocks go to the matrix cores together,
                // then their products join the chains in block order
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    v4i d[4];
#pragma unroll
                    for (int bi = 0; bi < 4; ++bi) {
                        if (decltype(full)::value || bi < nbi) {
                            const long av = (long)(uint64_t)(lo ? (uint32_t)xw[bi] : 0u) |
                                            (long)((uint64_t)(hi ? (uint32_t)xw[bi] : 0u) << 32);
                            const int w0 = bi == 0 ? ck.w0[r].x : bi == 1 ? ck.w0[r].y : bi == 2 ? ck.w0[r].z
                                                                                                : ck.w0[r].w;
                            const int w1 = bi == 0 ? ck.w1[r].x : bi == 1 ? ck.w1[r].y : bi == 2 ? ck.w1[r].z
                                                                                                : ck.w1[r].w;
                            const long bv = (long)(uint64_t)(uint32_t)w0 | (long)((uint64_t)(uint32_t)w1 << 32);
                            d[bi] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, v4i{0, 0, 0, 0}, 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int bi = 0; bi < 4; ++bi) {
                        if (decltype(full)::value || bi < nbi) {
                            const float scale = wd[r][bi] * xs[bi];
                            acc[p][r][0] = fmaf((float)d[bi].x, scale, acc[p][r][0]);
                            acc[p][r][1] = fmaf((float)d[bi].y, scale, acc[p][r][1]);
                            acc[p][r][2] = fmaf((float)d[bi].z, scale, acc[p][r][2]);
                            acc[p][r][3] = fmaf((float)d[bi].w, scale, acc[p][r][3]);
                        }
                    }
                }
            }
        };
        if (nbi == 4) blocks(std::true_type{});
        else blocks(std::false_type{});
    };

    for (int T = T0; T < tasks; T += nwaves) {
        if (T != T0) load(T, 0, ca);
#pragma unroll
        for (int p = 0; p < MP; ++p)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[p][r][t] = 0.0f;
        for (int c = 0; c < nbc; c += 2) {
            if (c + 1 < nbc) load(T, c + 1, cb);
            consume(ca, c);
            if (c + 1 >= nbc) break;
            if (c + 2 < nbc) load(T, c + 2, ca);
            consume(cb, c + 1);
        }
#pragma unroll
        for (int p = 0; p < MP; ++p)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) s[t] = acc[p][r][t] + __shfl_xor(acc[p][r][t], 16, 64);  // l + (l + 4)
                const float v = (s[0] + s[2]) + (s[1] + s[3]);
                const int tile = T * R + r, n = tile * 16 + j, m = m0 + 2 * p + (kq >> 1);
                if (!(kq & 1) && tile < tiles && n < N && m < M) epilogue(a, m, n, v, EPI);
            }
    }
}

size_t rows_lds(int mt, int K) {
    const int nbp = ((K >> 5) + 3) & ~3;
    return (size_t)mt * (8 * (nbp + 4) + nbp) * 4;  // 8 code words (padded rows) and a scale per block
}

template <int EPI>
hipError_t launch_valu_rows(const FusedGemvArgs& a, const int8_t* aq, const float* ad, hipStream_t s) {
    const int M = a.M, K = a.K;
    const size_t groups = ((size_t)a.N + 7) / 8;
    // R row groups per wave while the waves stay plentiful: an activation
    // word read from LDS then serves R weight rows
    int R = groups >= 4 * 4096 ? 4 : (groups >= 2 * 2048 ? 2 : 1);
    // MT activation rows per workgroup: as many as M needs up to 16, within
    // 64 KB of LDS (two workgroups per CU), and fewer when the row groups
    // alone would leave CUs idle (more workgroups along M, each re-reading
    // the weights from cache)
    int mt = 16;
    auto wgs_of = [&](int r) { return (unsigned)std::min<size_t>(((groups + r - 1) / r + 3) / 4, 1024); };
    while (mt > 4 && mt / 2 >= M) mt >>= 1;
    while (mt > 4 && rows_lds(mt, K) > 65536) mt >>= 1;
    while (mt > 4 && (size_t)wgs_of(mt == 16 ? std::min(R, 2) : R) * ((M + mt - 1) / mt) < 256) mt >>= 1;
    if (mt == 16) R = std::min(R, 2);
    const unsigned wgs = wgs_of(R);
    if (rows_lds(mt, K) > 65536) return hipErrorInvalidValue;
    const unsigned gy = (unsigned)((M + mt - 1) / mt);
    if (gy > 65535) return hipErrorInvalidValue;
    const dim3 g(wgs, gy);
    const size_t lds = rows_lds(mt, K);
#define ZG_Q8R(MT_, R_) hipLaunchKernelGGL((q8_rows_kernel<MT_, R_, EPI>), g, dim3(256), lds, s, a, aq, ad)
#define ZG_Q8R_R(MT_)              \
    if (R == 4) ZG_Q8R(MT_, 4);    \
    else if (R == 2) ZG_Q8R(MT_, 2); \
    else ZG_Q8R(MT_, 1);
    if (mt == 16) {
        // 16 activation rows with four row groups per wave spill registers:
        // two groups
        if (R >= 2) ZG_Q8R(16, 2);
        else ZG_Q8R(16, 1);
    } else if (mt == 8) {
        ZG_Q8R_R(8)
    } else {
        ZG_Q8R_R(4)
    }
#undef ZG_Q8R_R
#undef ZG_Q8R
    return hipGetLastError();
}

template <int EPI>
hipError_t launch_mfma_rows(const FusedGemvArgs& a, const int8_t* aq, const float* ad, hipStream_t s) {
    const int M = a.M, K = a.K;
    const size_t tiles = ((size_t)a.N + 15) / 16;
    // R 16-row tiles per wave task while the waves stay plentiful
    const int R = tiles >= 2 * 4096 ? 2 : 1;
    const unsigned wgs = (unsigned)std::min<size_t>(((tiles + R - 1) / R + 3) / 4, 1024);
    // MT activation rows per workgroup: as many as M needs up to 16, within
    // 64 KB of LDS (two workgroups per CU), and fewer when the tiles alone
    // would leave CUs idle (more workgroups along M, each re-reading the
    // weights from cache)
    int mt = 16;
    while (mt > 4 && mt / 2 >= M) mt >>= 1;
    while (mt > 4 && rows_lds(mt, K) > 65536) mt >>= 1;
    while (mt > 4 && (size_t)wgs * ((M + mt - 1) / mt) < 256) mt >>= 1;
    if (rows_lds(mt, K) > 65536) return hipErrorInvalidValue;
    const unsigned gy = (unsigned)((M + mt - 1) / mt);
    if (gy > 65535) return hipErrorInvalidValue;
    const dim3 g(wgs, gy);
    const size_t lds = rows_lds(mt, K);
#define ZG_Q8M(MP_, R_) hipLaunchKernelGGL((q8_mfma_kernel<MP_, R_, EPI>), g, dim3(256), lds, s, a, aq, ad)
#define ZG_Q8M_R(MP_)               \
    if (R == 2) ZG_Q8M(MP_, 2);     \
    else ZG_Q8M(MP_, 1);
    if (mt == 16) {
        ZG_Q8M_R(8)
    } else if (mt == 8) {
        ZG_Q8M_R(4)
    } else {
        ZG_Q8M_R(2)
    }
#undef ZG_Q8M_R
#undef ZG_Q8M
    return hipGetLastError();
}

// The matrix-core kernel takes 16-row tiles per wave task, the VALU kernel
// 8-row groups: with few tiles the VALU kernel keeps twice the waves busy,
// and with many rows or many tiles the matrix cores' cheaper products win
// (measured per shape: the 2B-shaped projections and the LM head at 8, 16
// and 32 rows).
template <int EPI>
hipError_t launch_rows(const FusedGemvArgs& a, const int8_t* aq, const float* ad, hipStream_t s) {
    const size_t tiles = ((size_t)a.N + 15) / 16;
    const bool mfma = tiles >= 512 || (a.M >= 16 && tiles >= 256) || (a.M >= 32 && tiles >= 128);
    return mfma ? launch_mfma_rows<EPI>(a, aq, ad, s) : launch_valu_rows<EPI>(a, aq, ad, s);
}

template <int PRO>
hipError_t launch_act_rows(const FusedGemvArgs& a, int8_t* aq, float* ad, hipStream_t s) {
    const int K = a.K, nbp = ((K >> 5) + 3) & ~3;
    const size_t lds = (size_t)(8 * (nbp + 4) + nbp) * 4;
    const dim3 g((unsigned)a.M);
#define ZG_Q8A(J) hipLaunchKernelGGL((q8_act_rows_kernel<PRO, J>), g, dim3(256), lds, s, a, aq, ad)
    if (K <= 1024) ZG_Q8A(1);
    else if (K <= 2048) ZG_Q8A(2);
    else if (K <= 4096) ZG_Q8A(4);
    else ZG_Q8A(8);
#undef ZG_Q8A
    return hipGetLastError();
}

// One row of the Q8_K coding per workgroup: codes (lane rows padded), the
// per-256 scales and the 16-element code sums, contiguous in the fused
// Q6_K kernel's LDS order (its staged copy is one run of words per row).
template <int PRO, int J>
__global__ __launch_bounds__(256) void q6k_act_rows_kernel(FusedGemvArgs a, int* __restrict__ out) {
    extern __shared__ int lds_q6a[];
    const int K = a.K, nsb = K >> 8, ms = 8 * ((K >> 5) + 4), rw = ms + nsb + (K >> 4);
    const int m = blockIdx.x;
    wg_prologue<PRO, kCodecQ8K, J>(a, m, true, nullptr, lds_q6a, nullptr, (float*)(lds_q6a + ms),
                                   lds_q6a + ms + nsb);  // ends with a barrier
    int* o = out + (size_t)m * rw;
    for (int i = threadIdx.x; i < rw; i += blockDim.x) o[i] = lds_q6a[i];
}

size_t q6k_row_bytes(int K) { return (size_t)(8 * ((K >> 5) + 4) + (K >> 8) + (K >> 4)) * 4; }

template <int EPI>
hipError_t launch_q6k_rows(const FusedGemvArgs& a, hipStream_t s) {
    const int M = a.M, K = a.K;
    const size_t groups = ((size_t)a.N + 7) / 8;
    const unsigned wgs = (unsigned)std::min<size_t>((groups + 3) / 4, 256 * 8);
    // up to 16 rows per workgroup within 64 KB of LDS, fewer when the row
    // groups alone would leave CUs idle
    int mt = 16;
    while (mt > 4 && mt / 2 >= M) mt >>= 1;
    while (mt > 4 && q6k_row_bytes(K) * mt > 65536) mt >>= 1;
    while (mt > 4 && (size_t)wgs * ((M + mt - 1) / mt) < 256) mt >>= 1;
    if (q6k_row_bytes(K) * mt > 65536) return hipErrorInvalidValue;
    const unsigned gy = (unsigned)((M + mt - 1) / mt);
    if (gy > 65535) return hipErrorInvalidValue;
    const dim3 g(wgs, gy);
    const size_t lds = q6k_row_bytes(K) * mt;
    if (mt == 16) hipLaunchKernelGGL((fused_q6k_kernel<16, 1, PRO_PLAIN, EPI, true>), g, dim3(256), lds, s, a);
    else if (mt == 8) hipLaunchKernelGGL((fused_q6k_kernel<8, 1, PRO_PLAIN, EPI, true>), g, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((fused_q6k_kernel<4, 1, PRO_PLAIN, EPI, true>), g, dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int PRO>
hipError_t launch_q6k_act_rows(const FusedGemvArgs& a, int* out, hipStream_t s) {
    const int K = a.K;
    const dim3 g((unsigned)a.M);
    const size_t lds = q6k_row_bytes(K);
#define ZG_Q6A(J) hipLaunchKernelGGL((q6k_act_rows_kernel<PRO, J>), g, dim3(256), lds, s, a, out)
    if (K <= 1024) ZG_Q6A(1);
    else if (K <= 2048) ZG_Q6A(2);
    else if (K <= 4096) ZG_Q6A(4);
    else ZG_Q6A(8);
#undef ZG_Q6A
    return hipGetLastError();
}

}  // namespace

bool q8_rows_supported(size_t K, size_t N, int pro) {
    return pro != PRO_GATED_PRE && fused_gemv_supported(kQ8_0, K, N, pro) && rows_lds(4, (int)K) <= 65536;
}

hipError_t q8_rows_gemv(const DeviceWeight& w, const FusedGemvArgs& args, void* scratch, hipStream_t s) {
    if (w.type != kQ8_0 || !q8_rows_supported(w.K, w.N, args.pro) || args.M <= 0 || !scratch ||
        (args.epi != EPI_STORE && args.epi != EPI_RESID) || args.xh_in || args.xh_out || args.rparts ||
        (args.parts && args.splits > 1) || args.rms_tiles_out || args.rms_ss_in || args.amax || args.emb_qs ||
        args.gate_dt)
        return hipErrorInvalidValue;
    if (args.pro == PRO_GATED && (args.group <= 0 || args.group > 1024 || (args.group & (args.group - 1)) ||
                                  w.K % (size_t)args.group))
        return hipErrorInvalidValue;
    FusedGemvArgs a = args;
    a.qs = w.qs;
    a.hdr = w.hdr;
    a.K = (int)w.K;
    a.N = (int)w.N;
    int8_t* aq = (int8_t*)scratch;
    float* ad = (float*)((char*)scratch + (((size_t)a.M * w.K + 255) & ~(size_t)255));
    hipError_t e;
    switch (a.pro) {
    case PRO_RMS: e = launch_act_rows<PRO_RMS>(a, aq, ad, s); break;
    case PRO_GATED: e = launch_act_rows<PRO_GATED>(a, aq, ad, s); break;
    case PRO_SILU_MUL: e = launch_act_rows<PRO_SILU_MUL>(a, aq, ad, s); break;
    case PRO_PLAIN: e = launch_act_rows<PRO_PLAIN>(a, aq, ad, s); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    return a.epi == EPI_RESID ? launch_rows<EPI_RESID>(a, aq, ad, s) : launch_rows<EPI_STORE>(a, aq, ad, s);
}

hipError_t q8_rows_prepared(const DeviceWeight& w, size_t M, const void* prepared, float* y, hipStream_t s) {
    if (w.type != kQ8_0 || !q8_rows_supported(w.K, w.N, PRO_PLAIN) || M == 0 || M > (size_t)65535 * 4)
        return hipErrorInvalidValue;
    FusedGemvArgs a;
    a.qs = w.qs;
    a.hdr = w.hdr;
    a.K = (int)w.K;
    a.N = (int)w.N;
    a.M = (int)M;
    a.epi = EPI_STORE;
    a.y = y;
    a.ldy = w.N;
    const int8_t* aq = (const int8_t*)prepared;
    const float* ad = (const float*)((const char*)prepared + ((M * w.K + 255) & ~(size_t)255));
    return launch_rows<EPI_STORE>(a, aq, ad, s);
}

bool q6k_rows_supported(size_t K, size_t N, int pro) {
    return pro != PRO_GATED_PRE && fused_gemv_supported(kQ6_K, K, N, pro) && q6k_row_bytes((int)K) * 4 <= 65536;
}

hipError_t q6k_rows_gemv(const DeviceWeight& w, const FusedGemvArgs& args, void* scratch, hipStream_t s) {
    if (w.type != kQ6_K || !q6k_rows_supported(w.K, w.N, args.pro) || args.M <= 0 || !scratch ||
        (args.epi != EPI_STORE && args.epi != EPI_RESID) || args.xh_in || args.xh_out || args.rparts ||
        (args.parts && args.splits > 1) || args.rms_tiles_out || args.rms_ss_in || args.amax || args.emb_qs ||
        args.gate_dt)
        return hipErrorInvalidValue;
    if (args.pro == PRO_GATED && (args.group <= 0 || args.group > 1024 || (args.group & (args.group - 1)) ||
                                  w.K % (size_t)args.group))
        return hipErrorInvalidValue;
    FusedGemvArgs a = args;
    a.qs = w.qs;
    a.hdr = w.hdr;
    a.K = (int)w.K;
    a.N = (int)w.N;
    int* st = (int*)scratch;
    hipError_t e;
    switch (a.pro) {
    case PRO_RMS: e = launch_q6k_act_rows<PRO_RMS>(a, st, s); break;
    case PRO_GATED: e = launch_q6k_act_rows<PRO_GATED>(a, st, s); break;
    case PRO_SILU_MUL: e = launch_q6k_act_rows<PRO_SILU_MUL>(a, st, s); break;
    case PRO_PLAIN: e = launch_q6k_act_rows<PRO_PLAIN>(a, st, s); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    a.staged = st;
    return a.epi == EPI_RESID ? launch_q6k_rows<EPI_RESID>(a, s) : launch_q6k_rows<EPI_STORE>(a, s);
}

}  // namespace zg
