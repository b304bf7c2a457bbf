// Prompt-sized projections (M >= kGemmRows rows): Y[m][n] (+)= sum_k X[m][k] W[n][k]
// with X the f16 activation tiles act16_kernel writes and W the Q4_K weight
// in MFMA tile order (ensure_mfma_tiles), dequantized in registers.
//
// Register-blocked on v_mfma_f32_32x32x16_f16: a workgroup of 4 waves, WN
// along N and 4/WN along M; each wave owns MT x NT output tiles of 32 x 32
// (MT*NT*16 accumulators).  The K loop walks 64-wide steps: the
// workgroup's AT = (4/WN)*MT activation tiles of a step (AT x 4 KB) are
// staged in LDS (two buffers, the next step's loads in flight during the
// MFMAs), each wave loads its NT weight tiles' nibbles (one 16-byte load
// per lane per tile) and dequantizes them once per step, so every
// dequantized B fragment feeds MT MFMAs and every A fragment read from LDS
// feeds NT.  The dequantization and the operand layouts are those of
// mfma_q4k_kernel (the decode path's batched GEMM); its f16 rounding of the
// weights and f32 accumulation make the result agree with the CPU's f32
// dot within the per-op tolerance.
#include <algorithm>

#include "zg_decode_common.hpp"

namespace zg {

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr float kF16Max = 65504.0f;

// Element (m, k) of the f16 A tiles for K columns: the act16_kernel layout.
__device__ __forceinline__ size_t a_tile_index(int m, int k, int K) {
    return ((((size_t)(m >> 5) * (K >> 8) + (k >> 8)) * 16 + ((k & 255) >> 4)) * 64 + ((k & 15) >> 3) * 32 +
            (m & 31)) * 8 + (k & 7);
}

template <int EPI, int MT, int NT, int WN, int WM>
__global__ __launch_bounds__(64 * WN * WM, 1) void gemm_q4k_kernel(FusedGemvArgs a, const _Float16* __restrict__ xh) {
    constexpr int AT = WM * MT, NTHR = 64 * WN * WM, APT = AT * 256 / NTHR;  // A slabs per thread
    static_assert(EPI != EPI_GLU || NT % 2 == 0, "SwiGLU pairs gate and up tiles");
    static_assert(AT * 256 % NTHR == 0, "whole activation slabs per thread");
    __shared__ h8v xs[2][AT * 256];  // AT tiles x 4 steps x 64 lanes of 16 bytes
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hsel = lane >> 5, r32 = lane & 31;
    const int wm = wv / WN, wn = wv - wm * WN;
    const int K = a.K, N = a.N, nbk = K >> 8;
    // split-K (residual projections with splits > 1): workgroup z takes the
    // z-th of S equal runs of 256-column blocks and writes its partial tile
    const int S = EPI == EPI_RESID && a.splits > 1 ? a.splits : 1, z = blockIdx.z;
    const int blk0 = z * nbk / S, blk1 = (z + 1) * nbk / S;
    const int nsub = 4 * blk1;  // one past this run's last 64-column step
    const int mtiles = (a.M + 31) >> 5;
    const int mt0 = blockIdx.y * AT;

    // this wave's weight tiles; with SwiGLU the first NT/2 are gate tiles and
    // the rest the up tiles N/64 later (rows j and N/2 + j pair up)
    constexpr int NW = EPI == EPI_GLU ? NT / 2 : NT;
    const int wtile0 = (blockIdx.x * WN + wn) * NW;
    int nbase[NT];
    bool nv[NT];
    uint32_t qoff[NT], hoff[NT];  // byte offsets of this lane's weight / header runs
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tile = EPI == EPI_GLU ? (t < NW ? wtile0 + t : wtile0 + t - NW + (N >> 6)) : wtile0 + t;
        nbase[t] = tile * 32;
        nv[t] = EPI == EPI_GLU ? (wtile0 + (t % NW)) * 32 + r32 < (N >> 1) : nbase[t] + r32 < N;
        const int tt = min(tile, (N - 1) >> 5);  // tiles past the end read the last one (results dropped)
        qoff[t] = ((uint32_t)tt * nbk * 256 + lane) * 16;
        hoff[t] = ((uint32_t)tt * nbk * 32 + r32) * 16;
    }
    // buffer resources sized to each operand (32-bit byte offsets: the host
    // refuses an operand of 4 GiB or more, prompt_gemm_bytes)
    const uint32_t ntl = (uint32_t)((N + 31) >> 5);
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.qs, 0, (int)(ntl * (uint32_t)nbk * 4096u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rh =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.hdr, 0, (int)(ntl * (uint32_t)nbk * 512u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)xh, 0, (int)((uint32_t)mtiles * (uint32_t)K * 64u), 0x00020000);
    // slab e (of AT*256) of a step: tile e/256, h8v e%256 of its 4-step run
    uint32_t aoff[APT];
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        const int e = tid + i * NTHR;
        const int mt = min(mt0 + e / 256, mtiles - 1);  // tiles past the end read the last one (results dropped)
        aoff[i] = ((uint32_t)mt * nbk * 16 * 64 + (e & 255)) * 16;
    }

    // Weights two steps ahead in a two-slot ring (slot = step parity), the
    // activation slab and the next block's headers one step / one block
    // ahead.  Requests past the end re-read the last step or block, so every
    // path issues the same loads and the compiler's load counting never
    // waits on a later request.  (Measured at the 2B shapes against one
    // step ahead: L=8192 model prefill 1% faster, L=2048 unchanged.)
    h8v ast[APT];
    v4u wq[2][NT], hc[NT], hn[NT];
    auto load_a = [&](int sb) {
        sb = min(sb, nsub - 1);
        const uint32_t astep = (uint32_t)((sb >> 2) * 16 + 4 * (sb & 3)) * 64 * 16;
#pragma unroll
        for (int i = 0; i < APT; ++i)
            ast[i] = __builtin_bit_cast(h8v, __builtin_amdgcn_raw_buffer_load_b128(rx, aoff[i] + astep, 0, 0));
    };
    auto load_w = [&](int sb, v4u (&dst)[NT]) {
        sb = min(sb, nsub - 1);
#pragma unroll
        for (int t = 0; t < NT; ++t) dst[t] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff[t] + (uint32_t)sb * 64 * 16, 0, 0);
    };
    auto load_h = [&](int blk, v4u (&dst)[NT]) {
        blk = min(blk, blk1 - 1);
#pragma unroll
        for (int t = 0; t < NT; ++t)
            dst[t] = __builtin_amdgcn_raw_buffer_load_b128(rh, hoff[t] + (uint32_t)blk * 32 * 16, 0, 0);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < APT; ++i) xs[buf][tid + i * NTHR] = ast[i];
    };

    f16v acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f16v{};

    load_a(4 * blk0);
    load_h(blk0, hc);
    load_w(4 * blk0, wq[0]);
    load_w(4 * blk0 + 1, wq[1]);
    store(0);
    __syncthreads();
    const h2v bias = h2v{(_Float16)1024.0f, (_Float16)1024.0f};
    for (int blk = blk0; blk < blk1; ++blk) {
        load_h(blk + 1, hn);
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            const int sb = 4 * blk + c4, cur = c4 & 1;
            load_a(sb + 1);
            // the two 32-groups of this step: scale and min rounded once to f16
            h2v sc[NT][2], nm[NT][2];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float d = f16_to_f32((uint16_t)(hc[t].x & 0xffffu));
                const float dmin = f16_to_f32((uint16_t)(hc[t].x >> 16));
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint32_t s, mn;
                    q4k_dev_scale_min(hc[t], 2 * c4 + h, s, mn);
                    const _Float16 sh = (_Float16)(d * (float)s), mh = (_Float16)(dmin * (float)mn);
                    sc[t][h] = h2v{sh, sh};
                    nm[t][h] = h2v{-mh, -mh};
                }
            }
            // each weight dword's low and high nibbles, masked once per step:
            // step j takes dwords (2 (j%2), 2 (j%2) + 1), low nibbles for j < 2
            uint32_t nib[NT][2][4];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint32_t wd[4] = {wq[cur][t].x, wq[cur][t].y, wq[cur][t].z, wq[cur][t].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    nib[t][0][q] = wd[q] & 0x0f0f0f0fu;
                    nib[t][1][q] = (wd[q] >> 4) & 0x0f0f0f0fu;
                }
            }
            load_w(sb + 2, wq[cur]);  // the slot is free once its nibbles are out
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h8v af[MT];
#pragma unroll
                for (int i = 0; i < MT; ++i) af[i] = xs[cur][(wm * MT + i) * 256 + j * 64 + lane];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    // step j: nibble half j/2 of the 8-byte piece j%2 (group 2*c4 + j/2)
                    const uint32_t w0 = nib[t][j >> 1][2 * (j & 1)], w1 = nib[t][j >> 1][2 * (j & 1) + 1];
                    // bytes (q, 0x64) pairs: the f16 bit patterns of 1024 + q
                    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
                    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
                    const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
                    const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
                    const h2v s2 = sc[t][j >> 1], n2 = nm[t][j >> 1];
                    const h2v e0 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p0) - bias, s2, n2);
                    const h2v e1 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p1) - bias, s2, n2);
                    const h2v e2 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p2) - bias, s2, n2);
                    const h2v e3 = __builtin_elementwise_fma(__builtin_bit_cast(h2v, p3) - bias, s2, n2);
                    // (a tile past N computes on a clamped copy; its columns are never stored)
                    const h8v wb = h8v{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
#pragma unroll
                    for (int i = 0; i < MT; ++i) acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], wb, acc[i][t], 0, 0, 0);
                }
            }
            store(cur ^ 1);  // (past the last step: a copy of it into the idle buffer)
            __syncthreads();
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) hc[t] = hn[t];
    }

    // D register r of tile (i, t) is row (r%4) + 8*(r/4) + 4*(lane/32) of the
    // activation tile, column lane%32 of the weight tile
    bool over = false;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int tile_m = mt0 + wm * MT + i;
        if (tile_m >= mtiles) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = tile_m * 32 + (r & 3) + 8 * (r >> 2) + 4 * hsel;
            if (EPI == EPI_GLU) {
#pragma unroll
                for (int t = 0; t < NW; ++t) {
                    if (!nv[t]) continue;
                    // up * silu(gate) in f32, rounded once to f16 into the down
                    // projection's A tiles (K = N/2 columns); a value past the
                    // f16 range raises status bit 4
                    const float v = m < a.M ? acc[i][t + NW][r] * ggml_silu(acc[i][t][r]) : 0.0f;
                    over |= !(fabsf(v) <= kF16Max);
                    ((_Float16*)a.xh_out)[a_tile_index(m, nbase[t] + r32, N >> 1)] = (_Float16)v;
                }
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (nv[t] && m < a.M) {
                        if (S > 1)
                            a.parts[((size_t)z * a.M + m) * N + nbase[t] + r32] = acc[i][t][r];
                        else
                            epilogue(a, m, nbase[t] + r32, acc[i][t][r], EPI);
                    }
            }
        }
    }
    if (EPI == EPI_GLU && over && a.status) atomicOr(a.status, 16);
}

// y[m][n] += (parts[0] + parts[1]) (+ parts[2] + parts[3]) at (m, n), the
// splits summed in order, float4 per thread; a non-finite sum raises status
// bit 1 as the residual epilogue does.
template <int S>
__global__ __launch_bounds__(256) void split_resid_kernel(FusedGemvArgs a) {
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x, n4 = (size_t)a.M * a.N / 4;
    if (i4 >= n4) return;
    const size_t e = 4 * i4, m = e / a.N, n = e % a.N, mn = (size_t)a.M * a.N;
    v4f p[S];
#pragma unroll
    for (int z = 0; z < S; ++z) p[z] = *(const v4f*)(a.parts + z * mn + e);
    float* yp = a.y + m * a.ldy + n;
    const v4f y = *(const v4f*)yp;
    v4f r;
    bool bad = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float acc = p[0][q];
#pragma unroll
        for (int z = 1; z < S; ++z) acc = acc + p[z][q];
        r[q] = y[q] + acc;
        bad |= !finite_f32(r[q]);
    }
    *(v4f*)yp = r;
    if (bad) atomicOr(a.status, 1);
}

}  // namespace

// Largest operand of the prompt GEMM in bytes: the f16 activation tiles
// (32 rows x K per tile), the 32-row weight tiles and their headers.  Every
// one must stay below 4 GiB (32-bit buffer offsets).
uint64_t prompt_gemm_bytes(size_t M, size_t K, size_t N) {
    const uint64_t mt = (M + 31) / 32, nt = (N + 31) / 32, nbk = K / 256;
    return std::max({mt * K * 64, nt * nbk * 4096, nt * nbk * 512});
}

bool prompt_gemm_supported(int type, size_t K, size_t N, int epi) {
    if (type != kQ4_K || K % 256 || K > 8192 || N == 0) return false;
    if (epi == EPI_GLU) return N % 64 == 0 && (N / 2) % 256 == 0;
    return true;
}

// Shapes: two weight tiles per wave (NT = 2), four waves along N, and the
// most activation tiles per wave (MT = 3, 2, 1) that still gives at least one
// workgroup per CU (256), else one.  Measured over M = 512, 2048, 8192 and
// the 2B-shaped projections (gate/up 12288 x 2048, GDN in 8224 x 2048, out
// 2048 x 2048, down 2048 x 6144): NT = 4 tiles with MT = 4 left a
// workgroup's 256 accumulators to one wave per SIMD and ran 1.3-1.6x
// slower (gate/up at M = 2048: 176 against 127 us); with NT = 2 the choice
// among MT = 1-4 and 2-8 waves moves the time by about 10%.
hipError_t prompt_gemm(const DeviceWeight& w, const FusedGemvArgs& args, const _Float16* xh, hipStream_t s) {
    if (!prompt_gemm_supported(w.type, w.K, w.N, args.epi) || !w.qs_t || !w.hdr_t || args.M <= 0)
        return hipErrorInvalidValue;
    if (args.epi == EPI_GLU && !args.xh_out) return hipErrorInvalidValue;
    if (prompt_gemm_bytes((size_t)args.M, w.K, w.N) >= ((uint64_t)1 << 32)) return hipErrorInvalidValue;
    FusedGemvArgs a = args;
    a.qs = w.qs_t;
    a.hdr = w.hdr_t;
    a.K = (int)w.K;
    a.N = (int)w.N;
    const int mtiles = (a.M + 31) / 32;
    const int ntiles = a.epi == EPI_GLU ? a.N / 64 : (a.N + 31) / 32;  // SwiGLU: gate/up tile pairs
    auto grid = [&](int mt, int nt, int wn, int wm) {
        const int nw = a.epi == EPI_GLU ? nt / 2 : nt;
        return dim3((unsigned)((ntiles + wn * nw - 1) / (wn * nw)), (unsigned)((mtiles + wm * mt - 1) / (wm * mt)));
    };
    auto count = [&](dim3 g) { return (long)g.x * g.y; };
#define ZG_GQ(E, MTV, NTV, WNV, WMV)                                                                                   \
    hipLaunchKernelGGL((gemm_q4k_kernel<E, MTV, NTV, WNV, WMV>), grid(MTV, NTV, WNV, WMV), dim3(64 * WNV * WMV), 0, s, \
                       a, xh)
#define ZG_GQE(E)                                                  \
    if (count(grid(3, 2, 4, 1)) >= 256) ZG_GQ(E, 3, 2, 4, 1);      \
    else if (count(grid(2, 2, 4, 1)) >= 256) ZG_GQ(E, 2, 2, 4, 1); \
    else ZG_GQ(E, 1, 2, 4, 1);
    // residual projections whose tiles give fewer than one 4-wave workgroup
    // per CU (or exactly one, for K >= 4096) split K in two or four runs of
    // 256-column blocks, and a second launch adds the runs into y: measured
    // at the 2B shapes, L=512 model prefill 7.58 -> 6.31 ms (four-way splits
    // where the tiles give at most 64 workgroups), L=2048 14.46 -> 14.28 ms
    const long c2 = count(grid(2, 2, 4, 1));
    int S = 1;
    if (a.epi == EPI_RESID && a.prompt_parts && a.N % 4 == 0 && a.ldy % 4 == 0) {
        if (c2 <= 64 && (a.K / 256) % 4 == 0) S = 4;
        else if ((c2 < 256 || (c2 == 256 && a.K >= 4096)) && (a.K / 256) % 2 == 0) S = 2;
    }
    if (S > 1 && (size_t)S * a.M * a.N > a.prompt_parts_n) S = 1;
    if (S > 1) {
        a.splits = S;
        a.parts = a.prompt_parts;
        dim3 g = grid(2, 2, 4, 1);
        g.z = (unsigned)S;
        hipLaunchKernelGGL((gemm_q4k_kernel<EPI_RESID, 2, 2, 4, 1>), g, dim3(256), 0, s, a, xh);
        const size_t n4 = (size_t)a.M * a.N / 4;
        if (S == 4) hipLaunchKernelGGL(split_resid_kernel<4>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, a);
        else hipLaunchKernelGGL(split_resid_kernel<2>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    a.splits = 0;
    if (a.epi == EPI_GLU) {
        ZG_GQE(EPI_GLU)
    } else if (a.epi == EPI_RESID) {
        ZG_GQE(EPI_RESID)
    } else {
        ZG_GQE(EPI_STORE)
    }
#undef ZG_GQE
#undef ZG_GQ
    return hipGetLastError();
}

}  // namespace zg
