// Chunked Gated DeltaNet prefill (WY/UT form) for gfx950.
//
// Reference: the chunk algorithm of
// cpu/src/numerics/torch_cpu/gdn/chunk/core.rs:152-363 (solve order of
// gdn/chunk.rs:16-76, products of chunk/core.rs:367-400), per chunk of C
// tokens and per head, with key-major state S [k][v]:
//   q, k  <- two-stage L2 (q additionally * 1/sqrt(d))
//   g     =  cumsum(log decay) (f64 running sum, f32 per token)
//   A     =  (beta k) k^T  .* Gamma,   intra = q k^T .* Gamma,
//            Gamma[t][s] = exp(g_t - g_s) for s <= t, else 0
//   U     =  solve(I + tril(A, -1), beta v)
//   W     =  solve(I + tril(A, -1), (beta k) .* exp(g))
//   corr  =  U - W S
//   o     =  intra corr + (q .* exp(g)) S
//   S     <- (k .* exp(g_last - g))^T corr + exp(g_last) S
//
// Four launches.  gdn_chunk_prep_kernel runs every (chunk, head) in
// parallel: normalisation, gates, A and intra on f32 MFMA (16x16x4), dq, dk
// and exp(g_last), into a record per (chunk, head); gdn_chunk_solve_kernel
// solves for U and W, one column per thread in the reference's summation
// order.  gdn_chunk_scan_kernel carries the state through the chunks
// in order, one workgroup per (head, 16-column value slab) since the value
// columns of S evolve independently: per chunk only W S, corr = U - W S and
// the state update, storing corr and the state entering the chunk.
// gdn_chunk_out_kernel then forms o = intra corr + dq S for every (chunk,
// head) in parallel.
//
// Every product is a single v_mfma_f32_16x16x4f32 accumulator chain over k
// in increasing order; the instruction accumulates its four products as a
// chain of fused multiply-adds, so each output equals the reference's FMA
// chain (chunk/core.rs:277-310) bit for bit.
#include <algorithm>
#include <atomic>

#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

namespace {

constexpr int kC = 64, kD = 128, kSW = 16;  // chunk rows, head width, scan slab width
constexpr int kPad = 132;                   // LDS row pitch (floats) of [rows][128] tiles
constexpr int kApad = 68;                   // LDS row pitch of [64][64] tiles
typedef float f4m __attribute__((ext_vector_type(4)));

// Record per (chunk, head), floats.  W first holds the solve's right-hand
// side (beta k) exp(g); U is overwritten in place by corr in the scan; A is
// the decayed (beta k) k^T (strictly lower part used); S holds the state
// entering the chunk, key-major [k][v].
constexpr size_t kOffU = 0, kOffW = kOffU + kC * kD, kOffDq = kOffW + kC * kD, kOffDk = kOffDq + kC * kD,
                 kOffIntra = kOffDk + kC * kD, kOffA = kOffIntra + kC * kC, kOffDecay = kOffA + kC * kC,
                 kOffS = kOffDecay + 64, kRec = kOffS + kD * kD;

__device__ __forceinline__ f4m mfma4(float a, float b, f4m c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Both products of a lower 16x16 tile over K = kD, (beta k) k^T and q k^T,
// as two interleaved MFMA chains (rows of 128 in LDS with pitch kPad).
// Lane l supplies row i0 + l%16 of beta k and q and row j0 + l%16 of k at
// column 4s + l/16; result register r is (i0 + 4(l/16) + r, j0 + l%16).
// Operands are read into registers first so that the chains do not wait on
// LDS between steps.
__device__ __forceinline__ void tile_pair(const float* Q, const float* K, int i0, int j0, int lane, float brow,
                                          f4m& a4, f4m& q4) {
    const float* kr = K + (i0 + (lane & 15)) * kPad + (lane >> 4);
    const float* qr = Q + (i0 + (lane & 15)) * kPad + (lane >> 4);
    const float* yr = K + (j0 + (lane & 15)) * kPad + (lane >> 4);
    float ka[kD / 4], qa[kD / 4], yb[kD / 4];
#pragma unroll
    for (int s = 0; s < kD / 4; ++s) {
        ka[s] = kr[4 * s] * brow;
        qa[s] = qr[4 * s];
        yb[s] = yr[4 * s];
    }
    __builtin_amdgcn_sched_barrier(0);
    a4 = f4m{0.0f, 0.0f, 0.0f, 0.0f};
    q4 = a4;
#pragma unroll
    for (int s = 0; s < kD / 4; ++s) {
        a4 = mfma4(ka[s], yb[s], a4);
        q4 = mfma4(qa[s], yb[s], q4);
    }
}

}  // namespace

// Grid (chunks, H), 256 threads: everything of a (chunk, head) but the
// solves.  LDS: q and k rows, 68 KB.
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ logd, int T, int H,
                                                             float* __restrict__ scratch) {
    __shared__ float qs[kC * kPad];
    __shared__ float ks[kC * kPad];
    __shared__ float gs[kC], bs[kC], eg[kC], el[kC], lg[kC];
    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = c * kC, rows = min(kC, T - t0);
    float* rec = scratch + ((size_t)c * H + h) * kRec;
    const float inv_sqrt = 1.0f / sqrtf((float)kD);
    const float eps = 1e-6f / (float)kD;

    // Two-stage L2 of q and k rows (forward.rs:564-576): sum of f32 squares
    // in f64, mean rounded to f32, f32 sqrt and reciprocal; q also carries
    // the output scale.  Thread (row tid/4, quarter tid%4) holds 32 elements
    // of the row of q and of k; zero rows past the last token.
    {
        const int t = tid >> 2, d0 = 32 * (tid & 3);
        v4f xq[8], xk[8];
        const size_t src = ((size_t)(t0 + t) * H + h) * kD + d0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xq[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            xk[i] = xq[i];
            if (t < rows) {
                xq[i] = *(const v4f*)(q + src + 4 * i);
                xk[i] = *(const v4f*)(k + src + 4 * i);
            }
        }
        if (tid < kC) {
            const bool in = tid < rows;
            bs[tid] = in ? beta[(size_t)(t0 + tid) * H + h] : 0.0f;
            lg[tid] = in ? logd[(size_t)(t0 + tid) * H + h] : 0.0f;
        }
        double sq = 0.0, sk = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a2 = xq[i][e] * xq[i][e], b2 = xk[i][e] * xk[i][e];
                sq += (double)a2;
                sk += (double)b2;
            }
        sq = wave_sum_xor<double>(sq, 4);
        sk = wave_sum_xor<double>(sk, 4);
        const float iq = 1.0f / sqrtf((float)(sq * (1.0 / kD)) + eps);
        const float ik = 1.0f / sqrtf((float)(sk * (1.0 / kD)) + eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v4f a, b;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float tq = xq[i][e] * iq;
                const float nq = tq * inv_sqrt;
                a[e] = nq * inv_sqrt;
                const float tk = xk[i][e] * ik;
                b[e] = tk * inv_sqrt;
            }
            *(v4f*)&qs[t * kPad + d0 + 4 * i] = a;
            *(v4f*)&ks[t * kPad + d0 + 4 * i] = b;
        }
    }
    __syncthreads();
    // g = cumsum(log decay) in f64 (chunk/core.rs:135-150; padded rows add 0)
    if (tid == 0) {
        float l[kC];
#pragma unroll
        for (int t = 0; t < kC; ++t) l[t] = lg[t];
        double running = 0.0;
#pragma unroll
        for (int t = 0; t < kC; ++t) {
            running += (double)l[t];
            gs[t] = (float)running;
        }
    }
    __syncthreads();

    // A = (beta k) k^T and intra = q k^T, decayed by exp(g_t - g_s) on and
    // below the diagonal (0 * the product above it within the diagonal
    // tiles, as the reference's exp(-inf) factor gives).  Neither is read
    // above the diagonal tiles (the solve reads A strictly below the
    // diagonal, the output kernel's intra chains stop at each row tile's
    // diagonal), so those tiles are neither formed nor written.  Lower tile
    // pairs go round-robin over the waves.
    if (tid < kC) {
        const float last = gs[kC - 1];
        eg[tid] = cr_expf(gs[tid]);
        el[tid] = cr_expf(last - gs[tid]);
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        const int n = wv + 4 * m;
        if (n >= 10) break;
        const int ti = n < 1 ? 0 : n < 3 ? 1 : n < 6 ? 2 : 3;
        const int tj = n - ti * (ti + 1) / 2;
        const int i0 = 16 * ti, j0 = 16 * tj;
        const float brow = bs[i0 + (lane & 15)];
        f4m a4, q4;
        tile_pair(qs, ks, i0, j0, lane, brow, a4, q4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = i0 + 4 * (lane >> 4) + r, s2 = j0 + (lane & 15);
            const float decay = s2 <= t ? cr_expf(gs[t] - gs[s2]) : 0.0f;
            rec[kOffA + t * kC + s2] = a4[r] * decay;
            rec[kOffIntra + t * kC + s2] = q4[r] * decay;
        }
    }
    __syncthreads();
    // dq = q exp(g), dk = k exp(g_last - g), and the W right-hand side
    // (beta k) exp(g)
#pragma unroll
    for (int i = 0; i < kC * kD / 4 / 256; ++i) {
        const int f = tid + 256 * i, t = f >> 5, d = 4 * (f & 31);
        const v4f qv = *(const v4f*)&qs[t * kPad + d], kv = *(const v4f*)&ks[t * kPad + d];
        *(v4f*)(rec + kOffDq + t * kD + d) = qv * eg[t];
        *(v4f*)(rec + kOffDk + t * kD + d) = kv * el[t];
        *(v4f*)(rec + kOffW + t * kD + d) = (kv * bs[t]) * eg[t];
    }
    if (tid < 64) rec[kOffDecay + tid] = cr_expf(gs[kC - 1]);  // replicated for vector loads
}

// Grid (chunks, H, 2), 128 threads: the unit-lower solves of gdn/chunk.rs:16-76
// (separate products, four interleaved partial sums, (s0+s2)+(s1+s3), scalar
// tail, one subtraction) for the 128 columns of U (z = 0, rhs beta v) or of
// W (z = 1, rhs in place), one column per thread, held in registers.  The
// coefficients are uniform across the wave and are read as scalar loads
// through `amat` (the same records, never written here).
__global__ __launch_bounds__(128) void gdn_chunk_solve_kernel(const float* __restrict__ v,
                                                              const float* __restrict__ beta,
                                                              const float* __restrict__ amat, int T, int H,
                                                              float* __restrict__ scratch) {
    // A is staged in LDS and read there as broadcast 16-byte reads: read
    // from memory as scalar loads its 2016 coefficients outgrew the scalar
    // registers, and the compiler parked them in vector-register lanes
    // (a write and a read instruction per coefficient)
    __shared__ float As[kC * kC];
    const int c = blockIdx.x, h = blockIdx.y, z = blockIdx.z;
    const int col = threadIdx.x;
    const int t0 = c * kC, rows = min(kC, T - t0);
    float* rec = scratch + ((size_t)c * H + h) * kRec;
    const float* A = amat + ((size_t)c * H + h) * kRec + kOffA;
#pragma unroll
    for (int i = 0; i < kC * kC / (4 * 128); ++i)
        *(v4f*)(As + 4 * (col + 128 * i)) = *(const v4f*)(A + 4 * (col + 128 * i));
    __syncthreads();
    float xr[kC];
    if (z == 0) {
#pragma unroll
        for (int t = 0; t < kC; ++t) {
            float r = 0.0f;
            if (t < rows) {
                const float vv = v[((size_t)(t0 + t) * H + h) * kD + col];
                r = vv * beta[(size_t)(t0 + t) * H + h];
            }
            xr[t] = r;
        }
    } else {
#pragma unroll
        for (int t = 0; t < kC; ++t) xr[t] = rec[kOffW + t * kD + col];
    }
#pragma unroll
    for (int row = 0; row < kC; ++row) {
        const int vend = row / 4 * 4;
        const float* arow = As + row * kC;
        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < vend; st += 4) {
            const v4f a4 = *(const v4f*)(arow + st);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const float p = a4[l] * xr[st + l];
                s4[l] = s4[l] + p;
            }
        }
        float sum = (s4[0] + s4[2]) + (s4[1] + s4[3]);
#pragma unroll
        for (int kk = vend; kk < row; ++kk) {
            const float p = arow[kk] * xr[kk];
            sum = sum + p;
        }
        xr[row] = xr[row] - sum;
        // the next row's coefficients are read only once the row before this
        // one is solved (the asm takes that value and orders the LDS reads):
        // hoisted further, the reads held most of A in registers
        if (row >= 1) asm volatile("" ::"v"(xr[row - 1]) : "memory");
    }
    float* dst = rec + (z == 0 ? kOffU : kOffW);
#pragma unroll
    for (int t = 0; t < kC; ++t) dst[t * kD + col] = xr[t];
}

// Grid (H, kD / kSW), 512 threads: value columns [16 slab, 16 slab + 16) of
// head h through all chunks in order (every slab of a head on one XCD, whose
// L2 then serves the shared W and dk).  The state is held key-major S[k][j]
// in LDS; in memory it is value-major [h][v][k] (the decode layout) or, with
// key_major, [h][k][v] (the chunk reference's layout).  Per chunk the four
// compute waves store the entering state, form pred = W S, corr = U - pred
// (written over U), then S <- dk^T corr + exp(g_last) S, reading W, dk, the
// U slab and the decay from LDS.  The four loader waves stage those: at
// chunk c they write chunk c + 1's operands (requested two chunks earlier,
// held in registers) into the LDS buffer chunk c - 1 used while the compute
// waves form corr, and request chunk c + 3's while they update the state,
// so no compute wave waits on global memory.  (Measured at 8192 tokens:
// 2.9 us per chunk with the old one-wave-group form, whose end-of-chunk
// wait covered the next chunk's loads and its own stores; 2.2 us here.)
__global__ __launch_bounds__(512) void gdn_chunk_scan_kernel(float* __restrict__ scratch, int T, int H,
                                                             float* __restrict__ state, int key_major) {
    __shared__ float S[kD][kSW + 1];
    __shared__ float Cr[kC][kSW + 1];
    __shared__ float Wl[2][kC * kPad];
    __shared__ float Dk[2][kC * kPad];
    __shared__ float Ub[2][kC][kSW];
    __shared__ float Dc[2];
    const int h = blockIdx.x, slab = blockIdx.y;
    const int tid = threadIdx.x, lt = tid & 255, lane = tid & 63, wv = lt >> 6;
    const bool loader = tid >= 256;
    const int j0 = slab * kSW, i0 = 16 * wv, jl = lane & 15, kq = lane >> 4;
    float* sh = state + (size_t)h * kD * kD;
    for (int i = tid; i < kD * kSW; i += 512) {
        const int kk = key_major ? i / kSW : i % kD, j = key_major ? i % kSW : i / kD;
        S[kk][j] = key_major ? sh[(size_t)kk * kD + j0 + j] : sh[(size_t)(j0 + j) * kD + kk];
    }
    const int nch = (T + kC - 1) / kC;

    // ---- loader waves: a chunk's operands in registers, then in LDS
    struct Ops {
        v4f w[8], dk[8];
        float u[4], decay;
    };
    auto fetch = [&](int c, Ops& o) {
        const float* rec = scratch + ((size_t)c * H + h) * kRec;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = lt + 256 * i;  // row f / 32, float4 f % 32
            o.w[i] = *(const v4f*)(rec + kOffW + (f >> 5) * kD + 4 * (f & 31));
            o.dk[i] = *(const v4f*)(rec + kOffDk + (f >> 5) * kD + 4 * (f & 31));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = lt + 256 * r;  // U slab row f / 16, column f % 16
            o.u[r] = rec[kOffU + (f >> 4) * kD + j0 + (f & 15)];
        }
        o.decay = rec[kOffDecay + lane];  // replicated: a vector load, not a scalar one
    };
    auto stage = [&](int buf, const Ops& o) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = lt + 256 * i;
            *(v4f*)&Wl[buf][(f >> 5) * kPad + 4 * (f & 31)] = o.w[i];
            *(v4f*)&Dk[buf][(f >> 5) * kPad + 4 * (f & 31)] = o.dk[i];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int f = lt + 256 * r;
            Ub[buf][f >> 4][f & 15] = o.u[r];
        }
        if (lt == 0) Dc[buf] = o.decay;
    };

    // ---- compute waves: one chunk from LDS buffer buf
    auto step = [&](int c, int buf) {
        float* rec = scratch + ((size_t)c * H + h) * kRec;
        // the state entering this chunk, for the output kernel
        {
            float sv[kD * kSW / 256];
#pragma unroll
            for (int i = 0; i < kD * kSW / 256; ++i) {
                const int f = lt + 256 * i;
                sv[i] = S[f / kSW][f % kSW];
            }
#pragma unroll
            for (int i = 0; i < kD * kSW / 256; ++i) {
                const int f = lt + 256 * i;
                rec[kOffS + (f / kSW) * kD + j0 + f % kSW] = sv[i];
            }
        }
        // pred = W S: wave w owns rows 16w..16w+15
        f4m acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s0 = 0; s0 < kD / 4; s0 += 16) {  // operand reads in two halves (registers)
            float wa[16], sb[16];
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                wa[s] = Wl[buf][(i0 + jl) * kPad + 4 * (s0 + s) + kq];
                sb[s] = S[4 * (s0 + s) + kq][jl];
            }
            __builtin_amdgcn_sched_barrier(0);  // issue the half's operand reads before its chain
#pragma unroll
            for (int s = 0; s < 16; ++s) acc = mfma4(wa[s], sb[s], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = i0 + 4 * kq + r;
            const float cr = Ub[buf][t][jl] - acc[r];
            Cr[t][jl] = cr;
            rec[kOffU + t * kD + j0 + jl] = cr;
        }
    };
    auto update = [&](int buf) {
        // S <- dk^T corr + decay S: wave w owns key rows 32w..32w+31
        const float decay = Dc[buf];
        f4m sn[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        float sold[2][4];
#pragma unroll
        for (int it2 = 0; it2 < 2; ++it2)
#pragma unroll
            for (int r = 0; r < 4; ++r) sold[it2][r] = S[32 * wv + 16 * it2 + 4 * kq + r][jl];
#pragma unroll
        for (int s0 = 0; s0 < kC / 4; s0 += 8) {
            float cb[8], da[2][8];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int tt = 4 * (s0 + s) + kq;
                cb[s] = Cr[tt][jl];
#pragma unroll
                for (int it2 = 0; it2 < 2; ++it2) da[it2][s] = Dk[buf][tt * kPad + 32 * wv + 16 * it2 + jl];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int it2 = 0; it2 < 2; ++it2) sn[it2] = mfma4(da[it2][s], cb[s], sn[it2]);
        }
#pragma unroll
        for (int it2 = 0; it2 < 2; ++it2)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sd = sold[it2][r] * decay;
                S[32 * wv + 16 * it2 + 4 * kq + r][jl] = sn[it2][r] + sd;
            }
    };

    // The two groups run separate loops that meet at the same barriers (two
    // per chunk), so the compiler counts each group's own memory operations:
    // the loaders' wait for chunk c + 1 does not wait for chunk c + 2, and
    // the compute waves' stores are never waited for.  Requests past the last
    // chunk re-read the last one, keeping that count the same on every path.
    if (loader) {
        Ops ra, rb;  // chunk c + 1 sits in rb for even c, in ra for odd c
        fetch(0, ra);
        fetch(min(1, nch - 1), rb);
        stage(0, ra);
        fetch(min(2, nch - 1), ra);
        __syncthreads();  // the slab and chunk 0's operands are in LDS
        // staging overlaps the compute waves' first half (state store, W S,
        // corr), the next request their second (the state update)
        auto chunk = [&](int c, Ops& nxt) {
            if (c + 1 < nch) stage((c + 1) & 1, nxt);
            lds_barrier();  // chunk c + 1 staged
            fetch(min(c + 3, nch - 1), nxt);
            lds_barrier();
        };
        int c = 0;
        for (; c + 1 < nch; c += 2) {
            chunk(c, rb);
            chunk(c + 1, ra);
        }
        if (c < nch) chunk(c, rb);
    } else {
        __syncthreads();
        for (int c = 0; c < nch; ++c) {
            step(c, c & 1);
            lds_barrier();  // corr visible to every compute wave
            update(c & 1);
            lds_barrier();  // S updated
        }
    }
    for (int i = tid; i < kD * kSW; i += 512) {
        const int kk = key_major ? i / kSW : i % kD, j = key_major ? i % kSW : i / kD;
        if (key_major)
            sh[(size_t)kk * kD + j0 + j] = S[kk][j];
        else
            sh[(size_t)(j0 + j) * kD + kk] = S[kk][j];
    }
}

// Persistent, one 512-thread workgroup per CU (its LDS holds one item):
// o = intra corr + dq S for (chunk, head) items blockIdx.x, + gridDim.x, ...
// in turn, S the state entering the chunk (chunk/core.rs:236-252: the intra
// product, then the inter product added).  The next item's operands (S,
// corr, dq, intra: 144 KB) are requested into registers before the current
// item's products, so a CU's loads overlap its MFMA chains.  Wave w
// computes row tile r = w (w < 4) or 7 - w (rows 16 r .. +15) of columns
// 64 (w / 4) .. +63, lane n of MFMA tile j holding column 64 (w / 4) + 4 n
// + j: the two waves sharing a SIMD take tiles r and 3 - r, and a lane's
// four columns are adjacent, read as one 16-byte word and stored as one.
// The intra product's chain stops after key 16 r + 15 (the record holds no
// tiles above the diagonal ones): intra is zero past the diagonal (the
// reference's pairwise decay is exp(-inf) there), so the
// remaining steps add only zeros, which change no finite sum but a zero's
// sign, and the reference's own `output += sum` into 0.0 (core.rs:288-318)
// clears that sign too, as (0 + intra) + inter does here.
// round_bf16 rounds each output to the nearest bf16, ties to even, as the
// reference's output_bf16 does (gdn.rs:69-76).
__global__ __launch_bounds__(512) void gdn_chunk_out_kernel(const float* __restrict__ scratch, int T, int H,
                                                            float* __restrict__ out, int round_bf16) {
    __shared__ float Sc[kD * kPad];
    __shared__ float Cr[kC * kPad];
    __shared__ float Dq[kC * kPad];
    __shared__ float In[kC * kApad];
    const int nitems = (T + kC - 1) / kC * H;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int rt = wv < 4 ? wv : 7 - wv;
    const int i0 = 16 * rt, c0 = 64 * (wv >> 2), jl = lane & 15, kq = lane >> 4;
    // raw buffer over out's T x H x 128 floats; the host checks that even
    // the last chunk's rows past T have byte offsets below 2^32 (unsigned
    // 32-bit offsets that cannot wrap back into range); 0x00020000 is the
    // gfx9 descriptor word for 32-bit raw access
    const __amdgpu_buffer_rsrc_t out_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(out, (short)0, (int)((unsigned)T * (unsigned)H * kD * 4u), 0x00020000);
    constexpr int NS = kD * kD / 4 / 512, NC = kC * kD / 4 / 512, NI = kC * kC / 4 / 512;
    v4f ps[NS], pc[NC], pd[NC], pi[NI];
    auto fetch = [&](int item) {  // item = chunk * H + head, the record's index
        const float* rec = scratch + (size_t)item * kRec;
#pragma unroll
        for (int i = 0; i < NS; ++i) ps[i] = *(const v4f*)(rec + kOffS + 4 * (tid + 512 * i));
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            pc[i] = *(const v4f*)(rec + kOffU + 4 * (tid + 512 * i));
            pd[i] = *(const v4f*)(rec + kOffDq + 4 * (tid + 512 * i));
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) pi[i] = *(const v4f*)(rec + kOffIntra + 4 * (tid + 512 * i));
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int f = tid + 512 * i;
            *(v4f*)&Sc[(f >> 5) * kPad + 4 * (f & 31)] = ps[i];
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int f = tid + 512 * i;
            *(v4f*)&Cr[(f >> 5) * kPad + 4 * (f & 31)] = pc[i];
            *(v4f*)&Dq[(f >> 5) * kPad + 4 * (f & 31)] = pd[i];
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int f = tid + 512 * i;
            *(v4f*)&In[(f >> 4) * kApad + 4 * (f & 15)] = pi[i];
        }
    };
    auto item_body = [&](int item) {
        const int c = item / H, h = item - c * H;
        const int t0 = c * kC;
        fetch(min(item + (int)gridDim.x, nitems - 1));  // in flight during the products
        f4m oo[4], it[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            oo[jt] = f4m{0.0f, 0.0f, 0.0f, 0.0f};
            it[jt] = oo[jt];
        }
        {
            float ia[kC / 4];
#pragma unroll
            for (int s = 0; s < kC / 4; ++s) ia[s] = In[(i0 + jl) * kApad + 4 * s + kq];
#pragma unroll
            for (int s0 = 0; s0 < kC / 4; s0 += 4) {
                if (s0 >= 4 * (rt + 1)) break;  // keys past the tile's last row
                v4f cb[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) cb[s] = *(const v4f*)&Cr[(4 * (s0 + s) + kq) * kPad + c0 + 4 * jl];
                __builtin_amdgcn_sched_barrier(0);  // a block of operand reads, then its MFMAs
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int jt = 0; jt < 4; ++jt) oo[jt] = mfma4(ia[s0 + s], cb[s][jt], oo[jt]);
            }
        }
        {
            float da[kD / 4];
#pragma unroll
            for (int s = 0; s < kD / 4; ++s) da[s] = Dq[(i0 + jl) * kPad + 4 * s + kq];
#pragma unroll
            for (int s0 = 0; s0 < kD / 4; s0 += 8) {
                v4f sb[8];
#pragma unroll
                for (int s = 0; s < 8; ++s) sb[s] = *(const v4f*)&Sc[(4 * (s0 + s) + kq) * kPad + c0 + 4 * jl];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int s = 0; s < 8; ++s)
#pragma unroll
                    for (int jt = 0; jt < 4; ++jt) it[jt] = mfma4(da[s0 + s], sb[s][jt], it[jt]);
            }
        }
        // unconditional buffer stores: the rows past the prompt's end fall
        // outside the buffer's range and the hardware drops them, so every
        // item issues the same 4 stores and the wait for the next item's
        // operands does not also wait for these
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + i0 + 4 * kq + r;
            v4f o4;
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                const float intra = 0.0f + oo[jt][r];
                float o = intra + it[jt][r];
                const unsigned b = __float_as_uint(o);
                const float ob = __uint_as_float((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
                o4[jt] = round_bf16 ? ob : o;
            }
            const unsigned at = (unsigned)((((size_t)t * H + h) * kD + c0 + 4 * jl) * 4);
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, o4), out_rsrc, (int)at, 0, 0);
        }
    };
    // Each pass requests the next item's operands, forms and stores this
    // item's outputs, then stages the next operands: the requests and the 4
    // stores sit in one block in that order, so the wait before the staging
    // covers the operands only (vmcnt(4)), not this item's stores.  The
    // last pass re-requests and stages the last item (clamped), unused.
    fetch(blockIdx.x);  // the grid never exceeds the item count
    stage();
    lds_barrier();
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
        item_body(item);
        lds_barrier();  // every wave is done reading this item
        stage();
        lds_barrier();
    }
}

// Compute units of the current device (persistent launches), cached per
// device.
static int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

size_t gdn_chunk_scratch_bytes(size_t T, size_t H) { return ((T + kC - 1) / kC) * H * kRec * sizeof(float); }

hipError_t gdn_chunk_prefill(const float* q, const float* k, const float* v, const float* beta, const float* logd,
                             size_t T, size_t H, float* state, float* out, float* scratch, bool key_major,
                             bool round_bf16, hipStream_t s) {
    if (T == 0 || H == 0 || (T + kC) * H * kD * 4 >= ((size_t)1 << 32)) return hipErrorInvalidValue;
    const unsigned nch = (unsigned)((T + kC - 1) / kC);
    hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(nch, (unsigned)H), dim3(256), 0, s, q, k, beta, logd, (int)T,
                       (int)H, scratch);
    hipLaunchKernelGGL(gdn_chunk_solve_kernel, dim3(nch, (unsigned)H, 2), dim3(128), 0, s, v, beta,
                       (const float*)scratch, (int)T, (int)H, scratch);
    hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3((unsigned)H, kD / kSW), dim3(512), 0, s, scratch, (int)T, (int)H,
                       state, key_major ? 1 : 0);
    const unsigned items = nch * (unsigned)H;
    hipLaunchKernelGGL(gdn_chunk_out_kernel, dim3(std::min(items, (unsigned)device_cus())), dim3(512), 0, s, scratch,
                       (int)T, (int)H, out, round_bf16 ? 1 : 0);
    return hipGetLastError();
}

}  // namespace zg
