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
// Two launches.  gdn_chunk_prep_kernel runs every (chunk, head) in parallel:
// normalisation, gates, A and intra on f32 MFMA (16x16x4), and the unit-lower
// solves, one column per thread in the reference's summation order.  It
// writes U, W, dq, dk, intra and exp(g_last) to a scratch record per
// (chunk, head).  gdn_chunk_scan_kernel carries the state: workgroup
// (value slab of 32 columns, head) walks the chunks in order (the value
// columns of S evolve independently) with every product on f32 MFMA.
#include <algorithm>

#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

namespace {

constexpr int kC = 64, kD = 128, kSlab = 32;
constexpr int kPad = 132;  // LDS row pitch (floats) for [64][128] tiles
typedef float f4m __attribute__((ext_vector_type(4)));

// Scratch record per (chunk, head), floats.
constexpr size_t kOffU = 0, kOffW = kOffU + kC * kD, kOffDq = kOffW + kC * kD, kOffDk = kOffDq + kC * kD,
                 kOffIntra = kOffDk + kC * kD, kOffDecay = kOffIntra + kC * kC, kRec = kOffDecay + 64;

// 16x16 output tile of X Y^T over K = kD (X, Y: rows of 128 in LDS with
// pitch kPad) on v_mfma_f32_16x16x4f32.  Lane l supplies X[i0 + l%16][4s + l/16]
// and Y[j0 + l%16][4s + l/16]; result register r is (i0 + 4(l/16) + r, j0 + l%16).
__device__ __forceinline__ f4m tile_xyT(const float* X, const float* Y, int i0, int j0, int lane, float xscale_row) {
    f4m acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* xr = X + (i0 + (lane & 15)) * kPad + (lane >> 4);
    const float* yr = Y + (j0 + (lane & 15)) * kPad + (lane >> 4);
#pragma unroll 8
    for (int s = 0; s < kD / 4; ++s) {
        const float xa = xr[4 * s] * xscale_row;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, yr[4 * s], acc, 0, 0, 0);
    }
    return acc;
}

}  // namespace

// Grid (chunks, H), 256 threads.
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                             const float* __restrict__ v,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ logd, int T, int H,
                                                             float* __restrict__ scratch) {
    __shared__ float qs[kC * kPad];
    __shared__ float ks[kC * kPad];
    __shared__ float as[kC][kC + 1];
    __shared__ float is_[kC][kC + 1];
    __shared__ float gs[kC], bs[kC], eg[kC], el[kC];
    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = c * kC, rows = min(kC, T - t0);
    float* rec = scratch + ((size_t)c * H + h) * kRec;
    const float inv_sqrt = 1.0f / sqrtf((float)kD);
    const float eps = 1e-6f / (float)kD;

    // q, k rows: two-stage L2 (zgo restatement of forward.rs:564-576), one row
    // per wave at a time, two elements per lane
    for (int t = wv; t < kC; t += 4) {
        float xq[2] = {0.0f, 0.0f}, xk[2] = {0.0f, 0.0f};
        if (t < rows) {
            const size_t src = ((size_t)(t0 + t) * H + h) * kD;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                xq[e] = q[src + lane + 64 * e];
                xk[e] = k[src + lane + 64 * e];
            }
        }
        double sq = 0.0, sk = 0.0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float a2 = xq[e] * xq[e], b2 = xk[e] * xk[e];
            sq += (double)a2;
            sk += (double)b2;
        }
        sq = wave_sum_xor<double>(sq, 64);
        sk = wave_sum_xor<double>(sk, 64);
        const float iq = 1.0f / sqrtf((float)(sq / (double)kD) + eps);
        const float ik = 1.0f / sqrtf((float)(sk / (double)kD) + eps);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float a = 0.0f, b = 0.0f;
            if (t < rows) {
                const float tq = xq[e] * iq;
                const float nq = tq * inv_sqrt;
                a = nq * inv_sqrt;
                const float tk = xk[e] * ik;
                b = tk * inv_sqrt;
            }
            qs[t * kPad + lane + 64 * e] = a;
            ks[t * kPad + lane + 64 * e] = b;
        }
    }
    if (tid < kC) bs[tid] = tid < rows ? beta[(size_t)(t0 + tid) * H + h] : 0.0f;
    if (tid == 0) {
        double running = 0.0;
        for (int t = 0; t < kC; ++t) {
            if (t < rows) running += (double)logd[(size_t)(t0 + t) * H + h];
            gs[t] = (float)running;
        }
    }
    __syncthreads();

    // A = (beta k) k^T and intra = q k^T, decayed; 16 tiles each, 4 per wave
    for (int tile = wv; tile < 16; tile += 4) {
        const int i0 = (tile >> 2) * 16, j0 = (tile & 3) * 16;
        const float brow = bs[i0 + (lane & 15)];
        const f4m a4 = tile_xyT(ks, ks, i0, j0, lane, brow);
        const f4m q4 = tile_xyT(qs, ks, i0, j0, lane, 1.0f);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = i0 + 4 * (lane >> 4) + r, s = j0 + (lane & 15);
            const float decay = s <= t ? cr_expf(gs[t] - gs[s]) : 0.0f;
            as[t][s] = a4[r] * decay;
            is_[t][s] = q4[r] * decay;
        }
    }
    // dq = q exp(g), dk = k exp(g_last - g); intra and exp(g_last) to scratch
    const float last = gs[kC - 1];
    if (tid < kC) {
        eg[tid] = cr_expf(gs[tid]);
        el[tid] = cr_expf(last - gs[tid]);
    }
    __syncthreads();
    for (int i = tid; i < kC * kD / 4; i += 256) {
        const int t = (4 * i) / kD, d = (4 * i) % kD;
        const v4f qv = *(const v4f*)&qs[t * kPad + d], kv = *(const v4f*)&ks[t * kPad + d];
        *(v4f*)(rec + kOffDq + 4 * i) = qv * eg[t];
        *(v4f*)(rec + kOffDk + 4 * i) = kv * el[t];
    }
    for (int i = tid; i < kC * kC; i += 256) rec[kOffIntra + i] = is_[i / kC][i % kC];
    if (tid == 0) rec[kOffDecay] = cr_expf(last);

    // unit-lower solves (gdn/chunk.rs:16-76: separate products, four
    // interleaved partial sums, (s0+s2)+(s1+s3), scalar tail, one subtraction):
    // thread j < 128 solves column j of U (rhs beta v), thread 128 + j column j
    // of W (rhs (beta k) exp(g)), the column in registers
    {
        const int col = tid & (kD - 1);
        float xr[kC];
#pragma unroll
        for (int t = 0; t < kC; ++t) {
            float r = 0.0f;
            if (t < rows) {
                if (tid < kD) {
                    const float vv = v[((size_t)(t0 + t) * H + h) * kD + col];
                    r = vv * bs[t];
                } else {
                    const float kb = ks[t * kPad + col] * bs[t];
                    r = kb * eg[t];
                }
            }
            xr[t] = r;
        }
#pragma unroll
        for (int row = 0; row < kC; ++row) {
            const int vend = row / 4 * 4;
            float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < vend; st += 4) {
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    const float p = as[row][st + l] * xr[st + l];
                    s4[l] = s4[l] + p;
                }
            }
            float sum = (s4[0] + s4[2]) + (s4[1] + s4[3]);
#pragma unroll
            for (int kk = vend; kk < row; ++kk) {
                const float p = as[row][kk] * xr[kk];
                sum = sum + p;
            }
            xr[row] = xr[row] - sum;
        }
        float* dst = rec + (tid < kD ? kOffU : kOffW);
#pragma unroll
        for (int t = 0; t < kC; ++t) dst[t * kD + col] = xr[t];
    }
}

// Grid (kD / kSlab, H), 256 threads: value columns [32 slab, 32 slab + 32) of
// head h across all chunks in order.  The state is held key-major S[k][j] in
// LDS; in memory it is value-major [h][v][k] (the decode layout) or, with
// key_major, [h][k][v] (the chunk reference's layout).  round_bf16 rounds
// each output to the nearest bf16 (ties to even), as the reference's
// output_bf16 does (gdn.rs:69-76).
__global__ __launch_bounds__(256) void gdn_chunk_scan_kernel(const float* __restrict__ scratch, int T, int H,
                                                             float* __restrict__ state, float* __restrict__ out,
                                                             int key_major, int round_bf16) {
    __shared__ float Ws[kC * kPad];  // W, later dk
    __shared__ float Dq[kC * kPad];
    __shared__ float S[kD][kSlab + 1];
    __shared__ float corr[kC][kSlab + 1];
    __shared__ float In[kC][kC + 1];
    const int slab = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int j0 = slab * kSlab;
    float* sh = state + (size_t)h * kD * kD;
    if (key_major) {
        for (int i = tid; i < kD * kSlab; i += 256) S[i / kSlab][i % kSlab] = sh[(size_t)(i / kSlab) * kD + j0 + i % kSlab];
    } else {
        for (int i = tid; i < kD * kSlab; i += 256) S[i % kD][i / kD] = sh[(size_t)(j0 + i / kD) * kD + i % kD];
    }
    const int nch = (T + kC - 1) / kC;
    for (int c = 0; c < nch; ++c) {
        const int t0 = c * kC, rows = min(kC, T - t0);
        const float* rec = scratch + ((size_t)c * H + h) * kRec;
        for (int i = tid; i < kC * kD / 4; i += 256) {
            const int t = (4 * i) / kD, d = (4 * i) % kD;
            *(v4f*)&Ws[t * kPad + d] = *(const v4f*)(rec + kOffW + 4 * i);
            *(v4f*)&Dq[t * kPad + d] = *(const v4f*)(rec + kOffDq + 4 * i);
        }
        for (int i = tid; i < kC * kC; i += 256) In[i / kC][i % kC] = rec[kOffIntra + i];
        const float decay = rec[kOffDecay];
        __syncthreads();
        // pred = W S and inter = dq S: wave w owns rows 16w..16w+15, both 16-column tiles
        const int i0 = 16 * wv;
        f4m pr[2], it[2];
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
            pr[jt] = f4m{0.0f, 0.0f, 0.0f, 0.0f};
            it[jt] = f4m{0.0f, 0.0f, 0.0f, 0.0f};
        }
        for (int s = 0; s < kD / 4; ++s) {
            const int kk = 4 * s + (lane >> 4);
            const float wa = Ws[(i0 + (lane & 15)) * kPad + kk];
            const float da = Dq[(i0 + (lane & 15)) * kPad + kk];
#pragma unroll
            for (int jt = 0; jt < 2; ++jt) {
                const float sb = S[kk][16 * jt + (lane & 15)];
                pr[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa, sb, pr[jt], 0, 0, 0);
                it[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(da, sb, it[jt], 0, 0, 0);
            }
        }
        // corr = U - pred
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = i0 + 4 * (lane >> 4) + r, j = 16 * jt + (lane & 15);
                corr[t][j] = rec[kOffU + t * kD + j0 + j] - pr[jt][r];
            }
        __syncthreads();
        // o = intra corr + inter
        f4m oo[2];
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) oo[jt] = f4m{0.0f, 0.0f, 0.0f, 0.0f};
        for (int s = 0; s < kC / 4; ++s) {
            const int kk = 4 * s + (lane >> 4);
            const float ia = In[i0 + (lane & 15)][kk];
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
                oo[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ia, corr[kk][16 * jt + (lane & 15)], oo[jt], 0, 0, 0);
        }
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = i0 + 4 * (lane >> 4) + r, j = 16 * jt + (lane & 15);
                if (t < rows) {
                    float o = oo[jt][r] + it[jt][r];
                    if (round_bf16) {
                        const unsigned b = __float_as_uint(o);
                        o = __uint_as_float((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
                    }
                    out[((size_t)(t0 + t) * H + h) * kD + j0 + j] = o;
                }
            }
        // dk into the W buffer (W no longer needed after the barrier)
        __syncthreads();
        for (int i = tid; i < kC * kD / 4; i += 256) {
            const int t = (4 * i) / kD, d = (4 * i) % kD;
            *(v4f*)&Ws[t * kPad + d] = *(const v4f*)(rec + kOffDk + 4 * i);
        }
        __syncthreads();
        // S <- dk^T corr + decay S: wave w owns key rows 32w..32w+31 (two tiles) x 2 column tiles
        f4m sn[2][2];
#pragma unroll
        for (int it2 = 0; it2 < 2; ++it2)
#pragma unroll
            for (int jt = 0; jt < 2; ++jt) sn[it2][jt] = f4m{0.0f, 0.0f, 0.0f, 0.0f};
        for (int s = 0; s < kC / 4; ++s) {
            const int tt = 4 * s + (lane >> 4);
#pragma unroll
            for (int it2 = 0; it2 < 2; ++it2) {
                const float ka = Ws[tt * kPad + 32 * wv + 16 * it2 + (lane & 15)];
#pragma unroll
                for (int jt = 0; jt < 2; ++jt)
                    sn[it2][jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka, corr[tt][16 * jt + (lane & 15)], sn[it2][jt], 0, 0, 0);
            }
        }
        float snew[2][2][4];
#pragma unroll
        for (int it2 = 0; it2 < 2; ++it2)
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kr = 32 * wv + 16 * it2 + 4 * (lane >> 4) + r, j = 16 * jt + (lane & 15);
                    const float sd = S[kr][j] * decay;
                    snew[it2][jt][r] = sn[it2][jt][r] + sd;
                }
        __syncthreads();
#pragma unroll
        for (int it2 = 0; it2 < 2; ++it2)
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    S[32 * wv + 16 * it2 + 4 * (lane >> 4) + r][16 * jt + (lane & 15)] = snew[it2][jt][r];
        __syncthreads();
    }
    if (key_major) {
        for (int i = tid; i < kD * kSlab; i += 256) sh[(size_t)(i / kSlab) * kD + j0 + i % kSlab] = S[i / kSlab][i % kSlab];
    } else {
        for (int i = tid; i < kD * kSlab; i += 256) sh[(size_t)(j0 + i / kD) * kD + i % kD] = S[i % kD][i / kD];
    }
}

size_t gdn_chunk_scratch_bytes(size_t T, size_t H) { return ((T + kC - 1) / kC) * H * kRec * sizeof(float); }

hipError_t gdn_chunk_prefill(const float* q, const float* k, const float* v, const float* beta, const float* logd,
                             size_t T, size_t H, float* state, float* out, float* scratch, bool key_major,
                             bool round_bf16, hipStream_t s) {
    if (T == 0 || H == 0) return hipErrorInvalidValue;
    const unsigned nch = (unsigned)((T + kC - 1) / kC);
    hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(nch, (unsigned)H), dim3(256), 0, s, q, k, v, beta, logd, (int)T,
                       (int)H, scratch);
    hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3(kD / kSlab, (unsigned)H), dim3(256), 0, s, scratch, (int)T, (int)H,
                       state, out, key_major ? 1 : 0, round_bf16 ? 1 : 0);
    return hipGetLastError();
}

}  // namespace zg
