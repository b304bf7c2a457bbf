// Batched prefill of one sequence: the per-token kernels of the decode step
// restated over n prompt tokens at once (the GDN layers through the chunked
// prefill of zg_prefill.hip, the projections through the batched MFMA
// GEMMs).  Reference semantics: QwenDenseCpu::prefill_transaction
// (model-qwen35/src/lib.rs:1119-1187) runs forward_token (forward.rs:451-516)
// once per token; this path computes the same functions of the prompt, in
// another order of summation (chunked GDN, blocked softmax), so it is held
// to the end-to-end tolerance, not to the bits.
#include <algorithm>

#include <type_traits>

#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

namespace {

template <typename KV>
__device__ __forceinline__ void kv_load4(const KV* p, float (&o)[4]) {
    if constexpr (sizeof(KV) == 2) {
        const uint2 v = *(const uint2*)p;
        o[0] = __uint_as_float(v.x << 16);
        o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16);
        o[3] = __uint_as_float(v.y & 0xffff0000u);
    } else {
        const v4f v = *(const v4f*)p;
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    }
}

__device__ __forceinline__ float prefill_rms_inv(double total, int n, float eps) {
    const float mean = (float)(total / (double)n);
    return 1.0f / sqrtf(mean + eps);
}

}  // namespace

// Grid ((3W + 255) / 256 + 1, ceil(n / TB)), 256 threads.  Thread = channel
// ch of the conv input rows P[t][0:3W] for TB consecutive tokens: the causal
// 4-tap conv of cpu/src/ops/gdn.rs:7-44 over a sliding window (each input
// read once; taps older than the prompt come from the row's ring, where the
// token at position p sits in slot p % 4), SiLU (forward.rs:548), split into
// q, k, v [n][W].  The last workgroup column forms the gates of
// lib.rs:339-362 for its TB tokens, one (token, head) per thread: beta =
// sigmoid(beta projection), log decay softplus(alpha + dt) * a.
template <int TB>
__global__ __launch_bounds__(256) void gdn_prefill_conv_kernel(const float* __restrict__ P, size_t ldp, int n, int W,
                                                               int H, const float* __restrict__ conv_w,
                                                               const float* __restrict__ ring, int pos0,
                                                               const float* __restrict__ dt,
                                                               const float* __restrict__ ssm_a, float* __restrict__ q,
                                                               float* __restrict__ k, float* __restrict__ v,
                                                               float* __restrict__ beta, float* __restrict__ logd) {
    const int t0 = blockIdx.y * TB, ch = blockIdx.x * 256 + threadIdx.x;
    const int t1 = min(t0 + TB, n);
    if (blockIdx.x == gridDim.x - 1) {
        // the gates: one (token, head) per thread (the f64 transcendentals
        // of gdn_coef are the slowest work of the launch; one thread per
        // head running TB tokens in turn held the whole grid back)
        for (int i = threadIdx.x; i < TB * H; i += 256) {
            const int t = t0 + i / H, h = i % H;
            if (t < t1) {
                const float* row = P + (size_t)t * ldp;
                float gain, bt, sp, gr;
                gdn_coef(row[4 * W + h], row[4 * W + H + h], dt[h], ssm_a[h], gain, bt, sp, gr);
                beta[(size_t)t * H + h] = bt;
                logd[(size_t)t * H + h] = gr;
            }
        }
        return;
    }
    if (ch < 3 * W) {
        float w3[3];  // inputs of tokens t-3, t-2, t-1
#pragma unroll
        for (int j = 1; j <= 3; ++j) {
            const int t = t0 - j;
            w3[3 - j] = t >= 0 ? P[(size_t)t * ldp + ch] : ring[(size_t)ch * 4 + ((pos0 + t) & 3)];
        }
        const v4f w = *(const v4f*)(conv_w + (size_t)ch * 4);
        float* dst = ch < W ? q + ch : (ch < 2 * W ? k + (ch - W) : v + (ch - 2 * W));
        float x[TB];
#pragma unroll
        for (int u = 0; u < TB; ++u) x[u] = t0 + u < t1 ? P[(size_t)(t0 + u) * ldp + ch] : 0.0f;
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            if (t0 + u >= t1) break;
            const float c0 = w3[0] * w.x;
            const float c1 = w3[1] * w.y;
            const float c2 = w3[2] * w.z;
            const float c3 = x[u] * w.w;
            float acc = c0 + c1;
            acc = acc + c2;
            acc = acc + c3;
            dst[(size_t)(t0 + u) * W] = ggml_silu(acc);
            w3[0] = w3[1];
            w3[1] = w3[2];
            w3[2] = x[u];
        }
    }
}

// Grid ((3W + 255) / 256), 256 threads: the conv inputs of the last four
// prompt tokens into the row's ring (after every conv of the prompt read it).
__global__ __launch_bounds__(256) void gdn_prefill_ring_kernel(const float* __restrict__ P, size_t ldp, int n, int W,
                                                               float* __restrict__ ring, int pos0) {
    const int ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= 3 * W) return;
    for (int t = max(0, n - 4); t < n; ++t) ring[(size_t)ch * 4 + ((pos0 + t) & 3)] = P[(size_t)t * ldp + ch];
}

// Grid (n, nq + nkv), 256 threads: head `task` of token t (forward.rs:680-
// 695 grouped RMS with q_norm / k_norm; source_rope_kv lib.rs:1552-1577 on
// the first 64 dimensions at position pos0 + t).  q heads go to Q [n][nq][256];
// the key (rounded to the cache type) and the value are appended to the cache.
template <typename KV>
__global__ __launch_bounds__(256) void attn_prefill_prep_kernel(const float* __restrict__ P, size_t ldp, int nq,
                                                                int nkv, const float* __restrict__ qnorm,
                                                                const float* __restrict__ knorm, float eps,
                                                                float theta_scale, int pos0, KV* __restrict__ kc,
                                                                KV* __restrict__ vc, float* __restrict__ Q,
                                                                const float* __restrict__ rope) {
    constexpr int D = 256;
    __shared__ double red[4];
    __shared__ float hv[D];
    __shared__ float rs[32], rc[32];
    const int t = blockIdx.x, task = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int p = pos0 + t;
    const float* row = P + (size_t)t * ldp;
    const bool isq = task < nq;
    const float x = isq ? row[(size_t)task * 2 * D + tid] : row[(size_t)nq * 2 * D + (size_t)(task - nq) * D + tid];
    const float gm = isq ? qnorm[tid] : knorm[tid];
    if (tid < 32) {
        if (rope) {  // the session's table: the same angles and rounding
            const float2 cs = ((const float2*)rope)[(size_t)p * 32 + tid];
            rc[tid] = cs.x;
            rs[tid] = cs.y;
        } else {
            float angle = (float)p;
            for (int i = 0; i < tid; ++i) angle *= theta_scale;
            rs[tid] = cr_sinf(angle);
            rc[tid] = cr_cosf(angle);
        }
    }
    const float sq = x * x;
    double s = wave_sum_xor<double>((double)sq, 64);
    if (lane == 0) red[tid >> 6] = s;
    __syncthreads();
    const float inv = prefill_rms_inv((red[0] + red[1]) + (red[2] + red[3]), D, eps);
    const float tv = x * inv;
    hv[tid] = tv * gm;
    __syncthreads();
    float y = hv[tid];
    if (tid < 32) {
        const float a = hv[tid], b = hv[tid + 32];
        y = fmaf(a, rc[tid], -(b * rs[tid]));
    } else if (tid < 64) {
        const float a = hv[tid - 32], b = hv[tid];
        y = fmaf(a, rs[tid - 32], b * rc[tid - 32]);
    }
    if (isq) {
        Q[((size_t)t * nq + task) * D + tid] = y;
    } else {
        const int kh = task - nq;
        const size_t at = ((size_t)p * nkv + kh) * D + tid;
        if constexpr (sizeof(KV) == 2) {
            uint32_t b = __float_as_uint(y);
            b += 0x7fffu + ((b >> 16) & 1u);
            kc[at] = (KV)(b >> 16);
            uint32_t c = __float_as_uint(row[(size_t)nq * 2 * D + (size_t)nkv * D + (size_t)kh * D + tid]);
            c += 0x7fffu + ((c >> 16) & 1u);
            vc[at] = (KV)(c >> 16);
        } else {
            kc[at] = y;
            vc[at] = row[(size_t)nq * 2 * D + (size_t)nkv * D + (size_t)kh * D + tid];
        }
    }
}

// Four cache elements in storage form (loaded ahead, converted when staged).
template <typename KV>
struct KVRaw4 {
    typename std::conditional<sizeof(KV) == 2, uint2, v4f>::type v;
    __device__ __forceinline__ void load(const KV* p) { v = *(const decltype(v)*)p; }
    __device__ __forceinline__ void get(float (&o)[4]) const {
        if constexpr (sizeof(KV) == 2) {
            o[0] = __uint_as_float(v.x << 16);
            o[1] = __uint_as_float(v.x & 0xffff0000u);
            o[2] = __uint_as_float(v.y << 16);
            o[3] = __uint_as_float(v.y & 0xffff0000u);
        } else {
            o[0] = v.x;
            o[1] = v.y;
            o[2] = v.z;
            o[3] = v.w;
        }
    }
};

typedef _Float16 ah4 __attribute__((ext_vector_type(4)));
typedef _Float16 ah8 __attribute__((ext_vector_type(8)));
typedef float af16 __attribute__((ext_vector_type(16)));

// Causal attention of 32 prompt tokens per workgroup on f16 MFMA.  Grid
// (ceil(n/32), nkv), 64 * G threads: wave g is query head kvh*G + g for
// tokens t0 .. t0+31, all G waves sharing each 32-key block of the KV head
// staged in LDS (K row-major, V transposed, both rounded to f16).
// v_mfma_f32_32x32x16_f16 lanes: A[m = l%32][k = 8(l/32) + e],
// B[k = 8(l/32) + e][n = l%32], C register r = row (r%4) + 8(r/4) + 4(l/32),
// column l%32.  Scores are formed transposed, S^T = K Q^T (query = column),
// so each lane owns one query: the online softmax (block maximum, rescale,
// forward.rs:700-751 semantics in another summation order) needs only the
// partner lane l^32, and the probabilities are already the B operand of
// O^T += V^T P^T when MFMA step s, half h, element e is taken to be key
// 16s + (e%4) + 8(e/4) + 4h of the block (any fixed key order contracts to
// the same sum).  q carries the 1/sqrt(d) scale before rounding to f16.
// Key chunks: a query tile's key blocks are split into chunks of kch blocks,
// one workgroup each (grid x = tiles * ns); a tile whose keys fit one chunk
// writes its output, the others write {m, l, unnormalised o} per (chunk,
// head, query) to `part` for attn_prefill_combine_kernel.
template <typename KV, int G>
__global__ __launch_bounds__(64 * G) void attn_prefill_mfma_kernel(const float* __restrict__ Q,
                                                                   const KV* __restrict__ kc,
                                                                   const KV* __restrict__ vc, int n, int nq,
                                                                   int nkv, int pos0, float scale,
                                                                   const float* __restrict__ P, size_t ldp,
                                                                   float* __restrict__ out, int* __restrict__ status,
                                                                   int ns, int kch, float* __restrict__ part) {
    constexpr int QT = 32, KB = 32, D = 256;
    bool over = false;  // a staged K or V value past the f16 range
    constexpr int KROW = D + 8;   // halves per staged key row (16-byte pad)
    constexpr int VROW = KB + 8;  // halves per staged value column
    __shared__ _Float16 ks[KB * KROW];
    __shared__ _Float16 vt[D * VROW];
    // the heaviest (latest) query tiles first, both kv heads of a tile
    // together, so that the causal tail is short
    const int lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int kvh = lin % (int)gridDim.y, rest = lin / (int)gridDim.y;
    const int ntiles = (int)gridDim.x / ns, tile = ntiles - 1 - rest / ns, chunk = rest % ns;
    const int g = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = kvh * G + g, t0 = tile * QT;
    const int hs = lane >> 5, c = lane & 31;
    const int tq = min(t0 + c, n - 1);
    ah8 qf[16];
    {
        const float* qrow = Q + ((size_t)tq * nq + h) * D + 8 * hs;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const v4f a = *(const v4f*)(qrow + 16 * k), b = *(const v4f*)(qrow + 16 * k + 4);
            qf[k] = ah8{(_Float16)(a.x * scale), (_Float16)(a.y * scale), (_Float16)(a.z * scale),
                        (_Float16)(a.w * scale), (_Float16)(b.x * scale), (_Float16)(b.y * scale),
                        (_Float16)(b.z * scale), (_Float16)(b.w * scale)};
        }
    }
    af16 o[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = af16{};
    float m = -INFINITY, l = 0.0f;
    const bool qvalid = t0 + c < n;
    const int tabs = pos0 + t0 + c;
    const int kend = pos0 + min(t0 + QT, n);  // keys 0 .. kend-1 are seen by some query of the tile
    const int nblk_t = (kend + KB - 1) / KB;
    const int nsplit = (nblk_t + kch - 1) / kch;  // this tile's chunks
    const int bstart = chunk * kch, nblk = min(nblk_t, bstart + kch);
    if (bstart >= nblk) return;  // a chunk past this tile's keys (uniform over the workgroup)
    const size_t kstep = (size_t)nkv * D;
    const KV* kb_ = kc + (size_t)kvh * D;
    const KV* vb_ = vc + (size_t)kvh * D;
    // this thread's share of a 32-key block: PF (key, 4-dim) slots of K and
    // V, kept in storage form; the next block's share is loaded while the
    // current one is computed where the slots divide evenly over the threads
    // and fit the registers (4 heads per kv head; 2 with a bf16 cache)
    constexpr int PF = KB * D / 4 / (64 * G);
    constexpr bool AHEAD = G == 4 || (G == 2 && sizeof(KV) == 2);
    static_assert(!AHEAD || PF * 64 * G == KB * D / 4, "slots divide over the threads");
    // V goes to LDS transposed, as dwords of two keys' halves: item it of
    // wave w takes key pair lane % 16 and dimensions 4 dg .. 4 dg + 3,
    // dg = 4 (w NI + it) + lane / 16, so the 64 lanes of a store hit 32 banks
    // twice (one key per lane and 2-byte stores put 16 lanes on one bank)
    constexpr int NI = AHEAD ? KB / 2 * (D / 4) / (64 * G) : 1;
    KVRaw4<KV> kr[AHEAD ? PF : 1], vr[NI][2];
    const int vpair = lane & 15, vdg = lane >> 4;
    auto load_share = [&](int b) {
#pragma unroll
        for (int it = 0; it < PF; ++it) {
            const int idx = threadIdx.x + it * 64 * G;
            const int key = idx / (D / 4), d4 = (idx % (D / 4)) * 4;
            const int j = min(b * KB + key, kend - 1);  // past the last key: a copy, masked below
            kr[it].load(kb_ + (size_t)j * kstep + d4);
        }
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int d4 = 4 * (4 * (g * NI + it) + vdg);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int j = min(b * KB + 2 * vpair + e, kend - 1);
                vr[it][e].load(vb_ + (size_t)j * kstep + d4);
            }
        }
    };
    if constexpr (AHEAD) load_share(bstart);
    for (int b = bstart; b < nblk; ++b) {
        const int j0 = b * KB;
        __syncthreads();  // the previous block's tiles are consumed
        if constexpr (AHEAD) {
#pragma unroll
            for (int it = 0; it < PF; ++it) {
                const int idx = threadIdx.x + it * 64 * G;
                const int key = idx / (D / 4), d4 = (idx % (D / 4)) * 4;
                float kv4[4];
                kr[it].get(kv4);
                *(ah4*)(ks + key * KROW + d4) =
                    ah4{(_Float16)kv4[0], (_Float16)kv4[1], (_Float16)kv4[2], (_Float16)kv4[3]};
#pragma unroll
                for (int i = 0; i < 4; ++i) over |= !(fabsf(kv4[i]) <= 65504.0f);
            }
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const int d4 = 4 * (4 * (g * NI + it) + vdg);
                float v0[4], v1[4];
                vr[it][0].get(v0);
                vr[it][1].get(v1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const _Float16 lo = (_Float16)v0[i], hi = (_Float16)v1[i];
                    const uint32_t w = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
                                       ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
                    *(uint32_t*)(vt + (d4 + i) * VROW + 2 * vpair) = w;
                    over |= !(fabsf(v0[i]) <= 65504.0f) || !(fabsf(v1[i]) <= 65504.0f);
                }
            }
            if (b + 1 < nblk) load_share(b + 1);
        } else {
            for (int idx = threadIdx.x; idx < KB * D / 4; idx += 64 * G) {
                const int key = idx / (D / 4), d4 = (idx % (D / 4)) * 4;
                const int j = min(j0 + key, kend - 1);  // past the last key: a copy, masked below
                float kv4[4], vv4[4];
                kv_load4(kb_ + (size_t)j * kstep + d4, kv4);
                kv_load4(vb_ + (size_t)j * kstep + d4, vv4);
                *(ah4*)(ks + key * KROW + d4) =
                    ah4{(_Float16)kv4[0], (_Float16)kv4[1], (_Float16)kv4[2], (_Float16)kv4[3]};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    vt[(d4 + i) * VROW + key] = (_Float16)vv4[i];
                    over |= !(fabsf(vv4[i]) <= 65504.0f) || !(fabsf(kv4[i]) <= 65504.0f);
                }
            }
        }
        __syncthreads();
        af16 sc = af16{};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const ah8 ka = *(const ah8*)(ks + c * KROW + 16 * k + 8 * hs);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[k], sc, 0, 0, 0);
        }
        float bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = j0 + (r & 3) + 8 * (r >> 2) + 4 * hs;
            if (!qvalid || key > tabs) sc[r] = -INFINITY;
            bm = fmaxf(bm, sc[r]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        // The reference maximum m moves (and o, l are rescaled) only when
        // some query's block maximum passes it by more than 8: until then
        // the probabilities exp(s - m) stay below e^8, well inside f16, and
        // o / l is the same quotient (the rescale costs as much as the
        // block's products: o lives in 128 accumulator registers).
        const bool raise = __ballot(bm > m + 8.0f) != 0;  // also every first finite block (m = -inf)
        float corr = 1.0f;
        if (raise) {
            const float mn = fmaxf(m, bm);
            corr = mn == -INFINITY ? 1.0f : __expf(m - mn);
            m = mn;
        }
        const bool none = m == -INFINITY;
        float ps = 0.0f;
        ah8 pb[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = none ? 0.0f : __expf(sc[r] - m);
            ps += p;
            pb[r >> 3][r & 7] = (_Float16)p;
        }
        ps += __shfl_xor(ps, 32, 64);
        l = l * corr + ps;
        if (raise) {
#pragma unroll
            for (int d = 0; d < 8; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[d][r] *= corr;
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const _Float16* vp = vt + (d * 32 + c) * VROW + 16 * st + 4 * hs;
                const ah4 lo = *(const ah4*)vp, hi = *(const ah4*)(vp + 8);
                const ah8 va = ah8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[st], o[d], 0, 0, 0);
            }
        }
    }
    if (nsplit > 1) {  // this chunk's partial: {m, l} then o for the combine
        float* rec = part + ((((size_t)tile * ns + chunk) * nq + h) * QT + c) * (D + 2);
        if (hs == 0) {
            rec[0] = m;
            rec[1] = l;
        }
#pragma unroll
        for (int d = 0; d < 8; ++d)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int dim = d * 32 + 8 * q + 4 * hs;
                *(v4f*)(rec + 2 + dim) = v4f{o[d][4 * q], o[d][4 * q + 1], o[d][4 * q + 2], o[d][4 * q + 3]};
            }
    } else if (qvalid) {
        const float inv = 1.0f / l;
        const float* gate = P + (size_t)(t0 + c) * ldp + (size_t)h * 2 * D + D;
        float* orow = out + ((size_t)(t0 + c) * nq + h) * D;
#pragma unroll
        for (int d = 0; d < 8; ++d)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int dim = d * 32 + 8 * q + 4 * hs;
                const v4f gv = *(const v4f*)(gate + dim);
                v4f ov;
#pragma unroll
                for (int e = 0; e < 4; ++e) ov[e] = o[d][4 * q + e] * inv * source_sigmoid(gv[e]);
                *(v4f*)(orow + dim) = ov;
            }
    }
    if (over && status) atomicOr(status, 16);
}

// Grid (tiles * 4, nq), 256 threads: thread t takes query 8 (x % 4) + t / 32
// of tile x / 4 and dimensions 8 (t % 32) .. +7, combining the chunks'
// partials weighted by exp(m_c - M), divided by the weighted sum of l_c,
// gated; every load is issued before the first use.  Tiles of one chunk
// were written directly.
__global__ __launch_bounds__(256) void attn_prefill_combine_kernel(int n, int nq, int pos0, int ns, int kch,
                                                                   const float* __restrict__ part,
                                                                   const float* __restrict__ P, size_t ldp,
                                                                   float* __restrict__ out) {
    constexpr int QT = 32, KB = 32, D = 256, NSMAX = 4;
    const int tile = blockIdx.x >> 2, h = blockIdx.y;
    const int c = 8 * (blockIdx.x & 3) + (threadIdx.x >> 5), d0 = 8 * (threadIdx.x & 31);
    const int t0 = tile * QT;
    const int kend = pos0 + min(t0 + QT, n);
    const int nsplit = ((kend + KB - 1) / KB + kch - 1) / kch;
    if (nsplit <= 1 || t0 + c >= n) return;
    const size_t cstride = (size_t)nq * QT * (D + 2);  // next chunk's record of the same (head, query)
    const float* rec0 = part + (((size_t)tile * ns * nq + h) * QT + c) * (D + 2);
    float mk[NSMAX], lk[NSMAX];
    v4f ok[NSMAX][2];
#pragma unroll
    for (int k = 0; k < NSMAX; ++k) {
        const float* rec = rec0 + (size_t)min(k, nsplit - 1) * cstride;
        mk[k] = rec[0];
        lk[k] = rec[1];
        ok[k][0] = *(const v4f*)(rec + 2 + d0);
        ok[k][1] = *(const v4f*)(rec + 2 + d0 + 4);
    }
    const float* gp = P + (size_t)(t0 + c) * ldp + (size_t)h * 2 * D + D + d0;
    const v4f g0 = *(const v4f*)gp, g1 = *(const v4f*)(gp + 4);
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < NSMAX; ++k)
        if (k < nsplit) M = fmaxf(M, mk[k]);
    float L = 0.0f, o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < NSMAX; ++k) {
        if (k < nsplit) {
            const float w = mk[k] == -INFINITY ? 0.0f : __expf(mk[k] - M);
            L += w * lk[k];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o[e] += w * ok[k][0][e];
                o[4 + e] += w * ok[k][1][e];
            }
        }
    }
    const float inv = 1.0f / L;
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    v4f r0, r1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        r0[e] = o[e] * inv * source_sigmoid(gv[e]);
        r1[e] = o[4 + e] * inv * source_sigmoid(gv[4 + e]);
    }
    float* orow = out + ((size_t)(t0 + c) * nq + h) * D + d0;
    *(v4f*)orow = r0;
    *(v4f*)(orow + 4) = r1;
}

size_t attn_prefill_part_bytes(size_t n, int nq) {
    const size_t ns = n >= 128 ? 4 : 1;
    return ns == 1 ? 0 : (n + 31) / 32 * ns * (size_t)nq * 32 * (256 + 2) * sizeof(float);
}

hipError_t gdn_prefill_conv(const float* P, size_t ldp, size_t n, size_t W, size_t H, const float* conv_w,
                            float* ring, int pos0, const float* dt, const float* ssm_a, float* q, float* k, float* v,
                            float* beta, float* logd, hipStream_t s) {
    if (n == 0 || W == 0 || H == 0 || H > 256) return hipErrorInvalidValue;
    constexpr int TB = 16;
    hipLaunchKernelGGL(gdn_prefill_conv_kernel<TB>, dim3((unsigned)((3 * W + 255) / 256 + 1), (unsigned)((n + TB - 1) / TB)),
                       dim3(256), 0, s, P, ldp, (int)n, (int)W, (int)H, conv_w, (const float*)ring, pos0, dt, ssm_a, q,
                       k, v, beta, logd);
    hipLaunchKernelGGL(gdn_prefill_ring_kernel, dim3((unsigned)((3 * W + 255) / 256)), dim3(256), 0, s, P, ldp,
                       (int)n, (int)W, ring, pos0);
    return hipGetLastError();
}

hipError_t attn_prefill(const AttnPrefillArgs& a, hipStream_t s) {
    const int G = a.nq / a.nkv;
    if (a.n == 0 || a.nkv <= 0 || a.nq % a.nkv || G < 1 || G > 4) return hipErrorInvalidValue;
    if (a.kv_bf16) {
        hipLaunchKernelGGL(attn_prefill_prep_kernel<uint16_t>, dim3((unsigned)a.n, (unsigned)(a.nq + a.nkv)),
                           dim3(256), 0, s, a.P, a.ldp, a.nq, a.nkv, a.qnorm, a.knorm, a.eps, a.theta_scale, a.pos0,
                           (uint16_t*)a.kcache, (uint16_t*)a.vcache, a.Q, a.rope);
    } else {
        hipLaunchKernelGGL(attn_prefill_prep_kernel<float>, dim3((unsigned)a.n, (unsigned)(a.nq + a.nkv)), dim3(256),
                           0, s, a.P, a.ldp, a.nq, a.nkv, a.qnorm, a.knorm, a.eps, a.theta_scale, a.pos0,
                           (float*)a.kcache, (float*)a.vcache, a.Q, a.rope);
    }
    // key chunks: 4 per query tile while the tiles give fewer than 256
    // workgroups (measured at 2048 tokens: one workgroup per tile left the
    // heaviest tiles' 64 key blocks on 128 workgroups, 260 us against 167;
    // at 8192 tokens the split ran slower), as many blocks each as the
    // longest tile needs
    const int ntiles = (int)((a.n + 31) / 32);
    const int ns = a.part && attn_prefill_part_bytes(a.n, a.nq) && ntiles * a.nkv < 256 ? 4 : 1;
    const int nblk_max = (int)((a.pos0 + a.n + 31) / 32);
    const int kch = (nblk_max + ns - 1) / ns;
    const dim3 grid((unsigned)(ntiles * ns), (unsigned)a.nkv);
#define ZG_AP(KV, GG)                                                                                              \
    hipLaunchKernelGGL((attn_prefill_mfma_kernel<KV, GG>), grid, dim3(64 * GG), 0, s, a.Q, (const KV*)a.kcache,   \
                       (const KV*)a.vcache, (int)a.n, a.nq, a.nkv, a.pos0, a.scale, a.P, a.ldp, a.out, a.status, ns, \
                       kch, a.part)
#define ZG_APG(KV)                  \
    switch (G) {                    \
    case 1: ZG_AP(KV, 1); break;    \
    case 2: ZG_AP(KV, 2); break;    \
    case 3: ZG_AP(KV, 3); break;    \
    default: ZG_AP(KV, 4); break;   \
    }
    if (a.kv_bf16) {
        ZG_APG(uint16_t)
    } else {
        ZG_APG(float)
    }
#undef ZG_APG
#undef ZG_AP
    if (ns > 1)
        hipLaunchKernelGGL(attn_prefill_combine_kernel, dim3((unsigned)(ntiles * 4), (unsigned)a.nq), dim3(256), 0, s,
                           (int)a.n, a.nq, a.pos0, ns, kch, (const float*)a.part, a.P, a.ldp, a.out);
    return hipGetLastError();
}

}  // namespace zg
