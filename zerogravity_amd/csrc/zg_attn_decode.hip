// Resident attention decode step and the greedy argmax.
#include <algorithm>

#include "zg_decode_common.hpp"

namespace zg {

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
            const size_t at = xh_tile_index(m, k, K, gridDim.z);  // B rows = gridDim.z
            if (a.status && !(fabsf(v) <= 65504.0f)) atomicOr(a.status, 16);
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

// ============================================ split-T attention (1..64 rows)
//
// Flash-decoding form of the same layer: workgroup (c, kv head, row) takes
// the tokens [c S, (c + 1) S) of the row (S = attn_split_span, a multiple
// of 32 fixed per launch, so a workgroup's key and value addresses do not
// depend on the position: its first tile of each is requested before the
// position arrives, and a span at or past the row's T = pos + 1 tokens
// records itself empty, m = -inf and l = 0, and ends).  It normalises and ropes the G query heads and the new
// key as attn_decode_qk_kernel does (the workgroup whose span holds the
// position appends K/V and uses its own rounded copies for that token),
// scores its tokens in the 32-accumulator order, and keeps per head the
// span's max m, l = sum of exp(s - m) and o = sum of exp(s - m) * v (exp
// through the hardware exp2, combine_exp).
// attn_combine_kernel then forms sum_c e^(m_c - M) o_c / sum_c e^(m_c - M)
// l_c over the row's spans (the empty ones weigh 0), M = max_c m_c, wave w
// summing spans w, w + 4, ... and the four waves' sums added in a fixed
// order (attn_combine_quarter_kernel: a quarter of the channels per
// workgroup, for few rows with many spans), and applies the sigmoid gate
// (forward.rs:751).  The reference (lib.rs:1276-1387)
// normalises with the global max first and runs the value sums as
// token-ordered chains: this regrouping agrees with it to f32 rounding (the
// per-op 1e-3 bar), not bit for bit.
constexpr int kSplitMaxSpan = 1024;  // tokens per workgroup (LDS scores)
// e^x through the hardware exp2 (a few ulp): the split form's weights, held
// to the reference at f32 rounding rather than bit for bit
__device__ __forceinline__ float combine_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
constexpr int kSplitMaxChunks = 256;

// Tokens per span, a multiple of 32: about 256 workgroups over the batch at
// a full context up to 4 rows (short spans: each workgroup's dependent
// chain is short, and at a 2k context one row gets one 32-token tile per
// workgroup), about 512 beyond (two per CU: a workgroup's prologue -- the
// q/k norms and RoPE -- costs more than a longer span); never more than
// kSplitMaxChunks spans.
int attn_split_span(size_t B, int nkv, size_t max_ctx) {
    const size_t target = B <= 4 ? 256 : 512;
    const size_t want = (max_ctx * B * (size_t)nkv + target - 1) / target;
    const size_t floor = (max_ctx + kSplitMaxChunks - 1) / kSplitMaxChunks;
    const size_t s = std::max({want, floor, (size_t)32});
    return (int)((s + 31) / 32 * 32);
}

int attn_split_chunks(size_t B, int nkv, size_t max_ctx) {
    const size_t S = (size_t)attn_split_span(B, nkv, max_ctx);
    return (int)((max_ctx + S - 1) / S);
}

bool attn_split_supported(size_t B, int nq, int nkv, size_t max_ctx) {
    return B >= 1 && B <= 64 && nkv > 0 && nq % nkv == 0 && nq / nkv <= 4 && max_ctx > 0 &&
           attn_split_span(B, nkv, max_ctx) <= kSplitMaxSpan && attn_split_chunks(B, nkv, max_ctx) <= kSplitMaxChunks;
}

size_t attn_split_part_bytes(size_t B, int nq, int nkv, size_t max_ctx) {
    return B * (size_t)nq * attn_split_chunks(B, nkv, max_ctx) * (256 + 2) * sizeof(float);
}

// Partials: {m, l} per (row, head, span) at part, then o [row][head][span][256];
// o is written for the spans that hold tokens of the row only.
template <typename KV, int G>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnDecodeArgs a, int nc, int span, float* __restrict__ part) {
    constexpr int D = 256;
    __shared__ float hv[G + 1][D];
    __shared__ float rsin[32], rcos[32];
    __shared__ v4f scp[kSplitMaxSpan];  // scores, then exp(s - m): [token][head]
    __shared__ float red[2][G][4];
    __shared__ float vrow[D];
    __shared__ float rob[4 * G * D];  // the waves' value sums of a short span
    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, s = tid & 7;
    const int t0 = c * span;
    KV* kc = (KV*)a.kcache + (size_t)b * a.cache_row_stride + (size_t)kvh * D;
    KV* vc = (KV*)a.vcache + (size_t)b * a.cache_row_stride + (size_t)kvh * D;
    const size_t tstep = (size_t)a.nkv * D;
    // keys of a 32-token tile: token t0 + 32 i + tid / 8, 32 dims per thread;
    // values: wave w takes tokens t0 + 32 i + 8 w + u (u < 8), lane l
    // channels 4l .. 4l+3.  Addresses clamped into the cache (rows past the
    // position are read and never used).
    KVPack<KV> kn[8], vn[8];
    auto load_keys = [&](int i) {
        const int tk = min(t0 + 32 * i + (tid >> 3), a.max_ctx - 1);
#pragma unroll
        for (int q = 0; q < 8; ++q) kn[q].load(kc + (size_t)tk * tstep + 32 * q + 4 * s);
    };
    auto load_values = [&](int i) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            vn[u].load(vc + (size_t)min(t0 + 32 * i + 8 * wv + u, a.max_ctx - 1) * tstep + 4 * lane);
    };
    // the position, the span's first key and value tiles, then the q heads
    // (tasks 0..G-1) and the key (task G), wave w taking tasks w, w+4
    const int p = a.pos[b];
    load_keys(0);
    load_values(0);
    const float* proj = a.proj + (size_t)b * a.proj_stride;
    const int QD2 = a.nq * 2 * D;
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
    const float vnew = proj[QD2 + (size_t)a.nkv * D + (size_t)kvh * D + tid];

    const int T = p + 1;
    const int t1 = min(T, t0 + span), n = t1 - t0;
    const size_t nrow = (size_t)gridDim.z * a.nq * nc;
    const size_t slot = ((size_t)b * a.nq + (size_t)kvh * G) * nc + c;  // head g at slot + g * nc
    float* ml = part;
    float* po = part + 2 * nrow;
    if (n <= 0) {  // past the row's tokens: an empty span, m = -inf and l = 0 (its o is never read)
        if (tid < G) {
            ml[2 * (slot + (size_t)tid * nc)] = -INFINITY;
            ml[2 * (slot + (size_t)tid * nc) + 1] = 0.0f;
        }
        return;
    }
    const bool owner = t0 <= p && p < t1;

    if (tid < 32) {
        if (a.rope) {  // the session's table: the same angles and rounding
            const float2 cs = ((const float2*)a.rope)[(size_t)p * 32 + tid];
            rcos[tid] = cs.x;
            rsin[tid] = cs.y;
        } else {
            float angle = (float)p;
            for (int t = 0; t < tid; ++t) angle *= a.theta_scale;
            rsin[tid] = cr_sinf(angle);
            rcos[tid] = cr_cosf(angle);
        }
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int task = 4 * i + wv;
        if (task <= G) {
            double sq = 0.0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float q = tv[i][r] * tv[i][r];
                sq += (double)q;
            }
            const float inv = rms_inv(wave_sum_all(sq), D, a.eps);
#pragma unroll
            for (int r = 0; r < 4; ++r) hv[task][lane + 64 * r] = (tv[i][r] * inv) * tg[i][r];
        }
    }
    lds_barrier();  // the angles, and each head's normalised values for its wave
#pragma unroll
    for (int task0 = 0; task0 <= G; task0 += 4) {
        const int task = task0 + wv;
        if (task <= G) {
            head_rope(hv[task], rsin, rcos, lane);
            // the key as the cache holds it (the same wave reads it back)
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (task == G) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const KV st = kv_st<KV>(hv[G][lane + 64 * r]);
                    if (owner) kc[(size_t)p * tstep + lane + 64 * r] = st;
                    hv[G][lane + 64 * r] = kv_ld<KV>(&st);
                }
            }
        }
    }
    const KV vst = kv_st<KV>(vnew);
    vrow[tid] = kv_ld<KV>(&vst);  // the position's value as the cache holds it
    if (owner) vc[(size_t)p * tstep + tid] = vst;
    lds_barrier();

    // ---- scores of the span's tiles
    const int nb = (n + 31) >> 5;
    {
        // the queries are read from LDS at each use (held in registers beside
        // the key and value tiles in flight they would halve the occupancy)
        for (int i = 0; i < nb; ++i) {
            KVPack<KV> cur[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) cur[q] = kn[q];
            if (i + 1 < nb) load_keys(i + 1);
            const int t = t0 + 32 * i + (tid >> 3);
            float kk[8][4];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (t == p) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) kk[q][e] = hv[G][32 * q + 4 * s + e];
                } else {
                    cur[q].unpack(kk[q]);
                }
            }
            float acc[G][4];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[g][e] = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const v4f qq = *(const v4f*)&hv[g][32 * q + 4 * s];
                    const float qe[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[g][e] = fmaf(qe[e], kk[q][e], acc[g][e]);
                }
            float dv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < G; ++g) {
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[g][e] = group8_tree_last(acc[g][e]);
                dv[g] = ((acc[g][0] + acc[g][1]) + (acc[g][2] + acc[g][3])) * a.scale;
            }
            if (t < t1 && s == 7) scp[t - t0] = v4f{dv[0], dv[1], dv[2], dv[3]};
        }
    }
    lds_barrier();

    if (n <= 64) {
        // ---- a span of at most 64 tokens: every wave forms the statistics
        // itself, lane i holding token i (the values below: there wave 0
        // holds every token and the other waves add zeros), and keeps p in
        // its lanes, read back per token with readlane, so no barrier
        // separates the scores from the value sums
        const v4f s4 = scp[lane];
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
        const bool live = lane < n;
        float m[G], l[G], pe[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            m[g] = wave_max_all(live ? sv[g] : -INFINITY);
            pe[g] = live ? combine_exp(sv[g] - m[g]) : 0.0f;
            l[g] = wave_sum_all(pe[g]);  // >= 1, so adding the other waves' +0 sums changes no bit
        }
        const int ws = __builtin_amdgcn_readfirstlane(wv);
        float o[G][4];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[g][e] = 0.0f;
        for (int i = 0; i < nb; ++i) {
            float cv[8][4];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                vn[u].unpack(cv[u]);
                if (t0 + 32 * i + 8 * ws + u == p) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) cv[u][e] = vrow[4 * lane + e];
                }
            }
            if (i + 1 < nb) load_values(i + 1);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int tt = 32 * i + 8 * ws + u;
                if (tt < n) {
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const float pg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe[g]), tt));
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[g][e] = fmaf(pg, cv[u][e], o[g][e]);
                    }
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
            *(v4f*)(rob + (wv * G + g) * D + 4 * lane) = v4f{o[g][0], o[g][1], o[g][2], o[g][3]};
        lds_barrier();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float og = (rob[g * D + tid] + rob[(G + g) * D + tid]) + (rob[(2 * G + g) * D + tid] + rob[(3 * G + g) * D + tid]);
            if (tid == 0) {
                ml[2 * (slot + (size_t)g * nc)] = m[g];
                ml[2 * (slot + (size_t)g * nc) + 1] = l[g];
            }
            po[(slot + (size_t)g * nc) * D + tid] = og;
        }
        return;
    }

    // ---- span statistics per head: m, p = exp(s - m), l
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float v = -INFINITY;
        for (int i = tid; i < n; i += 256) v = fmaxf(v, scp[i][g]);
        v = wave_max_all(v);
        if (lane == 0) red[0][g][wv] = v;
    }
    lds_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = fmaxf(fmaxf(red[0][g][0], red[0][g][1]), fmaxf(red[0][g][2], red[0][g][3]));
    float sum[G];
#pragma unroll
    for (int g = 0; g < G; ++g) sum[g] = 0.0f;
    for (int i = tid; i < n; i += 256) {
        const v4f e4 = scp[i];
        float e[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int g = 0; g < G; ++g) {
            e[g] = combine_exp(e[g] - m[g]);
            sum[g] += e[g];
        }
        scp[i] = v4f{e[0], e[1], e[2], e[3]};
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float v = wave_sum_all(sum[g]);
        if (lane == 0) red[1][g][wv] = v;
    }
    lds_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g) l[g] = (red[1][g][0] + red[1][g][1]) + (red[1][g][2] + red[1][g][3]);

    // ---- o = sum of p * v over the span: per wave its tokens (the next
    // tile's values requested while a tile is summed), then the four waves
    // added in wave order through LDS (the score LDS, once read)
    float o[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[g][e] = 0.0f;
    for (int i = 0; i < nb; ++i) {
        float cv[8][4];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            vn[u].unpack(cv[u]);
            if (t0 + 32 * i + 8 * wv + u == p) {  // the position's own value, as stored
#pragma unroll
                for (int e = 0; e < 4; ++e) cv[u][e] = vrow[4 * lane + e];
            }
        }
        if (i + 1 < nb) load_values(i + 1);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int tt = 32 * i + 8 * wv + u;
            if (tt < n) {
                const v4f pr = scp[tt];
                const float pp[4] = {pr.x, pr.y, pr.z, pr.w};
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[g][e] = fmaf(pp[g], cv[u][e], o[g][e]);
            }
        }
    }
    lds_barrier();
    float* ro = (float*)scp;  // [wave][head][256]
#pragma unroll
    for (int g = 0; g < G; ++g)
        *(v4f*)(ro + (wv * G + g) * D + 4 * lane) = v4f{o[g][0], o[g][1], o[g][2], o[g][3]};
    lds_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float og = (ro[g * D + tid] + ro[(G + g) * D + tid]) + (ro[(2 * G + g) * D + tid] + ro[(3 * G + g) * D + tid]);
        if (tid == 0) {
            ml[2 * (slot + (size_t)g * nc)] = m[g];
            ml[2 * (slot + (size_t)g * nc) + 1] = l[g];
        }
        po[(slot + (size_t)g * nc) * D + tid] = og;
    }
}

// Grid (q_heads, B): the spans' partials of one head combined, gated.
// Every wave forms the spans' maximum and weighted exp-sum itself (lane l
// holds spans l, l + 64, ...), so the only barrier is the one before the
// four waves' value sums are added.  The weights e^(m_c - M) and the gate's
// sigmoid take combine_exp too.

__global__ __launch_bounds__(256) void attn_combine_kernel(AttnDecodeArgs a, int nc, const float* __restrict__ part) {
    constexpr int D = 256, CB = 16;  // spans per wave per batch of loads
    __shared__ v4f ow[4][D / 4];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const size_t nrow = (size_t)gridDim.y * a.nq * nc, slot = ((size_t)b * a.nq + h) * nc;
    const float* ml = part + 2 * slot;
    const v4f* po = (const v4f*)(part + 2 * nrow + slot * D) + lane;
    // every span has {m, l} (an empty one -inf, 0), so no load waits on the
    // position; wave w's first CB spans w, w + 4, ... (lane l: channels
    // 4l .. 4l+3) are requested with them
    float mc[4], lc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // nc <= 256
        const int c = lane + 64 * i;
        mc[i] = c < nc ? ml[2 * c] : -INFINITY;
        lc[i] = c < nc ? ml[2 * c + 1] : 0.0f;
    }
    const float gate = a.proj[(size_t)b * a.proj_stride + (size_t)h * 2 * D + D + tid];
    const int nw = (nc - wv + 3) / 4;  // this wave's spans
    v4f ov[CB];
#pragma unroll
    for (int k = 0; k < CB; ++k)
        if (k < nw) ov[k] = po[(size_t)(wv + 4 * k) * (D / 4)];
    const float mx = wave_max_all(fmaxf(fmaxf(mc[0], mc[1]), fmaxf(mc[2], mc[3])));
    float wc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wc[i] = mc[i] == -INFINITY ? 0.0f : combine_exp(mc[i] - mx);
    const float L = wave_sum_all((wc[0] * lc[0] + wc[1] * lc[1]) + (wc[2] * lc[2] + wc[3] * lc[3]));
    // wave w's sum over its spans in span order (span c's weight from lane
    // c % 64); an empty span (weight 0) is skipped, its o never written
    v4f o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < nw; k0 += CB) {
        if (k0) {
#pragma unroll
            for (int k = 0; k < CB; ++k)
                if (k0 + k < nw) ov[k] = po[(size_t)(wv + 4 * (k0 + k)) * (D / 4)];
        }
#pragma unroll
        for (int k = 0; k < CB; ++k) {
            if (k0 + k < nw) {
                const int c = wv + 4 * (k0 + k), q = c >> 6;
                const float src = q == 0 ? wc[0] : q == 1 ? wc[1] : q == 2 ? wc[2] : wc[3];
                const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(src), c & 63));
                if (wk != 0.0f) {
                    o.x = fmaf(wk, ov[k].x, o.x);
                    o.y = fmaf(wk, ov[k].y, o.y);
                    o.z = fmaf(wk, ov[k].z, o.z);
                    o.w = fmaf(wk, ov[k].w, o.w);
                }
            }
        }
    }
    ow[wv][lane] = o;
    __syncthreads();
    const float* of = (const float*)ow;  // [wave][channel]
    const float ot = (of[tid] + of[D + tid]) + (of[2 * D + tid] + of[3 * D + tid]);
    const float v = (ot / L) * (1.0f / (1.0f + combine_exp(-gate)));
    a.out[(size_t)b * a.out_stride + (size_t)h * D + tid] = v;
    if (tid == 0 && !(L >= 1.0f && L < INFINITY)) atomicOr(a.status, 8);
    if (a.xh) {  // batched rows: also the output projection's f16 A tiles
        const int k = h * D + tid, m = b, K = a.nq * D;
        const size_t at = xh_tile_index(m, k, K, gridDim.y);  // B rows = gridDim.y
        if (a.status && !(fabsf(v) <= 65504.0f)) atomicOr(a.status, 16);
        ((_Float16*)a.xh)[at] = (_Float16)v;
    }
}

// Grid (q_heads, 4, B), for up to 4 rows with more than 48 spans each (the
// batched rows' f16 tiles are not written here): workgroup
// (h, d, b) takes the 64 channels [64 d, 64 d + 64) of head h, so each
// workgroup reads a quarter of the head's partials.  Lane l of wave w holds
// channels 64 d + 4 (l & 15) .. + 3 and sums the spans r, r + 16, r + 32,
// ... in span order, r = 4 w + (l >> 4); the four lane groups of a wave are
// added as (g0 + g1) + (g2 + g3) and the four waves' sums in wave order.
// The statistics, weights and gate are those of attn_combine_kernel.
__global__ __launch_bounds__(256) void attn_combine_quarter_kernel(AttnDecodeArgs a, int nc, const float* __restrict__ part) {
    constexpr int D = 256, CB = 16;  // nc <= 256: at most 16 spans per lane
    __shared__ float ow[4][64];
    const int h = blockIdx.x, dq = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = 4 * wv + (lane >> 4);
    const size_t nrow = (size_t)gridDim.z * a.nq * nc, slot = ((size_t)b * a.nq + h) * nc;
    const float* ml = part + 2 * slot;
    const v4f* po = (const v4f*)(part + 2 * nrow + slot * D + 64 * dq) + (lane & 15);
    float mc[4], lc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = lane + 64 * i;
        mc[i] = c < nc ? ml[2 * c] : -INFINITY;
        lc[i] = c < nc ? ml[2 * c + 1] : 0.0f;
    }
    const float gate = tid < 64 ? a.proj[(size_t)b * a.proj_stride + (size_t)h * 2 * D + D + 64 * dq + tid] : 0.0f;
    const int nw = (nc - r + 15) >> 4;  // this lane's spans (r < 16 <= nc)
    v4f ov[CB];
#pragma unroll
    for (int k = 0; k < CB; ++k)
        if (k < nw) ov[k] = po[(size_t)(r + 16 * k) * (D / 4)];
    const float mx = wave_max_all(fmaxf(fmaxf(mc[0], mc[1]), fmaxf(mc[2], mc[3])));
    float wc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wc[i] = mc[i] == -INFINITY ? 0.0f : combine_exp(mc[i] - mx);
    const float L = wave_sum_all((wc[0] * lc[0] + wc[1] * lc[1]) + (wc[2] * lc[2] + wc[3] * lc[3]));
    v4f o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < CB; ++k) {
        // span c = r + 16 k sits in lane c & 63 of wc[k >> 2] (r < 16)
        const int c = r + 16 * k;
        const float wk = __shfl(wc[k >> 2], c & 63, kWave);
        if (k < nw && wk != 0.0f) {
            o.x = fmaf(wk, ov[k].x, o.x);
            o.y = fmaf(wk, ov[k].y, o.y);
            o.z = fmaf(wk, ov[k].z, o.z);
            o.w = fmaf(wk, ov[k].w, o.w);
        }
    }
    float e[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        e[i] += __shfl_xor(e[i], 16, kWave);
        e[i] += __shfl_xor(e[i], 32, kWave);
    }
    if (lane < 16) *(v4f*)&ow[wv][4 * lane] = v4f{e[0], e[1], e[2], e[3]};
    __syncthreads();
    if (tid >= 64) return;
    const float ot = (ow[0][tid] + ow[1][tid]) + (ow[2][tid] + ow[3][tid]);
    const float v = (ot / L) * (1.0f / (1.0f + combine_exp(-gate)));
    a.out[(size_t)b * a.out_stride + (size_t)h * D + 64 * dq + tid] = v;
    if (tid == 0 && !(L >= 1.0f && L < INFINITY)) atomicOr(a.status, 8);
}

// RoPE angles of positions [0, n): entry 32 p + t is (cos, sin) of p times
// theta_scale^t, the angle formed by repeated f32 products as the decode
// kernels form it, with the same correctly rounded cos and sin.
__global__ __launch_bounds__(256) void rope_table_kernel(float2* __restrict__ tab, int n, float theta_scale) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n * 32) return;
    const int p = i >> 5, t = i & 31;
    float angle = (float)p;
    for (int q = 0; q < t; ++q) angle *= theta_scale;
    tab[i] = make_float2(cr_cosf(angle), cr_sinf(angle));
}

hipError_t rope_table(float* tab, size_t n, float theta_scale, hipStream_t s) {
    if (!tab || n == 0 || n > (1u << 24)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n * 32 + 255) / 256)), dim3(256), 0, s, (float2*)tab, (int)n,
                       theta_scale);
    return hipGetLastError();
}

hipError_t attn_decode_split(const AttnDecodeArgs& a, size_t B, float* part, hipStream_t s) {
    if (!attn_split_supported(B, a.nq, a.nkv, (size_t)a.max_ctx) || !part) return hipErrorInvalidValue;
    const int G = a.nq / a.nkv, nc = attn_split_chunks(B, a.nkv, (size_t)a.max_ctx);
    const int span = attn_split_span(B, a.nkv, (size_t)a.max_ctx);
    const dim3 g((unsigned)nc, (unsigned)a.nkv, (unsigned)B);
#define ZG_SP(KV)                                                                                            \
    switch (G) {                                                                                             \
    case 1: hipLaunchKernelGGL((attn_split_kernel<KV, 1>), g, dim3(256), 0, s, a, nc, span, part); break;    \
    case 2: hipLaunchKernelGGL((attn_split_kernel<KV, 2>), g, dim3(256), 0, s, a, nc, span, part); break;    \
    case 3: hipLaunchKernelGGL((attn_split_kernel<KV, 3>), g, dim3(256), 0, s, a, nc, span, part); break;    \
    default: hipLaunchKernelGGL((attn_split_kernel<KV, 4>), g, dim3(256), 0, s, a, nc, span, part); break;   \
    }
    if (a.kv_bf16) {
        ZG_SP(uint16_t)
    } else {
        ZG_SP(float)
    }
#undef ZG_SP
    if (B <= 4 && nc > 48 && !a.xh)  // a quarter of the head's channels per workgroup: a quarter of its partials to read
        hipLaunchKernelGGL(attn_combine_quarter_kernel, dim3((unsigned)a.nq, 4, (unsigned)B), dim3(256), 0, s, a, nc,
                           (const float*)part);
    else
        hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)a.nq, (unsigned)B), dim3(256), 0, s, a, nc,
                           (const float*)part);
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

// The publication rule of a decode step (QwenDenseCpu::commit,
// model-qwen35/src/lib.rs:1211-1225: the draft becomes the state only when
// the whole step succeeded): with the status word clear, row b's position
// moves on and its GDN state half flips to the draft the step wrote; else
// nothing changes, so a failed step leaves the published state as it was.
__device__ __forceinline__ void commit_row(const StepCommit& c, bool ok, int b) {
    if (!ok) return;
    const int np = c.pos[b] + 1;
    c.pos[b] = np;
    c.ntok[b] = np + 1;
    if (c.cur) c.cur[b] ^= 1;
}

// The same rule with the status word, position and half read when the
// kernel starts (no kernel of the step writes them while the greedy
// kernels run), so those reads overlap the partials' instead of following
// the reduction.
struct CommitRead {
    int status = 0, pos = 0, cur = 0;
};
__device__ __forceinline__ CommitRead commit_read(const StepCommit& c, const int* status, int b) {
    CommitRead r;
    if (c.pos) {
        r.status = *status;
        r.pos = c.pos[b];
        if (c.cur) r.cur = c.cur[b];
    }
    return r;
}
__device__ __forceinline__ void commit_row(const StepCommit& c, const CommitRead& r, int b) {
    if (!c.pos || r.status != 0) return;
    const int np = r.pos + 1;
    c.pos[b] = np;
    c.ntok[b] = np + 1;
    if (c.cur) c.cur[b] = r.cur ^ 1;
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pmax, const int* __restrict__ pidx,
                                                          uint32_t* __restrict__ greedy, const int* __restrict__ status,
                                                          StepCommit c) {
    const int b = blockIdx.x, lane = threadIdx.x;
    float m = lane < kArgBlocks ? pmax[b * kArgBlocks + lane] : -INFINITY;
    int mi = lane < kArgBlocks ? pidx[b * kArgBlocks + lane] : 0x7fffffff;
    const CommitRead cr = commit_read(c, status, b);
    for (int off = 32; off > 0; off >>= 1) argmax_merge(m, mi, __shfl_xor(m, off, 64), __shfl_xor(mi, off, 64));
    if (lane == 0) {
        greedy[b] = mi == 0x7fffffff ? 0u : (uint32_t)mi;
        commit_row(c, cr, b);
    }
}

__global__ __launch_bounds__(64) void commit_step_kernel(StepCommit c, const int* __restrict__ status, int B) {
    const int b = threadIdx.x;
    if (b < B) commit_row(c, *status == 0, b);
}

hipError_t argmax_step(const float* logits, size_t V, size_t ld, size_t B, uint32_t* greedy, int* status, float* pmax,
                       int* pidx, const StepCommit* commit, hipStream_t s) {
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks, (unsigned)B), dim3(256), 0, s, logits, (int)V, ld, status,
                       pmax, pidx);
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)B), dim3(64), 0, s, pmax, pidx, greedy, status,
                       commit ? *commit : StepCommit{});
    return hipGetLastError();
}

// One row's greedy id from `parts` (max, first index) partials, then the
// commit rule of argmax_final_kernel.
__global__ __launch_bounds__(256) void argmax_parts_kernel(const float* __restrict__ pmax, const int* __restrict__ pidx,
                                                           int parts, uint32_t* __restrict__ greedy,
                                                           const int* __restrict__ status, StepCommit c) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    // the first 8 x 256 partials requested at once (one round trip for the
    // one-row LM head's 2048), then merged: the merge keeps the largest
    // value and on a tie the smaller index, so its order does not matter
    constexpr int PER = 8;
    float pv[PER];
    int pi[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int i = tid + 256 * q;
        pv[q] = i < parts ? pmax[min(i, parts - 1)] : -INFINITY;
        pi[q] = i < parts ? pidx[min(i, parts - 1)] : 0x7fffffff;
    }
    const CommitRead cr = commit_read(c, status, 0);
#pragma unroll
    for (int q = 0; q < PER; ++q) argmax_merge(best, bi, pv[q], pi[q]);
    for (int i = tid + 256 * PER; i < parts; i += 256) argmax_merge(best, bi, pmax[i], pidx[i]);
    for (int off = 32; off > 0; off >>= 1) argmax_merge(best, bi, __shfl_xor(best, off, 64), __shfl_xor(bi, off, 64));
    if (lane == 0) {
        sv[wv] = best;
        si[wv] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) argmax_merge(best, bi, sv[w], si[w]);
        greedy[0] = bi == 0x7fffffff ? 0u : (uint32_t)bi;
        commit_row(c, cr, 0);
    }
}

hipError_t argmax_final(const float* pmax, const int* pidx, int parts, uint32_t* greedy, int* status,
                        const StepCommit* commit, hipStream_t s) {
    if (parts <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_parts_kernel, dim3(1), dim3(256), 0, s, pmax, pidx, parts, greedy, status,
                       commit ? *commit : StepCommit{});
    return hipGetLastError();
}

hipError_t commit_step(const StepCommit& c, const int* status, size_t B, hipStream_t s) {
    if (B == 0 || B > 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(commit_step_kernel, dim3(1), dim3(64), 0, s, c, status, (int)B);
    return hipGetLastError();
}

size_t argmax_partials(size_t B) { return B * kArgBlocks; }


}  // namespace zg
