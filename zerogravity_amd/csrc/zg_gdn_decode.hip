// Resident GDN decode step (conv ring, L2, gates, recurrence).
#include "zg_decode_common.hpp"

namespace zg {

// ============================================================ GDN decode

// Grid (H * 4, B), 256 threads: workgroup (h, quarter) owns value columns
// quarter*32 .. +31 of head h.  The causal conv keeps a 4-slot ring per
// channel: the token at position p is written to slot p%4 while the taps
// x[p-3], x[p-2], x[p-1] are read from the other three slots, so the
// workgroups of one head that all read the q/k channels never race with the
// one (quarter 0) that writes them.  conv: cpu/src/ops/gdn.rs:7-44 (left to
// right, no FMA) + SiLU (forward.rs:548); L2, gates and recurrence as
// gdn_recurrent_kernel<true>.
// HEAD: one workgroup of 4 x 256 threads per (head, row) -- quarter q is
// threads 256q.. -- sharing the conv, norms and gates, and finishing with
// the gated RMSNorm of the head's output into the next GEMM's f16 tiles.
template <bool HEAD>
__global__ __launch_bounds__(HEAD ? 1024 : 256) void gdn_decode_kernel(GdnDecodeArgs a) {
    constexpr int D = 128;
    __shared__ float qk[2 * D];
    __shared__ float vv[HEAD ? D : 32];
    __shared__ float gates[2];
    __shared__ float ob[HEAD ? D : 1];
    const int h = HEAD ? blockIdx.x : blockIdx.x >> 2, b = blockIdx.y;
    const int quarter = HEAD ? (int)(threadIdx.x >> 8) : (int)(blockIdx.x & 3);
    const int tid = threadIdx.x & 255;
    const int W = a.H * D;
    const int lane = tid & 63, wv = tid >> 6;
    const int jl = wv * 8 + (lane >> 3);  // column within the quarter
    const int j = quarter * 32 + jl;
    const int s = lane & 7;
    const float* xin = a.proj + (size_t)b * a.proj_stride;
    float* ring = a.ring + (size_t)b * 3 * W * 4;
    // one workgroup per quarter: every argument the prologue uses in one
    // round trip (loaded where first used, they would take several), the
    // conv and gate inputs requested, then the row's state half and
    // position in the next round trip (a scalar wait covers every scalar
    // load in flight)
    if constexpr (!HEAD)
        asm volatile("" ::"s"(a.norm), "s"(a.gated), "s"(a.state), "s"(a.cur), "s"(a.pos), "s"(a.dt), "s"(a.ssm_a),
                     "s"(a.state_row), "s"(a.state_half), "s"(a.conv_w), "s"(a.H));
    // The conv and gate inputs are requested first, then this thread's 16
    // state values (the bulk of the traffic): a wave's loads complete in
    // issue order, so the conv, norms and gates wait only for their own
    // inputs while the state is in flight.  HEAD: threads 0..255 own the q/k
    // channels and 256..383 the value channels, one each; else every thread
    // owns q/k channel tid and threads < 32 also value channel
    // quarter*32 + tid.  Loads are unconditional (clamped in range) and each
    // sum is used on two paths, so that none moves behind the state loads.
    struct ConvIn {
        v4f r, w;
        float x;
    };
    auto conv_load = [&](int ch) {
        ConvIn c;
        c.r = *(const v4f*)(ring + (size_t)ch * 4);
        c.w = *(const v4f*)(a.conv_w + (size_t)ch * 4);
        c.x = xin[ch];
        return c;
    };
    const int ch_qk = tid < D ? h * D + tid : W + h * D + (tid - D);
    const int vc = HEAD ? max(0, min((int)threadIdx.x - 256, D - 1)) : quarter * 32 + (tid & 31);
    const int ch_v = 2 * W + h * D + vc;
    const int ch_a = HEAD && threadIdx.x >= 256 ? ch_v : ch_qk;
    const ConvIn in_a = conv_load(ch_a);
    ConvIn in_v;
    if constexpr (!HEAD) in_v = conv_load(ch_v);
    const float g_a = xin[4 * W + h], g_b = xin[4 * W + a.H + h], g_dt = a.dt[h], g_sa = a.ssm_a[h];
    // HEAD: wave 0's gated-norm inputs, requested now so that the tail does
    // not wait for them (loads are not moved across the barriers below)
    v4f tail_g = v4f{0.0f, 0.0f, 0.0f, 0.0f}, tail_z = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (HEAD && threadIdx.x < 64) {
        const int t = threadIdx.x & 31;
        tail_g = *(const v4f*)(a.norm + 4 * t);
        tail_z = *(const v4f*)(xin + 3 * W + h * D + 4 * t);
    }
    // one workgroup per quarter with `gated`: the column's z and norm
    // weight for the output projection's product, requested now as well
    float gz = 0.0f, gg = 0.0f;
    if (!HEAD && a.gated) {
        gz = xin[3 * W + h * D + j];
        gg = a.norm[j];
    }
    // the row's state: read from half cur[b], written to the other half (the
    // draft the step's commit publishes), or in place without cur; one
    // workgroup per quarter reads cur and pos through the scalar unit
    // (nothing writes them while the step's kernels run)
    typedef const __attribute__((address_space(4))) int* const_int;
    const int cb = !a.cur ? 0 : HEAD ? a.cur[b] : ((const_int)a.cur)[b];
    const int pq = HEAD ? 0 : ((const_int)a.pos)[b];
    const size_t row_floats = a.state_row ? a.state_row : (size_t)a.H * D * D;
    const size_t within = ((size_t)h * D + j) * D + 4 * s;
    const float* col = a.state + (size_t)b * row_floats + (size_t)cb * a.state_half + within;
    float* col_out = a.state + (size_t)b * row_floats + (a.cur ? (size_t)(1 - cb) * a.state_half : 0) + within;
    // a row's state (1 MB per layer) is read once and written once per step
    // and the step's states outgrow the 256 MB Infinity Cache from B = 8
    // on: non-temporal loads and stores leave L2 and the Infinity Cache to
    // the step's other operands
    v4f sv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) sv[c] = __builtin_nontemporal_load((const v4f*)(col + 32 * c));
    const int p = HEAD ? a.pos[b] : pq;
    const int s0 = (p + 1) & 3, s1 = (p + 2) & 3, s2 = (p + 3) & 3, sw = p & 3;
    auto conv = [&](const ConvIn& c) {
        const float hv[4] = {c.r.x, c.r.y, c.r.z, c.r.w};
        const float t0 = hv[s0] * c.w.x;
        const float t1 = hv[s1] * c.w.y;
        const float t2 = hv[s2] * c.w.z;
        const float t3 = c.x * c.w.w;
        float acc = t0 + t1;
        acc = acc + t2;
        acc = acc + t3;
        return acc;
    };
    if constexpr (HEAD) {
        const float cv = conv(in_a);
        if (threadIdx.x < 256) {
            qk[threadIdx.x] = ggml_silu(cv);
            ring[(size_t)ch_qk * 4 + sw] = in_a.x;
        } else if (threadIdx.x < 256 + D) {
            vv[vc] = ggml_silu(cv);
            ring[(size_t)ch_v * 4 + sw] = in_a.x;
        }
    } else {
        qk[tid] = ggml_silu(conv(in_a));
        if (quarter == 0) ring[(size_t)ch_qk * 4 + sw] = in_a.x;
        if (tid < 32) {
            vv[tid] = ggml_silu(conv(in_v));
            ring[(size_t)ch_v * 4 + sw] = in_v.x;
        }
    }
    // the head's gates (f64-evaluated transcendentals) once per workgroup,
    // by the wave without value channels, unless the projection formed them
    if (!a.gates_formed && tid == 192 && (!HEAD || quarter == 0)) {
        float gn, bt, sp, gr;
        gdn_coef(g_a, g_b, g_dt, g_sa, gn, bt, sp, gr);
        gates[0] = gn;
        gates[1] = bt;
    }
    lds_barrier();  // the state loads stay in flight

    const float dsq = 1.0f / sqrtf((float)D);
    const float eps_d = a.eps / (float)D;
    const float gain = a.gates_formed ? g_a : gates[0], beta = a.gates_formed ? g_b : gates[1];
    const float vj = vv[HEAD ? j : jl];
    float cv[4][4];
    float o;
    if constexpr (HEAD) {
        // the same arithmetic with q and k re-read from LDS where they are
        // used rather than held in registers across the recurrence: 1024
        // threads then fit in 64 registers, two (head, row) workgroups per CU
        auto qk4 = [&](int base, int c) { return *(const v4f*)(qk + base + 32 * c + 4 * s); };
        double sq = 0.0, sk = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const v4f qv = qk4(0, c), kv = qk4(D, c);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float a2 = qv[t] * qv[t];
                const float b2 = kv[t] * kv[t];
                sq += (double)a2;
                sk += (double)b2;
            }
        }
        sq = group8_sum_all(sq);
        sk = group8_sum_all(sk);
        const float iq = 1.0f / sqrtf((float)(sq / (double)D) + eps_d);
        const float ik = 1.0f / sqrtf((float)(sk / (double)D) + eps_d);
        auto normed = [&](int base, float inv, float (&r)[4][4]) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const v4f v = qk4(base, c);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float tv = v[t] * inv;
                    r[c][t] = tv * dsq;
                }
            }
        };
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const v4f v = sv[c];
            cv[c][0] = v.x * gain; cv[c][1] = v.y * gain; cv[c][2] = v.z * gain; cv[c][3] = v.w * gain;
        }
        // the empty asm with a memory clobber makes the compiler load q and
        // k again below instead of keeping the values read for the sums
        asm volatile("" ::: "memory");
        float k[4][4];
        normed(D, ik, k);
        const float prev = column_dot(cv, k);
        const float delta = (vj - prev) * beta;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) cv[c][t] = fmaf(k[c][t], delta, cv[c][t]);
        asm volatile("" ::: "memory");
        float q[4][4];
        normed(0, iq, q);
        o = column_dot(cv, q);
    } else {
        float q[4][4], k[4][4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                q[c][t] = qk[32 * c + 4 * s + t];
                k[c][t] = qk[D + 32 * c + 4 * s + t];
            }
        // two-stage L2 (forward.rs:564-576)
        double sq = 0.0, sk = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float a2 = q[c][t] * q[c][t];
                const float b2 = k[c][t] * k[c][t];
                sq += (double)a2;
                sk += (double)b2;
            }
        sq = group8_sum_all(sq);
        sk = group8_sum_all(sk);
        const float iq = 1.0f / sqrtf((float)(sq / (double)D) + eps_d);
        const float ik = 1.0f / sqrtf((float)(sk / (double)D) + eps_d);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float tq = q[c][t] * iq;
                q[c][t] = tq * dsq;
                const float tk = k[c][t] * ik;
                k[c][t] = tk * dsq;
            }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const v4f v = sv[c];
            cv[c][0] = v.x * gain; cv[c][1] = v.y * gain; cv[c][2] = v.z * gain; cv[c][3] = v.w * gain;
        }
        const float prev = column_dot(cv, k);
        const float delta = (vj - prev) * beta;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t) cv[c][t] = fmaf(k[c][t], delta, cv[c][t]);
        o = column_dot(cv, q);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) __builtin_nontemporal_store(v4f{cv[c][0], cv[c][1], cv[c][2], cv[c][3]}, (v4f*)(col_out + 32 * c));
    const float core = o * a.scale;
    if (s == 0) a.core[(size_t)b * W + h * D + j] = core;
    // (core * norm) * silu(z): PRO_GATED's product (forward.rs:586-594
    // before the 1/rms), once per element instead of in every workgroup of
    // the output projection
    if (!HEAD && a.gated && s == 0) a.gated[(size_t)b * W + h * D + j] = (core * gg) * ggml_silu(gz);
    if constexpr (HEAD) {
        // gated RMSNorm of the head (forward.rs:586-594) in act16_kernel's
        // arithmetic: 32 lanes of wave 0, elements 4t..4t+3 each, f64 sum of
        // f32 squares over the group, then ((e * inv) * gamma) * silu(z)
        if (s == 0) ob[j] = o * a.scale;
        __syncthreads();
        if (threadIdx.x < 64) {  // the whole wave runs the 32-lane tree; lanes 32.. repeat the group
            const int t = threadIdx.x & 31;
            float e[4];
            double sq = 0.0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                e[i] = ob[4 * t + i];
                const float q2 = e[i] * e[i];
                sq += (double)q2;
            }
            sq = group_sum_last<32>(sq);
            sq = __shfl(sq, ((int)threadIdx.x & 32) | 31, 64);
            const float gi = rms_inv(sq, D, a.eps);
            const float gg[4] = {tail_g.x, tail_g.y, tail_g.z, tail_g.w};
            const float zz[4] = {tail_z.x, tail_z.y, tail_z.z, tail_z.w};
            typedef _Float16 h4v __attribute__((ext_vector_type(4)));
            h4v hv4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float y = ((e[i] * gi) * gg[i]) * ggml_silu(zz[i]);
                if (a.status && threadIdx.x < 32 && !(fabsf(y) <= 65504.0f)) atomicOr(a.status, 16);
                hv4[i] = (_Float16)y;
            }
            const int k = h * D + 4 * t, m = b;
            const size_t at = xh_tile_index(m, k, W, gridDim.y);  // B rows = gridDim.y; 4 columns in one 8-run
            if (threadIdx.x < 32) *(h4v*)((_Float16*)a.xh + at) = hv4;
        }
    }
}

hipError_t gdn_decode(const GdnDecodeArgs& a, size_t B, hipStream_t s) {
    if (a.H <= 0 || B == 0 || (a.gated && !a.norm)) return hipErrorInvalidValue;
    if (a.xh) {
        if (!a.norm || (a.H * 128) % 256) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gdn_decode_kernel<true>, dim3((unsigned)a.H, (unsigned)B), dim3(1024), 0, s, a);
    } else {
        hipLaunchKernelGGL(gdn_decode_kernel<false>, dim3((unsigned)(a.H * 4), (unsigned)B), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace zg
