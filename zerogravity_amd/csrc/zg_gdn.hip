// Gated DeltaNet decode kernels (gfx950): causal conv + SiLU, per-head
// coefficients, and the recurrent state update with the q/k L2 norm fused.
//
// Reference semantics (zerogravity repository):
//   conv step           cpu/src/ops/gdn.rs:7-44
//   coefficients        model-qwen35/src/lib.rs:339-362 (softplus :328-336, sigmoid :324-326)
//   q/k L2 norm         forward.rs:564-576 (grouped RMS, gamma 1/sqrt(d), eps/d)
//   recurrence          lib.rs:1446-1499 (value-major state, per column j:
//                       decay, prev = col.k, delta = (v_j - prev)*beta,
//                       col += k*delta, o_j = (col.q)*scale)
//
// State layout in HBM: [row][head][j (value)][i (key)] f32, the CPU layout
// (lib.rs:81-83).  One column j is 512 contiguous bytes; eight lanes own a
// column, sixteen keys each, so a wavefront streams 8 columns = 4 KB with
// 16-byte loads and writes them back in place: the state is read once and
// written once per token (the roofline of this kernel).
#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

// ---------------------------------------------------------------- conv

// One thread per (row, channel).  raw = h0*w0 + h1*w1 + h2*w2 + x*w3 with
// left-to-right f32 rounding (no FMA), history <- [h1, h2, x]; out is
// silu(raw) when apply_silu, else raw.
__global__ void gdn_conv_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ hist,
                                float* __restrict__ out, int C, int rows, int apply_silu, size_t x_stride,
                                size_t hist_stride, size_t out_stride) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)C * rows) return;
    const size_t b = i / C, c = i % C;
    float* h = hist + b * hist_stride + c * 3;
    const float xv = x[b * x_stride + c];
    const float h0 = h[0], h1 = h[1], h2 = h[2];
    const float t0 = h0 * w[c * 4 + 0];
    const float t1 = h1 * w[c * 4 + 1];
    const float t2 = h2 * w[c * 4 + 2];
    const float t3 = xv * w[c * 4 + 3];
    float raw = t0 + t1;
    raw = raw + t2;
    raw = raw + t3;
    h[0] = h1;
    h[1] = h2;
    h[2] = xv;
    out[b * out_stride + c] = apply_silu ? ggml_silu(raw) : raw;
}

hipError_t gdn_conv(const float* x, const float* w, float* hist, float* out, size_t C, size_t rows, int apply_silu,
                    size_t x_stride, size_t hist_stride, size_t out_stride, hipStream_t s) {
    const size_t n = C * rows;
    hipLaunchKernelGGL(gdn_conv_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, w, hist, out, (int)C,
                       (int)rows, apply_silu, x_stride, hist_stride, out_stride);
    return hipGetLastError();
}

// ---------------------------------------------------------- coefficients


__global__ void gdn_coef_kernel(const float* __restrict__ alpha, const float* __restrict__ beta,
                                const float* __restrict__ dt, const float* __restrict__ a, int H,
                                float* __restrict__ gain, float* __restrict__ beta_out, float* __restrict__ sp,
                                float* __restrict__ gr) {
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= H) return;
    float g, b, s, r;
    gdn_coef(alpha[h], beta[h], dt[h], a[h], g, b, s, r);
    gain[h] = g;
    beta_out[h] = b;
    sp[h] = s;
    gr[h] = r;
}

hipError_t gdn_coefficients(const float* alpha, const float* beta, const float* dt, const float* a, size_t H,
                            float* gain, float* beta_out, float* sp, float* gr, hipStream_t s) {
    hipLaunchKernelGGL(gdn_coef_kernel, dim3((unsigned)((H + 63) / 64)), dim3(64), 0, s, alpha, beta, dt, a, (int)H,
                       gain, beta_out, sp, gr);
    return hipGetLastError();
}

// ------------------------------------------------------------- recurrence

// Grid: x = heads * (d/8) / 4 workgroups of 4 waves, y = rows.  Wave w of
// the grid owns columns j0..j0+7 of one head (lane = (j - j0) * 8 + s).
//
// FUSED (model path): q, k, v come from the conv+SiLU output
// mixed[row] = [q (H*d) | k (H*d) | v (H*d)], q and k are L2-normalised here
// (f64 sum of f32 squares over the head, f32 mean, 1/sqrtf(mean + eps/d),
// then (x*inv)*(1/sqrt d)), and gain/beta come from the raw alpha/beta
// projections, ssm_dt and ssm_a.
// Not FUSED (region path): q, k, v are given, as are gain and beta per head.
template <bool FUSED>
__global__ __launch_bounds__(256) void gdn_recurrent_kernel(
    const float* __restrict__ qsrc, const float* __restrict__ ksrc, const float* __restrict__ vsrc, size_t src_stride,
    const float* __restrict__ alpha, const float* __restrict__ beta_p, size_t coef_stride,
    const float* __restrict__ dt, const float* __restrict__ a, float eps, float scale,
    const float* __restrict__ scale_h, float* __restrict__ state, float* __restrict__ out, size_t out_stride, int H) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);  // wave index within the row
    const int h = gw / (D / 8);
    const int j = (gw % (D / 8)) * 8 + (lane >> 3);
    const int s = lane & 7;
    const size_t row = blockIdx.y;
    if (h >= H) return;

    const float* qrow = qsrc + row * src_stride + (size_t)h * D + 4 * s;
    const float* krow = ksrc + row * src_stride + (size_t)h * D + 4 * s;
    float q[4][4], k[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const v4f qa = *(const v4f*)(qrow + 32 * c);
        const v4f ka = *(const v4f*)(krow + 32 * c);
        q[c][0] = qa.x; q[c][1] = qa.y; q[c][2] = qa.z; q[c][3] = qa.w;
        k[c][0] = ka.x; k[c][1] = ka.y; k[c][2] = ka.z; k[c][3] = ka.w;
    }
    float gain, beta;
    if (FUSED) {
        // two-stage L2 (forward.rs:564-576): the 8 lanes of a column cover the head
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
        sq = wave_sum_xor<double>(sq, 8);
        sk = wave_sum_xor<double>(sk, 8);
        const float dsq = 1.0f / sqrtf((float)D);
        const float eps_d = eps / (float)D;
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
        float sp, gr;
        gdn_coef(alpha[row * coef_stride + h], beta_p[row * coef_stride + h], dt[h], a[h], gain, beta, sp, gr);
    } else {
        gain = alpha[row * coef_stride + h];
        beta = beta_p[row * coef_stride + h];
        if (scale_h) scale = scale_h[row * coef_stride + h];
    }
    const float vj = vsrc[row * src_stride + (size_t)h * D + j];
    float* col = state + ((row * H + h) * D + j) * D + 4 * s;
    float cv[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const v4f v = *(const v4f*)(col + 32 * c);
        cv[c][0] = v.x * gain; cv[c][1] = v.y * gain; cv[c][2] = v.z * gain; cv[c][3] = v.w * gain;
    }
    const float prev = column_dot(cv, k);
    const float delta = (vj - prev) * beta;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) cv[c][t] = fmaf(k[c][t], delta, cv[c][t]);
    const float o = column_dot(cv, q);
#pragma unroll
    for (int c = 0; c < 4; ++c) *(v4f*)(col + 32 * c) = v4f{cv[c][0], cv[c][1], cv[c][2], cv[c][3]};
    if (s == 0) out[row * out_stride + (size_t)h * D + j] = o * scale;
}

hipError_t gdn_recurrent(bool fused, const float* q, const float* k, const float* v, size_t src_stride,
                         const float* alpha, const float* beta, size_t coef_stride, const float* dt, const float* a,
                         float eps, float scale, const float* scale_h, float* state, float* out, size_t out_stride,
                         size_t H, size_t D, size_t rows, hipStream_t s) {
    if (D != 128 || H == 0 || rows == 0) return hipErrorInvalidValue;
    dim3 grid((unsigned)(H * (D / 8) / 4), (unsigned)rows);
    if (fused)
        hipLaunchKernelGGL(gdn_recurrent_kernel<true>, grid, dim3(256), 0, s, q, k, v, src_stride, alpha, beta,
                           coef_stride, dt, a, eps, scale, scale_h, state, out, out_stride, (int)H);
    else
        hipLaunchKernelGGL(gdn_recurrent_kernel<false>, grid, dim3(256), 0, s, q, k, v, src_stride, alpha, beta,
                           coef_stride, dt, a, eps, scale, scale_h, state, out, out_stride, (int)H);
    return hipGetLastError();
}

}  // namespace zg
