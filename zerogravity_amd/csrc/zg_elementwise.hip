// Normalisation and pointwise kernels of the decode path (gfx950).
//   RMSNorm / grouped RMSNorm: model-qwen35/src/lib.rs:263-306
//   GGML polynomial exp / SiLU: cpu/src/ops.rs:317-355, lib.rs:310-321
//   Add / SigmoidGate: lib.rs:1258-1271, 324-326
#include "zg_device.hpp"
#include "zg_internal.hpp"
#include "zg_pointwise.hpp"

namespace zg {

// One workgroup per group; f64 sum of f32-rounded squares, f32 mean,
// inv = 1/sqrtf(mean + eps), y = (x*inv)*w with w shared by every group.
__global__ __launch_bounds__(256) void rms_group_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        int width, float eps, float* __restrict__ out) {
    __shared__ double red[4];
    __shared__ float inv_s;
    const size_t g = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xg = x + g * width;
    double s = 0.0;
    for (int i = tid; i < width; i += 256) {
        float v = xg[i];
        float sq = v * v;
        s += (double)sq;
    }
    s = wave_sum_xor<double>(s, 64);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        double total = (red[0] + red[1]) + (red[2] + red[3]);
        float mean = (float)(total / (double)width);
        float root = sqrtf(mean + eps);
        inv_s = 1.0f / root;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = tid; i < width; i += 256) {
        float t = xg[i] * inv;
        out[g * width + i] = t * w[i];
    }
}

__global__ void silu_kernel(const float* __restrict__ x, const float* __restrict__ m, size_t n,
                            float* __restrict__ out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float y = ggml_silu(x[i]);
    out[i] = m ? m[i] * y : y;
}

__global__ void binary_kernel(int kind, const float* __restrict__ a, const float* __restrict__ b, size_t n,
                              float* __restrict__ out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = kind == 0 ? a[i] + b[i] : a[i] * source_sigmoid(b[i]);
}

hipError_t rms_groups(const float* x, const float* w, size_t width, size_t groups, float eps, float* out,
                      hipStream_t s) {
    if (width == 0 || groups == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_group_kernel, dim3((unsigned)groups), dim3(256), 0, s, x, w, (int)width, eps, out);
    return hipGetLastError();
}

hipError_t silu(const float* x, const float* m, size_t n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(silu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, m, n, out);
    return hipGetLastError();
}

hipError_t binary(int kind, const float* a, const float* b, size_t n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(binary_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kind, a, b, n, out);
    return hipGetLastError();
}

}  // namespace zg
