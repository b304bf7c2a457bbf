// Measurement kernels for the launch and hand-off floors of this GPU
// (libzg_probe.so; bench.py --workload floors).  Nothing on the hot path
// calls them: they time what the design of the decode step rests on.
//
//   zg_probe_chain     a HIP graph of dependent launches, each reading the
//                      previous launch's K-float output (loads issued at once)
//   zg_probe_handoff   the same dependency inside one persistent cooperative
//                      kernel: LL words (value | flag << 32, agent-scope
//                      atomics), or a counter with agent-scope data, or a
//                      counter with release/acquire fences.  Every spin is
//                      bounded (50 ms of s_memrealtime) and checks an abort
//                      word, so a failed protocol ends the kernel.
//   zg_probe_stream    GEMV-shaped launches in a graph: read a K-float
//                      activation, stream this launch's weight bytes
//                      (16-byte nontemporal loads), write one float per wave;
//                      weights rotate over more than the 256 MB MALL
//   zg_probe_rmw       in-place read-modify-write of a buffer (the GDN state
//                      traffic pattern), rotating over copies
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr uint64_t kSpinTicks = 5000000;  // 50 ms at the 100 MHz s_memrealtime clock

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ v4u ld16_agent(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);  // sc1: coherent at agent scope
}

template <int NPT>
__global__ __launch_bounds__(256) void chain_kernel(const float* __restrict__ in, float* __restrict__ out, int N) {
    __shared__ float red[4];
    v4f q[NPT];
#pragma unroll
    for (int j = 0; j < NPT; ++j) q[j] = *(const v4f*)(in + 4 * (threadIdx.x + 256 * j));
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) s += (q[j].x + q[j].y) + (q[j].z + q[j].w);
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const int per = N / gridDim.x;
    if ((int)threadIdx.x < per) out[blockIdx.x * per + threadIdx.x] = (red[0] + red[1] + red[2] + red[3]) * 1e-3f;
}

// MODE 0: LL words; 1: counter + agent-scope data; 2: counter + fences
template <int MODE, int NPT>
__global__ __launch_bounds__(256) void handoff_kernel(unsigned* buf, unsigned* ctr, unsigned* abort_w, int P, int N,
                                                      unsigned epoch, float* out) {
    __shared__ float red[4];
    __shared__ int bad;
    const int tid = threadIdx.x, nwg = gridDim.x, w = blockIdx.x, per = N / nwg;
    if (tid == 0) bad = 0;
    __syncthreads();
    float carry = 1.0f;
    for (int p = 0; p < P; ++p) {
        const unsigned flag = epoch * 4096u + (unsigned)p + 1u;
        unsigned* b = buf + (size_t)(p & 1) * 2 * N;
        if (tid < per) {
            const float v = carry * 0.5f + (float)(w * per + tid) * 1e-6f;
            if (MODE == 0) st_agent64((uint64_t*)b + w * per + tid, (uint64_t)__float_as_uint(v) | ((uint64_t)flag << 32));
            else if (MODE == 1) st_agent(b + w * per + tid, __float_as_uint(v));
            else b[w * per + tid] = __float_as_uint(v);
        }
        if (MODE != 0) {
            if (MODE == 1) __builtin_amdgcn_s_waitcnt(0);
            else __threadfence();
            __syncthreads();
            if (tid == 0) {
                __hip_atomic_fetch_add(ctr + p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                while (ld_agent(ctr + p) < (unsigned)nwg * (epoch + 1)) {
                    if (ld_agent(abort_w)) { bad = 1; break; }
                    if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) { st_agent(abort_w, 1); bad = 1; break; }
                }
            }
            __syncthreads();
            if (MODE == 2) __threadfence();
        }
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(b, 0, 0x7fffffff, 0x00020000);
        v4u q[NPT];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NPT; ++j)
            q[j] = MODE == 2 ? *(const v4u*)(b + 4 * (tid + 256 * j)) : ld16_agent(rs, (tid + 256 * j) * 16);
        if (MODE == 0) {
#pragma unroll
            for (int j = 0; j < NPT; ++j) {
                if (q[j].y != flag || q[j].w != flag) {
                    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                    do {
                        q[j] = ld16_agent(rs, (tid + 256 * j) * 16);
                        if (ld_agent(abort_w)) { bad = 1; break; }
                        if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) { st_agent(abort_w, 1); bad = 1; break; }
                    } while (q[j].y != flag || q[j].w != flag);
                }
                s += __uint_as_float(q[j].x) + __uint_as_float(q[j].z);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NPT; ++j)
                s += (__uint_as_float(q[j].x) + __uint_as_float(q[j].y)) + (__uint_as_float(q[j].z) + __uint_as_float(q[j].w));
        }
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        if ((tid & 63) == 0) red[tid >> 6] = s;
        __syncthreads();
        carry = (red[0] + red[1] + red[2] + red[3]) * (1.0f / N);
        __syncthreads();
        if (bad) break;
    }
    if (tid == 0 && w == 0) out[0] = carry;
}

template <int NL>
__global__ __launch_bounds__(256) void stream_kernel(const float* __restrict__ x, const v4u* __restrict__ w,
                                                     float* __restrict__ y, size_t n16) {
    __shared__ float red[4];
    const int tid = threadIdx.x;
    v4f xa[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) xa[j] = *(const v4f*)(x + 4 * tid + 1024 * j);
    v4u q[NL];
    const size_t base = (size_t)blockIdx.x * 256 * NL;
#pragma unroll
    for (int j = 0; j < NL; ++j) q[j] = __builtin_nontemporal_load(w + std::min(base + (size_t)j * 256 + tid, n16 - 1));
    float s = (xa[0].x + xa[0].y) + (xa[1].x + xa[1].y);
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    unsigned acc = 0;
#pragma unroll
    for (int j = 0; j < NL; ++j) acc += q[j].x ^ q[j].y ^ q[j].z ^ q[j].w;
    float v = (float)(acc & 255) * 1e-9f + (red[0] + red[1] + red[2] + red[3]) * 1e-3f;
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((tid & 63) == 0) y[(blockIdx.x * 4 + (tid >> 6)) & 2047] = v;
}

__global__ __launch_bounds__(256) void rmw_kernel(v4f* __restrict__ p, size_t n4, float g) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        v4f v = p[i];
        v = v * g;
        p[i] = v;
    }
}

struct Timer {
    hipEvent_t a = nullptr, b = nullptr;
    Timer() {
        (void)hipEventCreate(&a);
        (void)hipEventCreate(&b);
    }
    ~Timer() {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
};

// best of `reps` replays of a captured graph, ms
template <typename F>
int time_graph(hipStream_t st, F launch, int reps, float* best_ms) {
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    if (hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed) != hipSuccess) return -6;
    launch();
    if (hipStreamEndCapture(st, &g) != hipSuccess) return -6;
    if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) return -6;
    (void)hipGraphDestroy(g);
    Timer t;
    float best = 1e30f;
    int rc = 0;
    for (int r = 0; r < reps + 1 && !rc; ++r) {
        if (hipEventRecord(t.a, st) != hipSuccess || hipGraphLaunch(ge, st) != hipSuccess ||
            hipEventRecord(t.b, st) != hipSuccess || hipEventSynchronize(t.b) != hipSuccess) {
            rc = -6;
            break;
        }
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, t.a, t.b);
        if (r > 0) best = std::min(best, ms);
    }
    (void)hipGraphExecDestroy(ge);
    *best_ms = best;
    return rc;
}

}  // namespace

extern "C" {

// Per-phase microseconds of a chain of `phases` dependent launches of `wgs`
// workgroups that each read N floats (N = 2048 or 6144).
int zg_probe_chain(int wgs, int N, int phases, float* us) {
    if ((N != 2048 && N != 6144) || wgs <= 0 || phases <= 0) return -1;
    float *a = nullptr, *b = nullptr;
    hipStream_t st = nullptr;
    if (hipMalloc(&a, N * 4) || hipMalloc(&b, N * 4) || hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) return -6;
    (void)hipMemset(a, 0, N * 4);
    (void)hipMemset(b, 0, N * 4);
    (void)hipDeviceSynchronize();
    float ms = 0.0f;
    int rc = time_graph(st, [&] {
        for (int p = 0; p < phases; ++p) {
            const float* in = (p & 1) ? b : a;
            float* out = (p & 1) ? a : b;
            if (N == 2048) hipLaunchKernelGGL(chain_kernel<2>, dim3(wgs), dim3(256), 0, st, in, out, N);
            else hipLaunchKernelGGL(chain_kernel<6>, dim3(wgs), dim3(256), 0, st, in, out, N);
        }
    }, 5, &ms);
    *us = ms * 1000.0f / phases;
    (void)hipStreamDestroy(st);
    (void)hipFree(a);
    (void)hipFree(b);
    return rc;
}

// Per-phase microseconds of the same dependency inside one cooperative
// kernel (mode 0 LL words, 1 counter + agent-scope data, 2 counter +
// fences).  Returns 1 when a bounded wait expired (the measurement is void).
int zg_probe_handoff(int mode, int wgs, int N, int phases, float* us) {
    if (mode < 0 || mode > 2 || (N != 2048 && N != 6144) || wgs <= 0 || N % wgs || phases <= 0 || phases > 4000)
        return -1;
    unsigned *buf = nullptr, *ctr = nullptr, *abort_w = nullptr;
    float* out = nullptr;
    hipStream_t st = nullptr;
    if (hipMalloc(&buf, (size_t)4 * N * 4) || hipMalloc(&ctr, (size_t)phases * 4) || hipMalloc(&abort_w, 4) ||
        hipMalloc(&out, 64) || hipStreamCreateWithFlags(&st, hipStreamNonBlocking))
        return -6;
    (void)hipMemset(buf, 0, (size_t)4 * N * 4);
    (void)hipMemset(ctr, 0, (size_t)phases * 4);
    (void)hipMemset(abort_w, 0, 4);
    (void)hipDeviceSynchronize();
    Timer t;
    float best = 1e30f;
    int rc = 0;
    for (unsigned ep = 0; ep < 6 && !rc; ++ep) {
        unsigned epoch = mode == 0 ? ep + 1 : ep;
        void* args[] = {&buf, &ctr, &abort_w, &phases, &N, &epoch, &out};
        const void* f;
        if (mode == 0) f = N == 2048 ? (const void*)handoff_kernel<0, 4> : (const void*)handoff_kernel<0, 12>;
        else if (mode == 1) f = N == 2048 ? (const void*)handoff_kernel<1, 2> : (const void*)handoff_kernel<1, 6>;
        else f = N == 2048 ? (const void*)handoff_kernel<2, 2> : (const void*)handoff_kernel<2, 6>;
        if (hipEventRecord(t.a, st) || hipLaunchCooperativeKernel(f, dim3(wgs), dim3(256), args, 0, st) ||
            hipEventRecord(t.b, st) || hipEventSynchronize(t.b)) {
            rc = -6;
            break;
        }
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, t.a, t.b);
        if (ep > 0) best = std::min(best, ms);
    }
    unsigned aborted = 0;
    (void)hipMemcpy(&aborted, abort_w, 4, hipMemcpyDeviceToHost);
    *us = best * 1000.0f / phases;
    (void)hipStreamDestroy(st);
    (void)hipFree(buf);
    (void)hipFree(ctr);
    (void)hipFree(abort_w);
    (void)hipFree(out);
    return rc ? rc : (aborted ? 1 : 0);
}

// Per-launch microseconds of GEMV-shaped launches streaming `bytes` each
// over `wgs`-ish workgroups (16-byte loads per thread: the fewest of 1, 2,
// 4, 8, 16 that cover the bytes), weights rotating over > 1 GB.
int zg_probe_stream(size_t bytes, int wgs, int launches, float* us) {
    if (bytes < 4096 || wgs <= 0 || launches <= 0) return -1;
    const size_t n16 = bytes / 16, total = (size_t)1200 << 20;
    const size_t per = (n16 + (size_t)wgs * 256 - 1) / ((size_t)wgs * 256);
    if (per > 16) return -1;
    const int NL = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
    const unsigned grid = (unsigned)((n16 + (size_t)256 * NL - 1) / ((size_t)256 * NL));
    void* pool = nullptr;
    float *x = nullptr, *y = nullptr;
    hipStream_t st = nullptr;
    if (hipMalloc(&pool, total) || hipMalloc(&x, 8192 * 4) || hipMalloc(&y, 8192 * 4) ||
        hipStreamCreateWithFlags(&st, hipStreamNonBlocking))
        return -6;
    (void)hipMemset(pool, 1, total);
    (void)hipMemset(x, 0, 8192 * 4);
    (void)hipDeviceSynchronize();
    const int copies = (int)std::min<size_t>(total / (n16 * 16), 400);
    float ms = 0.0f;
    int rc = time_graph(st, [&] {
        for (int l = 0; l < launches; ++l) {
            const v4u* w = (const v4u*)((char*)pool + (size_t)(l % copies) * n16 * 16);
#define ZG_PS(NN) hipLaunchKernelGGL(stream_kernel<NN>, dim3(grid), dim3(256), 0, st, x, w, y, n16)
            if (NL == 1) ZG_PS(1);
            else if (NL == 2) ZG_PS(2);
            else if (NL == 4) ZG_PS(4);
            else if (NL == 8) ZG_PS(8);
            else ZG_PS(16);
#undef ZG_PS
        }
    }, 5, &ms);
    *us = ms * 1000.0f / launches;
    (void)hipStreamDestroy(st);
    (void)hipFree(pool);
    (void)hipFree(x);
    (void)hipFree(y);
    return rc;
}

// GB/s (bytes read + written) of in-place read-modify-write over `bytes`,
// launches rotating over copies totalling > 1 GB.
int zg_probe_rmw(size_t bytes, int launches, float* gbs) {
    if (bytes < 65536 || launches <= 0) return -1;
    const size_t total = (size_t)1200 << 20, n4 = bytes / 16;
    const int copies = (int)std::max<size_t>(1, std::min<size_t>(total / bytes, 64));
    void* pool = nullptr;
    hipStream_t st = nullptr;
    if (hipMalloc(&pool, (size_t)copies * bytes) || hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) return -6;
    (void)hipMemset(pool, 0, (size_t)copies * bytes);
    (void)hipDeviceSynchronize();
    const unsigned grid = (unsigned)std::min<size_t>((n4 + 255) / 256, 8192);
    float ms = 0.0f;
    int rc = time_graph(st, [&] {
        for (int l = 0; l < launches; ++l)
            hipLaunchKernelGGL(rmw_kernel, dim3(grid), dim3(256), 0, st, (v4f*)((char*)pool + (size_t)(l % copies) * bytes),
                               n4, 0.999f);
    }, 5, &ms);
    *gbs = (float)(2.0 * bytes * launches / (ms * 1e-3) / 1e9);
    (void)hipStreamDestroy(st);
    (void)hipFree(pool);
    return rc;
}

}  // extern "C"
