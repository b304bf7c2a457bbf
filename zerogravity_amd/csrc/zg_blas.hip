// Library GEMM for prompt-sized batched prefill: hipBLASLt on f16 operands
// with f32 accumulation.
//
// The batched prefill (zg_prefill_batched) multiplies an n-row activation by
// every stacked projection of a layer.  From a few hundred prompt rows that
// is a plain dense GEMM, which hipBLASLt's gfx950 kernels run at 40-70% of
// the f16 MFMA peak where the dequantizing MFMA kernels reach 20-28%.  The
// Q4_K weight is dequantized once (exact arithmetic, rounded once to f16,
// ensure_f16_weight) and kept in HBM for later prompts.
//
// Row-major D[M][N] = A[M][K] . W[N][K]^T is, in the library's column-major
// terms, D^T (N x M, ld ldd) = op_T(W as K x N, ld K) . A^T (K x M, ld K).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "zg_internal.hpp"

namespace zg {

namespace {

constexpr size_t kWorkspace = 64u << 20;
constexpr size_t kMaxPlans = 256;  // (prompt length, projection) shapes kept planned

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, ld = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

struct DeviceBlas {
    hipblasLtHandle_t handle = nullptr;
    void* workspace = nullptr;
    std::map<std::tuple<int, int, int, bool, size_t, bool>, Plan> plans;
};

std::mutex g_mu;
std::map<int, DeviceBlas> g_dev;

hipError_t lt(hipblasStatus_t st) { return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorUnknown; }

}  // namespace

hipError_t blas_gemm_f16(int device, int M, int N, int K, const void* A, const void* W, void* D, bool d_f32,
                         size_t ldd, float beta, hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0 || ldd < (size_t)N || (!d_f32 && beta != 0.0f)) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceBlas& db = g_dev[device];
    if (!db.handle) {
        if (lt(hipblasLtCreate(&db.handle)) != hipSuccess) {
            db.handle = nullptr;
            return hipErrorUnknown;
        }
        hipError_t e = hipMalloc(&db.workspace, kWorkspace);
        if (e != hipSuccess) {
            db.workspace = nullptr;
            return e;
        }
    }
    const auto key = std::make_tuple(M, N, K, d_f32, ldd, beta != 0.0f);
    auto it = db.plans.find(key);
    if (it == db.plans.end() && db.plans.size() >= kMaxPlans) {
        // prompt lengths vary without bound: start the cache over
        for (auto& kv : db.plans) {
            (void)hipblasLtMatrixLayoutDestroy(kv.second.ld);
            (void)hipblasLtMatrixLayoutDestroy(kv.second.la);
            (void)hipblasLtMatrixLayoutDestroy(kv.second.lw);
            (void)hipblasLtMatmulDescDestroy(kv.second.desc);
        }
        db.plans.clear();
    }
    if (it == db.plans.end()) {
        Plan p;
        hipError_t e = lt(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
        const hipblasOperation_t tw = HIPBLAS_OP_T, ta = HIPBLAS_OP_N;
        if (e == hipSuccess)
            e = lt(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &tw, sizeof(tw)));
        if (e == hipSuccess)
            e = lt(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &ta, sizeof(ta)));
        if (e == hipSuccess) e = lt(hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_16F, K, N, K));
        if (e == hipSuccess) e = lt(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, K, M, K));
        if (e == hipSuccess) e = lt(hipblasLtMatrixLayoutCreate(&p.ld, d_f32 ? HIP_R_32F : HIP_R_16F, N, M, ldd));
        hipblasLtMatmulPreference_t pref = nullptr;
        if (e == hipSuccess) e = lt(hipblasLtMatmulPreferenceCreate(&pref));
        size_t wsz = kWorkspace;
        if (e == hipSuccess)
            e = lt(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz,
                                                         sizeof(wsz)));
        hipblasLtMatmulHeuristicResult_t res{};
        int got = 0;
        if (e == hipSuccess)
            e = lt(hipblasLtMatmulAlgoGetHeuristic(db.handle, p.desc, p.lw, p.la, p.ld, p.ld, pref, 1, &res, &got));
        if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
        if (e == hipSuccess && got < 1) e = hipErrorNotSupported;
        if (e != hipSuccess) {
            if (p.ld) (void)hipblasLtMatrixLayoutDestroy(p.ld);
            if (p.la) (void)hipblasLtMatrixLayoutDestroy(p.la);
            if (p.lw) (void)hipblasLtMatrixLayoutDestroy(p.lw);
            if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
            return e;
        }
        p.algo = res.algo;
        it = db.plans.emplace(key, p).first;
    }
    const Plan& p = it->second;
    const float alpha = 1.0f;
    return lt(hipblasLtMatmul(db.handle, p.desc, &alpha, W, p.lw, A, p.la, &beta, D, p.ld, D, p.ld, &p.algo,
                              db.workspace, kWorkspace, s));
}

}  // namespace zg
