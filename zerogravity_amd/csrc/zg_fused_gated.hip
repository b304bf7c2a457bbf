// Fused decode GEMV kernels with the PRO_GATED prologue.
#include "zg_fused_kernels.hpp"

namespace zg {
template hipError_t launch_pro<PRO_GATED>(const FusedGemvArgs& a, int type, hipStream_t s);

// PRO_GATED_PRE: the one-row matrix-core GEMV only.
hipError_t launch_gated_pre(const FusedGemvArgs& a, int type, hipStream_t s) {
    if (!gemv1_fits(a, type) || a.epi == EPI_GLU) return hipErrorInvalidValue;
    return a.epi == EPI_RESID ? launch_gemv1_q4k<PRO_GATED_PRE, EPI_RESID>(a, s)
                              : launch_gemv1_q4k<PRO_GATED_PRE, EPI_STORE>(a, s);
}
}  // namespace zg
