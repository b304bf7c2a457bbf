// Fused decode GEMV kernels with the PRO_SILU_MUL prologue.
#include "zg_fused_kernels.hpp"

namespace zg {
template hipError_t launch_pro<PRO_SILU_MUL>(const FusedGemvArgs& a, int type, hipStream_t s);
}  // namespace zg
