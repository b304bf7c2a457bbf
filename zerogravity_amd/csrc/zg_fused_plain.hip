// Fused decode GEMV kernels with the PRO_PLAIN prologue.
#include "zg_fused_kernels.hpp"

namespace zg {
template hipError_t launch_pro<PRO_PLAIN>(const FusedGemvArgs& a, int type, hipStream_t s);
}  // namespace zg
