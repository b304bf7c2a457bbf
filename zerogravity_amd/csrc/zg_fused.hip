// Dispatch of the fused decode GEMV (zg_fused_*.hip hold the kernels).
#include "zg_fused_kernels.hpp"

namespace zg {

template <int PRO>
hipError_t launch_pro(const FusedGemvArgs& a, int type, hipStream_t s);
extern template hipError_t launch_pro<PRO_RMS>(const FusedGemvArgs&, int, hipStream_t);
extern template hipError_t launch_pro<PRO_GATED>(const FusedGemvArgs&, int, hipStream_t);
extern template hipError_t launch_pro<PRO_SILU_MUL>(const FusedGemvArgs&, int, hipStream_t);
extern template hipError_t launch_pro<PRO_PLAIN>(const FusedGemvArgs&, int, hipStream_t);
hipError_t launch_gated_pre(const FusedGemvArgs& a, int type, hipStream_t s);

bool fused_glu_supported(int type, size_t K, size_t N) {
    // a row group must hold whole (gate, up) pairs: 64 lanes over <= 32
    // lanes per row (K <= 2048), rpw even
    return type == kQ4_K && K % 256 == 0 && K <= 2048 && N % 2 == 0 && N > 0;
}

bool batched_glu_supported(int type, size_t K, size_t N) {
    return type == kQ4_K && K % 256 == 0 && K <= 8192 && N % 64 == 0 && (N / 2) % 256 == 0;
}

bool fused_gemv_supported(int type, size_t K, size_t N, int pro) {
    if (N == 0 || K == 0 || N > (1u << 30)) return false;
    if (pro == PRO_GATED && (K % 128 || K / 128 > 256 || 256 % (K / 128))) return false;
    if (pro == PRO_GATED_PRE && (type != kQ4_K || K % 512)) return false;
    if (K > 8192) return false;  // prologue slabs
    if (type == kQ4_K || type == kQ6_K) return K % 256 == 0;
    if (type == kQ8_0 || type == kQ4_1) return K % 32 == 0;
    if (type == kF32) return K % 4 == 0;
    return false;
}

int gemv1_greedy_parts(const DeviceWeight& w, int pro) {
    FusedGemvArgs a;
    a.M = 1;
    a.K = (int)w.K;
    a.N = (int)w.N;
    a.pro = pro;
    a.epi = EPI_STORE;
    if (!fused_gemv_supported(w.type, w.K, w.N, pro) || !gemv1_fits(a, w.type)) return 0;
    return gemv1_grid((int)w.N, EPI_STORE);
}

bool gated_pre_supported(const DeviceWeight& w) {
    FusedGemvArgs a;
    a.M = 1;
    a.K = (int)w.K;
    a.N = (int)w.N;
    a.pro = PRO_GATED_PRE;
    a.epi = EPI_RESID;
    a.group = 128;
    return fused_gemv_supported(w.type, w.K, w.N, PRO_GATED_PRE) && gemv1_fits(a, w.type);
}

bool gemv1_embed_supported(const DeviceWeight& w, const DeviceWeight& emb) {
    return emb.type == kQ4_K && emb.K == w.K && emb.N > 0 && emb.N < (1u << 31) &&
           gemv1_greedy_parts(w, PRO_RMS) > 0;
}

hipError_t fused_gemv(const DeviceWeight& w, const FusedGemvArgs& args, hipStream_t s) {
    if (!fused_gemv_supported(w.type, w.K, w.N, args.pro) || args.M <= 0) return hipErrorInvalidValue;
    if ((args.pro == PRO_GATED || args.pro == PRO_GATED_PRE) && args.group != 128)
        return hipErrorInvalidValue;  // 32 lanes x 4 per group
    if (args.epi == EPI_GLU && !fused_glu_supported(w.type, w.K, w.N)) return hipErrorInvalidValue;
    FusedGemvArgs a = args;
    a.qs = w.qs;
    a.hdr = w.hdr;
    a.K = (int)w.K;
    a.N = (int)w.N;
    // formed GDN gates: only the one-row matrix-core GEMV's store epilogue does it
    if (a.gate_dt && (a.epi != EPI_STORE || !gemv1_fits(a, w.type) || !a.gate_a || a.gate_heads <= 0 ||
                      a.gate_row < 0 || a.gate_row + 2 * a.gate_heads > a.N))
        return hipErrorInvalidValue;
    switch (a.pro) {
    case PRO_RMS: return launch_pro<PRO_RMS>(a, w.type, s);
    case PRO_GATED: return launch_pro<PRO_GATED>(a, w.type, s);
    case PRO_SILU_MUL: return launch_pro<PRO_SILU_MUL>(a, w.type, s);
    case PRO_PLAIN: return launch_pro<PRO_PLAIN>(a, w.type, s);
    case PRO_GATED_PRE: return launch_gated_pre(a, w.type, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace zg
