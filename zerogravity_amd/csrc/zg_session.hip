// Boundary B: the resident Qwen3.5 hybrid model and its decode sessions
// (the reference's LoadedQwenModel + QwenDenseCpu, model-qwen35/src/
// lib.rs:386-507,1058-1254, with the per-token schedule of forward.rs:451-755).
//
// Weights that share an input are registered as one matrix with their rows
// stacked (GGUF rows are independent, so the outputs are unchanged):
//   GDN in-proj  = [attn_qkv | attn_gate | ssm_alpha | ssm_beta]
//   attn in-proj = [attn_q | attn_k | attn_v]
//   FFN          = [ffn_gate | ffn_up]
// A decode step is then 5 launches per GDN layer, 6 per attention layer and
// 3 around them, replayed as one HIP graph per (rows, token/logit/greedy
// buffers, commit): every kernel reads positions from device memory, so the
// captured step is valid at any position.
//
// Publication (QwenDenseCpu::next_logits / commit, lib.rs:1057-1070,
// 1211-1225; prefill_transaction, lib.rs:1114-1187): a step writes the KV
// row at the position (outside the published prefix), the conv ring slot
// p % 4 (whose old value, x[p-4], no tap reads any more) and the GDN state
// into the draft half of a double-buffered per-row state.  Its last kernel
// publishes it -- positions advance and each row's `cur` half flips -- only
// when the step's status word is clear, so a failed step leaves position,
// conv history, GDN state and KV prefix exactly as they were.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "zg_context.hpp"

using namespace zgc;

namespace {

// Matrices that share an input are stacked by rows into one launch; where
// their codecs differ the stack splits into runs of one codec, each written
// at its column offset of the shared output row.
struct Part {
    zg_weight* w = nullptr;
    uint64_t col = 0;
};
using Stack = std::vector<Part>;

bool all_type(const Stack& st, int type) {
    for (const Part& p : st)
        if (!p.w || p.w->dw.type != type) return false;
    return !st.empty();
}

struct LayerW {
    bool full = false;
    Stack in_proj, ffn_gu;
    zg_weight *out_proj = nullptr, *ffn_down = nullptr;
    float *attn_norm = nullptr, *post_norm = nullptr, *conv_w = nullptr, *ssm_norm = nullptr, *ssm_a = nullptr,
          *ssm_dt = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

}  // namespace

struct zg_model {
    zg_ctx* ctx = nullptr;
    uint64_t source = 0;
    uint64_t serial = 0;  // distinguishes models for snapshot ownership
    zg_geometry g{};
    std::vector<LayerW> layers;
    zg_weight* embd = nullptr;
    float* out_norm = nullptr;
    std::vector<void*> vecs;  // device copies of F32 parameter vectors
    size_t n_gdn = 0, n_attn = 0;
    bool all_q4k = true;  // every projection Q4_K: batched split-K residuals allowed
    std::vector<zg_weight*> refs;  // resident weights this model holds a reference on
};

struct zg_session {
    zg_model* m = nullptr;
    size_t max_batch = 0, max_ctx = 0;
    int kv_bf16 = 1;
    std::vector<int> pos;  // host copy of each row's next position
    // A failed launch leaves every row's device state unknown: all rows are
    // marked, and the session is usable again once each marked row has been
    // reset, restored or imported (or the whole session reset).
    bool poisoned = false;
    std::vector<uint8_t> row_bad;
    bool pos_dirty = true;  // device positions must be re-uploaded from pos
    bool use_graphs = true;
    // device buffers
    std::vector<void*> allocs;
    int *d_pos = nullptr, *d_ntok = nullptr, *d_status = nullptr, *pidx = nullptr;
    unsigned* tickets = nullptr;
    uint32_t *d_tokens = nullptr, *d_greedy = nullptr;
    float *x = nullptr, *y0 = nullptr, *core = nullptr, *ao = nullptr, *logits = nullptr, *scores = nullptr,
          *pmax = nullptr, *att_stats = nullptr;
    float* gated = nullptr;  // one-row steps: ssm_out's gated product, written by the GDN kernel
    // split-T attention partials (all-Q4_K models, 1..64 rows; null otherwise)
    float* att_part = nullptr;
    float* rope = nullptr;  // (cos, sin) of every position's 32 angles, with att_part
    void* xh = nullptr;  // f16 activations of the batched (B > 1) projections
    float* parts = nullptr;  // split-K partial tiles of residual projections (B > 1)
    void* xh3 = nullptr;     // the stream's RMS input tiles a residual projection leaves (B > 1)
    double* rss = nullptr;   // and their per-tile sums of squares [rows][hidden/16 or hidden/32]
    void* xh2 = nullptr;     // the SwiGLU product in f16 tiles, down projection input (B > 1)
    size_t y0w = 0;
    std::vector<float*> ring, rec;  // per GDN layer: conv ring [B][3W][4], state [B][2][H][128][128]
    std::vector<void*> kc, vc;      // per attention layer: [B][max_ctx][kv_heads*256]
    std::vector<int> layer_slot;    // layer -> index into ring/rec or kc/vc
    // per-row GDN state half holding the published state (the other half is
    // the draft a step writes); host mirror of d_cur
    int* d_cur = nullptr;
    std::vector<int> cur;
    size_t pending_rows = 0;  // rows of an uncommitted zg_session_propose
    // steps queued by zg_decode_step_device on a caller's stream: host
    // entry points wait on this event and re-read positions from the device
    hipEvent_t dev_ev = nullptr;
    bool async_steps = false;
    // captured steps, least recently used evicted beyond kGraphCache
    struct GraphEntry {
        hipGraphExec_t exec = nullptr;
        uint64_t used = 0;
    };
    std::map<std::tuple<size_t, const void*, const void*, const void*, int>, GraphEntry> graphs;
    uint64_t graph_clock = 0;
    // batched prefill buffers, sized for pf_cap prompt tokens
    size_t pf_cap = 0;
    std::vector<void*> pf;
};

namespace {

const zg_tensor_desc* find_tensor(const zg_tensor_desc* t, size_t n, const std::string& name) {
    for (size_t i = 0; i < n; ++i)
        if (t[i].name && name == t[i].name) return &t[i];
    return nullptr;
}

std::string lname(unsigned i, const char* suffix) { return "blk." + std::to_string(i) + "." + suffix; }

// The model holds one reference on each resident weight it uses: the
// weight is freed when its last model is destroyed, unless an API caller
// registered it (then zg_source_release frees it).
void take_ref(zg_model* m, zg_weight* w) {
    if (std::find(m->refs.begin(), m->refs.end(), w) != m->refs.end()) return;
    w->model_refs += 1;
    m->refs.push_back(w);
}

// Rows of several [K, N_i] GGUF matrices stacked into registered weights:
// one per run of consecutive matrices sharing a codec, at its column offset.
int load_stack(zg_model* m, const zg_tensor_desc* ts, size_t n, const std::vector<std::string>& names, uint64_t K,
               const std::vector<uint64_t>& Ns, const std::string& key, int pro, Stack* out) {
    zg_ctx* ctx = m->ctx;
    std::vector<const zg_tensor_desc*> parts;
    for (size_t i = 0; i < names.size(); ++i) {
        const zg_tensor_desc* t = find_tensor(ts, n, names[i]);
        if (!t) return fail(ctx, ZG_E_MALFORMED, "missing tensor " + names[i]);
        if (t->shape0 != K || t->shape1 != Ns[i])
            return fail(ctx, ZG_E_MALFORMED, "tensor " + names[i] + " geometry differs from the model configuration");
        int rc = check_matrix(ctx, t->ggml_type, K, Ns[i], t->data, t->nbytes);
        if (rc == ZG_UNSUPPORTED) return fail(ctx, ZG_E_UNSUPPORTED, "tensor " + names[i] + ": " + last_message(ctx));
        if (rc) return rc;
        if (!zg::fused_gemv_supported(t->ggml_type, K, Ns[i], pro))
            return fail(ctx, ZG_E_UNSUPPORTED, "resident decode has no projection kernel for " + names[i]);
        parts.push_back(t);
    }
    out->clear();
    uint64_t col = 0;
    for (size_t i = 0, run = 0; i < parts.size(); ++run) {
        size_t j = i;
        uint64_t rows = 0;
        size_t bytes = 0;
        while (j < parts.size() && parts[j]->ggml_type == parts[i]->ggml_type) {
            rows += Ns[j];
            bytes += parts[j]->nbytes;
            ++j;
        }
        const int type = parts[i]->ggml_type;
        if (type != ZG_Q4_K) m->all_q4k = false;
        const std::string k = run == 0 ? key : key + "." + std::to_string(run);
        Part p;
        p.col = col;
        int rc;
        if (j == i + 1) {
            rc = lookup_or_register(ctx, m->source, k.c_str(), type, K, rows, parts[i]->data, parts[i]->nbytes, &p.w);
        } else {
            std::vector<uint8_t> buf(bytes);
            size_t at = 0;
            for (size_t q = i; q < j; ++q) {
                memcpy(buf.data() + at, parts[q]->data, parts[q]->nbytes);
                at += parts[q]->nbytes;
            }
            rc = lookup_or_register(ctx, m->source, k.c_str(), type, K, rows, buf.data(), bytes, &p.w);
        }
        if (rc) return rc;
        take_ref(m, p.w);
        out->push_back(p);
        col += rows;
        i = j;
    }
    return ZG_COMPLETED;
}

int load_single(zg_model* m, const zg_tensor_desc* ts, size_t n, const std::string& name, uint64_t K, uint64_t N,
                int pro, zg_weight** out) {
    Stack st;
    int rc = load_stack(m, ts, n, {name}, K, {N}, name, pro, &st);
    if (!rc) *out = st[0].w;
    return rc;
}

int load_vector(zg_model* m, const zg_tensor_desc* ts, size_t n, const std::string& name, uint64_t len, float** out) {
    zg_ctx* ctx = m->ctx;
    const zg_tensor_desc* t = find_tensor(ts, n, name);
    if (!t) return fail(ctx, ZG_E_MALFORMED, "missing tensor " + name);
    if (t->ggml_type != ZG_F32 || t->shape0 * t->shape1 != len || t->nbytes != len * 4 || !t->data)
        return fail(ctx, ZG_E_MALFORMED, "parameter " + name + " must be F32 of " + std::to_string(len) + " values");
    if (!all_finite((const float*)t->data, len)) return fail(ctx, ZG_E_MALFORMED, "nonfinite parameter " + name);
    void* d = nullptr;
    ZG_HIP(hipMalloc(&d, len * 4));
    m->vecs.push_back(d);
    ZG_HIP(hipMemcpy(d, t->data, len * 4, hipMemcpyHostToDevice));
    *out = (float*)d;
    return ZG_COMPLETED;
}

// Boundary B admission: the numerical profile and tensor table the plan
// hands over must be the schedule step() runs (the GGUF source profile,
// LoadedQwenModel::require_execution_profile, model-qwen35/src/source/
// binding.rs:363-371; a provider prepares whatever plan it is given,
// core/src/provider.rs:38-42, so the refusal is the backend's).  Host only:
// no device, no context.  Every tensor the schedule reads must be present
// with the role's shape, a codec the role's kernels take and its exact
// packed length; values (finite scales, finite parameters) are checked when
// zg_model_load uploads them.
int admit_model(int profile, const zg_geometry* g, const zg_tensor_desc* ts, size_t n, std::string* why) {
    auto no = [&](int code, const std::string& m) {
        *why = m;
        return code;
    };
    if (profile != ZG_PROFILE_GGUF_SOURCE_V1)
        return no(ZG_E_UNSUPPORTED, "numerical profile " + std::to_string(profile) +
                                        " is not the GGUF source profile this backend runs");
    if (!g || !ts) return no(ZG_E_MALFORMED, "missing geometry or tensor table");
    if (g->layers == 0 || g->layers > 4096 || g->full_attention_interval == 0 || g->gdn_dim != 128 ||
        g->head_dim != 256 || g->q_heads == 0 || g->kv_heads == 0 || g->q_heads % g->kv_heads ||
        g->q_heads / g->kv_heads > 4 || g->gdn_heads == 0 || g->gdn_heads > 64 || !(g->eps > 0.0f) ||
        g->max_context == 0 || g->hidden % 256 || g->ffn % 256 || g->vocab == 0)
        return no(ZG_E_UNSUPPORTED, "model geometry outside the resident decode path (gdn_dim 128, head_dim 256)");
    auto matrix = [&](const std::string& name, uint64_t K, uint64_t N, int pro) {
        const zg_tensor_desc* t = find_tensor(ts, n, name);
        if (!t) return no(ZG_E_MALFORMED, "missing tensor " + name);
        if (t->shape0 != K || t->shape1 != N)
            return no(ZG_E_MALFORMED, "tensor " + name + " geometry differs from the model configuration");
        if (!t->data) return no(ZG_E_MALFORMED, "tensor " + name + " has no data");
        if (!supported_type(t->ggml_type))
            return no(ZG_E_UNSUPPORTED, "tensor " + name + ": ggml type " + std::to_string(t->ggml_type) +
                                            " not offered by this backend");
        if (K % block_elems(t->ggml_type) || zg::gguf_row_bytes(t->ggml_type, K) * N != t->nbytes)
            return no(ZG_E_MALFORMED, "tensor " + name + ": packed byte length mismatch");
        if (!zg::fused_gemv_supported(t->ggml_type, K, N, pro))
            return no(ZG_E_UNSUPPORTED, "resident decode has no projection kernel for " + name);
        return (int)ZG_COMPLETED;
    };
    auto vector = [&](const std::string& name, uint64_t len) {
        const zg_tensor_desc* t = find_tensor(ts, n, name);
        if (!t) return no(ZG_E_MALFORMED, "missing tensor " + name);
        if (t->ggml_type != ZG_F32 || t->shape0 * t->shape1 != len || t->nbytes != len * 4 || !t->data)
            return no(ZG_E_MALFORMED, "parameter " + name + " must be F32 of " + std::to_string(len) + " values");
        return (int)ZG_COMPLETED;
    };
    const uint64_t H = g->hidden, F = g->ffn, V = g->vocab, W = (uint64_t)g->gdn_heads * g->gdn_dim;
    const uint64_t QD = (uint64_t)g->q_heads * g->head_dim, KD = (uint64_t)g->kv_heads * g->head_dim;
    int rc = matrix("token_embd.weight", H, V, zg::PRO_RMS);
    if (!rc) rc = vector("output_norm.weight", H);
    for (unsigned i = 0; i < g->layers && !rc; ++i) {
        const bool full = ((i + 1) % g->full_attention_interval) == 0;  // config.rs:146-167
        rc = vector(lname(i, "attn_norm.weight"), H);
        if (!rc) rc = vector(lname(i, "post_attention_norm.weight"), H);
        if (!rc) rc = matrix(lname(i, "ffn_gate.weight"), H, F, zg::PRO_RMS);
        if (!rc) rc = matrix(lname(i, "ffn_up.weight"), H, F, zg::PRO_RMS);
        if (!rc) rc = matrix(lname(i, "ffn_down.weight"), F, H, zg::PRO_SILU_MUL);
        if (full) {
            if (!rc) rc = matrix(lname(i, "attn_q.weight"), H, 2 * QD, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "attn_k.weight"), H, KD, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "attn_v.weight"), H, KD, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "attn_output.weight"), QD, H, zg::PRO_PLAIN);
            if (!rc) rc = vector(lname(i, "attn_q_norm.weight"), g->head_dim);
            if (!rc) rc = vector(lname(i, "attn_k_norm.weight"), g->head_dim);
        } else {
            if (!rc) rc = matrix(lname(i, "attn_qkv.weight"), H, 3 * W, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "attn_gate.weight"), H, W, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "ssm_alpha.weight"), H, g->gdn_heads, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "ssm_beta.weight"), H, g->gdn_heads, zg::PRO_RMS);
            if (!rc) rc = matrix(lname(i, "ssm_out.weight"), W, H, zg::PRO_GATED);
            if (!rc) rc = vector(lname(i, "ssm_conv1d.weight"), 4 * 3 * W);
            if (!rc) rc = vector(lname(i, "ssm_norm.weight"), g->gdn_dim);
            if (!rc) rc = vector(lname(i, "ssm_a"), g->gdn_heads);
            if (!rc) rc = vector(lname(i, "ssm_dt.bias"), g->gdn_heads);
        }
    }
    return rc;
}

int dalloc(zg_session* s, void** p, size_t bytes) {
    zg_ctx* ctx = s->m->ctx;
    ZG_HIP(hipMalloc(p, bytes < 256 ? 256 : bytes));
    // on the context's stream, finished before return: the stream is
    // non-blocking, so a null-stream hipMemset could still be clearing the
    // buffer when kernels on it start
    ZG_HIP(hipMemsetAsync(*p, 0, bytes < 256 ? 256 : bytes, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    s->allocs.push_back(*p);
    return ZG_COMPLETED;
}

size_t conv_floats(const zg_geometry& g) { return (size_t)g.gdn_heads * g.gdn_dim * 3 * 3; }  // exported history
size_t ring_floats(const zg_geometry& g) { return (size_t)g.gdn_heads * g.gdn_dim * 3 * 4; }  // device ring
size_t rec_floats(const zg_geometry& g) { return (size_t)g.gdn_heads * g.gdn_dim * g.gdn_dim; }
size_t kvw(const zg_geometry& g) { return (size_t)g.kv_heads * g.head_dim; }
// Row `row`'s GDN state half `half` of GDN layer slot `slot`.
float* rec_half(zg_session* s, size_t slot, size_t row, int half) {
    return s->rec[slot] + (row * 2 + (size_t)half) * rec_floats(s->m->g);
}
constexpr size_t kGraphCache = 16;  // captured step graphs kept per session

// One decode step for rows [0, B): tokens in `tokens` (device), positions in
// d_pos / d_ntok.  Logits to `logits` (may be the session buffer), greedy
// ids to `greedy` (nullable).  With `commit` the last launch publishes the
// step (positions advance, GDN halves flip) when the status word is clear;
// without it the step stays a draft for zg_session_commit.  Asynchronous on
// st, no host synchronisation, capturable.
int step(zg_session* s, size_t B, const uint32_t* tokens, float* logits, uint32_t* greedy, bool commit,
         hipStream_t st) {
    zg_model* m = s->m;
    zg_ctx* ctx = m->ctx;
    const zg_geometry& g = m->g;
    const size_t H = g.hidden, F = g.ffn, V = g.vocab, W = (size_t)g.gdn_heads * g.gdn_dim;
    const size_t QD = (size_t)g.q_heads * g.head_dim;
    int pending = 0;  // splits of a residual GEMM whose partial tiles the next RMS activation adds
    // batched rows: a residual projection (K <= 2048, no splits) left the
    // next RMS projection's f16 tiles (xh3) and per-tile sums of squares
    // (rss) of the current stream
    bool rms_ready = false;
    int rss_n = 0;  // sums of squares per row in rss
    // one row: the first projection dequantises the token's embedding in its
    // prologue (and stores it as the residual stream) instead of an embedding launch
    const zg::DeviceWeight* first_in = m->layers.empty() || m->layers[0].in_proj.size() != 1
                                           ? nullptr : &m->layers[0].in_proj[0].w->dw;
    const uint32_t* embed_tok =
        B == 1 && first_in && zg::gemv1_embed_supported(*first_in, m->embd->dw) ? tokens : nullptr;
    // one row: the GDN input projection forms the layer's gates in its
    // epilogue (FusedGemvArgs::gate_dt) for the next projection launched
    struct {
        const float *dt = nullptr, *a = nullptr;
        int row = 0, heads = 0;
    } gate_req;
    auto gemv = [&](zg_weight* w, int pro, const float* x, size_t ldx, const float* x2, size_t ldx2,
                    const float* gamma, int epi, float* y, size_t ldy, void* xh_out = nullptr,
                    const void* xh_in = nullptr, bool greedy_parts = false, const float* gamma_next = nullptr) {
        zg::FusedGemvArgs f;
        f.M = (int)B;
        if (gate_req.dt) {
            f.gate_dt = gate_req.dt;
            f.gate_a = gate_req.a;
            f.gate_row = gate_req.row;
            f.gate_heads = gate_req.heads;
            gate_req.dt = nullptr;
        }
        if (greedy_parts) {
            f.amax = s->pmax;
            f.aidx = s->pidx;
        }
        if (embed_tok && pro == zg::PRO_RMS && x == s->x) {
            f.tok = embed_tok;
            f.emb_qs = m->embd->dw.qs;
            f.emb_hdr = m->embd->dw.hdr;
            f.emb_rows = (int)m->embd->dw.N;
            f.x_out = s->x;
            embed_tok = nullptr;
        }
        f.pro = pro;
        f.epi = epi;
        f.x = x;
        f.ldx = ldx;
        f.x2 = x2;
        f.ldx2 = ldx2;
        f.gamma = gamma;
        f.eps = g.eps;
        f.group = (int)g.gdn_dim;
        f.y = y;
        f.ldy = ldy;
        f.status = s->d_status;
        f.xh_out = xh_out;
        f.xh_in = xh_in;
        // one row: one launch with the prologue in-kernel (the int8 matrix-core
        // GEMV); more rows of Q4_K weights: the activation in f16 and the MFMA
        // GEMM (weights read once); other codecs: the fused 1-4 row kernels
        if (pending && !(B > 1 && w->dw.type == zg::kQ4_K && pro == zg::PRO_RMS && x == s->x))
            return hipErrorInvalidValue;  // a pending split-K residual must be consumed by the next RMS projection
        if (B > 1 && w->dw.type == zg::kQ4_K) {
            if (pending && pro == zg::PRO_RMS && x == s->x) {
                f.rparts = s->parts;
                f.rsplits = pending;
                f.xw = s->x;
                pending = 0;
            } else if (rms_ready && pro == zg::PRO_RMS && x == s->x) {
                f.xh_in = s->xh3;  // the stream's tiles and sums of squares
                f.rms_ss_in = s->rss;
                f.rms_ss_n = rss_n;
            }
            if (epi == zg::EPI_RESID && y == s->x && m->all_q4k) {
                // the next RMS projection's input in the epilogue, without
                // K splits: on the 16-row kernel (which never splits K) when
                // the stream's width takes its layout, else for a short K
                // (32 activation rows read quickly); a long K otherwise
                // splits (the next RMS activation launch adds the parts)
                const bool k16 = zg::batched16_supported(B, w->dw.K, w->dw.N, zg::EPI_RESID);
                const bool h16 = zg::xh16_layout(B, H);
                rms_ready = gamma_next && H % 256 == 0 && H <= 2048 && ldy == H &&
                            (h16 ? k16 : !k16 && w->dw.K <= 2048);
                rss_n = (int)(k16 ? H / 16 : H / 32);
                const int sp = rms_ready || k16 ? 1 : zg::batched_splits(w->dw.N, w->dw.K);
                if (rms_ready) {
                    f.rms_tiles_out = (_Float16*)s->xh3;
                    f.rms_gamma = gamma_next;
                    f.rms_ss_out = s->rss;
                } else if (sp > 1) {
                    f.parts = s->parts;
                    f.splits = sp;
                    pending = sp;
                }
            } else if (epi == zg::EPI_RESID && y == s->x) {
                rms_ready = false;
            }
            return zg::batched_gemv(w->dw, f, s->xh, st);
        }
        if (epi == zg::EPI_RESID && y == s->x) rms_ready = false;
        // Q8_0 and Q6_K beyond four rows: the activation coded once into the
        // scratch (no tiles are pending there: only Q4_K projections consume
        // them), then one weight stream per 16 rows
        if (B > 4 && !xh_in && !xh_out &&
            ((w->dw.type == zg::kQ8_0 && zg::q8_rows_supported(w->dw.K, w->dw.N, pro)) ||
             (w->dw.type == zg::kQ6_K && zg::q6k_rows_supported(w->dw.K, w->dw.N, pro))))
            return zg::batched_gemv(w->dw, f, s->xh, st);
        return zg::fused_gemv(w->dw, f, st);
    };
    if (!embed_tok) ZG_HIP(zg::embed(m->embd->dw, tokens, s->x, B, s->d_status, st));
    for (size_t i = 0; i < m->layers.size(); ++i) {
        LayerW& L = m->layers[i];
        const int slot = s->layer_slot[i];
        // one row through the matrix-core GEMV: the GDN gates come formed
        const bool gates = !L.full && B == 1 && L.in_proj.size() == 1 && L.in_proj[0].col == 0 &&
                           zg::gemv1_greedy_parts(L.in_proj[0].w->dw, zg::PRO_RMS) > 0;
        for (const Part& p : L.in_proj) {
            if (gates) {
                gate_req.dt = L.ssm_dt;
                gate_req.a = L.ssm_a;
                gate_req.row = (int)(4 * W);
                gate_req.heads = (int)g.gdn_heads;
            }
            ZG_HIP(gemv(p.w, zg::PRO_RMS, s->x, H, nullptr, 0, L.attn_norm, zg::EPI_STORE, s->y0 + p.col, s->y0w));
        }
        if (!L.full) {
            zg::GdnDecodeArgs d;
            d.proj = s->y0;
            d.proj_stride = s->y0w;
            d.conv_w = L.conv_w;
            d.ring = s->ring[slot];
            d.pos = s->d_pos;
            d.dt = L.ssm_dt;
            d.ssm_a = L.ssm_a;
            d.eps = g.eps;
            d.scale = 1.0f / sqrtf((float)g.gdn_dim);
            d.state = s->rec[slot];
            d.status = s->d_status;
            d.cur = s->d_cur;
            d.state_row = 2 * rec_floats(g);
            d.state_half = rec_floats(g);
            d.core = s->core;
            d.H = (int)g.gdn_heads;
            d.gates_formed = gates ? 1 : 0;
            // batched rows: the kernel also writes ssm_out's gated-norm f16
            // activation tiles (one workgroup per head), so the batched GEMM
            // runs without an activation launch
            const bool tiles = B > 1 && L.out_proj->dw.type == zg::kQ4_K;
            if (tiles) {
                d.xh = s->xh;
                d.norm = L.ssm_norm;
            }
            // one row: the kernel also forms (core * ssm_norm) * silu(z), and
            // ssm_out's prologue only applies the per-head 1/rms
            const bool pre = B == 1 && zg::gated_pre_supported(L.out_proj->dw);
            if (pre) {
                d.gated = s->gated;
                d.norm = L.ssm_norm;
            }
            ZG_HIP(zg::gdn_decode(d, B, st));
            // gated RMSNorm (ssm_norm) * silu(z) -> ssm_out -> residual
            if (pre)
                ZG_HIP(gemv(L.out_proj, zg::PRO_GATED_PRE, s->core, W, s->gated, W, nullptr, zg::EPI_RESID, s->x, H,
                            nullptr, nullptr, false, L.post_norm));
            else
                ZG_HIP(gemv(L.out_proj, zg::PRO_GATED, s->core, W, s->y0 + 3 * W, s->y0w, L.ssm_norm, zg::EPI_RESID,
                            s->x, H, nullptr, tiles ? s->xh : nullptr, false, L.post_norm));
        } else {
            zg::AttnDecodeArgs a;
            a.proj = s->y0;
            a.proj_stride = s->y0w;
            a.qnorm = L.q_norm;
            a.knorm = L.k_norm;
            a.eps = g.eps;
            a.theta_scale = powf(10000000.0f, -2.0f / 64.0f);
            a.scale = 1.0f / sqrtf((float)g.head_dim);
            a.pos = s->d_pos;
            a.kcache = s->kc[slot];
            a.vcache = s->vc[slot];
            a.cache_row_stride = s->max_ctx * kvw(g);
            a.kv_bf16 = s->kv_bf16;
            a.scores = s->scores;
            a.score_stride = (size_t)g.q_heads * s->max_ctx;
            a.head_stride = s->max_ctx;
            a.out = s->ao;
            a.out_stride = QD;
            a.status = s->d_status;
            a.stats = s->att_stats;
            a.nq = (int)g.q_heads;
            a.nkv = (int)g.kv_heads;
            a.max_ctx = (int)s->max_ctx;
            // batched rows: the value kernel also writes o_proj's f16 tiles
            const bool tiles = B > 1 && L.out_proj->dw.type == zg::kQ4_K;
            if (tiles) a.xh = s->xh;
            if (s->att_part && zg::attn_split_supported(B, a.nq, a.nkv, s->max_ctx)) {
                a.rope = s->rope;
                ZG_HIP(zg::attn_decode_split(a, B, s->att_part, st));
            }
            else
                ZG_HIP(zg::attn_decode(a, B, st));
            ZG_HIP(gemv(L.out_proj, zg::PRO_PLAIN, s->ao, QD, nullptr, 0, nullptr, zg::EPI_RESID, s->x, H, nullptr,
                        tiles ? s->xh : nullptr, false, L.post_norm));
        }
        // the RMSNorm weight of the next projection that reads the stream
        const float* next_norm = i + 1 < m->layers.size() ? m->layers[i + 1].attn_norm
                                                          : (logits || greedy ? m->out_norm : nullptr);
        const zg::DeviceWeight& gu = L.ffn_gu[0].w->dw;
        const bool glu = L.ffn_gu.size() == 1 && L.ffn_down->dw.type == zg::kQ4_K &&
                         (B > 1 ? zg::batched_glu_supported(gu.type, gu.K, gu.N) : zg::fused_glu_supported(gu.type, gu.K, gu.N));
        if (glu) {
            // SwiGLU in the gate/up epilogue: the down projection takes the
            // product as a plain activation (f16 tiles when batched)
            ZG_HIP(gemv(L.ffn_gu[0].w, zg::PRO_RMS, s->x, H, nullptr, 0, L.post_norm, zg::EPI_GLU, s->y0, s->y0w,
                        B > 1 ? s->xh2 : nullptr));
            ZG_HIP(gemv(L.ffn_down, zg::PRO_PLAIN, s->y0, s->y0w, nullptr, 0, nullptr, zg::EPI_RESID, s->x, H, nullptr,
                        B > 1 ? s->xh2 : nullptr, false, next_norm));
        } else {
            for (const Part& p : L.ffn_gu)
                ZG_HIP(gemv(p.w, zg::PRO_RMS, s->x, H, nullptr, 0, L.post_norm, zg::EPI_STORE, s->y0 + p.col, s->y0w));
            ZG_HIP(gemv(L.ffn_down, zg::PRO_SILU_MUL, s->y0, s->y0w, s->y0 + F, s->y0w, nullptr, zg::EPI_RESID, s->x,
                        H));
        }
    }
    zg::StepCommit sc;
    sc.pos = s->d_pos;
    sc.ntok = s->d_ntok;
    sc.cur = s->d_cur;
    if (logits || greedy) {
        float* lg = logits ? logits : s->logits;
        // one row: the LM head's workgroups leave the greedy partials
        const int parts = B == 1 && greedy ? zg::gemv1_greedy_parts(m->embd->dw, zg::PRO_RMS) : 0;
        ZG_HIP(gemv(m->embd, zg::PRO_RMS, s->x, H, nullptr, 0, m->out_norm, zg::EPI_STORE, lg, V, nullptr, nullptr,
                    parts > 0));
        if (greedy) {
            if (parts > 0)
                ZG_HIP(zg::argmax_final(s->pmax, s->pidx, parts, greedy, s->d_status, commit ? &sc : nullptr, st));
            else
                ZG_HIP(zg::argmax_step(lg, V, V, B, greedy, s->d_status, s->pmax, s->pidx, commit ? &sc : nullptr,
                                       st));
            return ZG_COMPLETED;
        }
    }
    if (commit) ZG_HIP(zg::commit_step(sc, s->d_status, B, st));
    return ZG_COMPLETED;
}

// The step through a cached HIP graph (one per rows/buffer set/commit),
// captured on first use; the least recently used graph is dropped beyond
// kGraphCache.  ZG_GRAPHS=0 in the environment launches the kernels
// directly.
int run_step(zg_session* s, size_t B, const uint32_t* tokens, float* logits, uint32_t* greedy, bool commit,
             hipStream_t st) {
    zg_ctx* ctx = s->m->ctx;
    if (!s->use_graphs) return step(s, B, tokens, logits, greedy, commit, st);
    const auto key = std::make_tuple(B, (const void*)tokens, (const void*)logits, (const void*)greedy, (int)commit);
    auto it = s->graphs.find(key);
    if (it == s->graphs.end()) {
        if (s->graphs.size() >= kGraphCache) {
            auto old = s->graphs.begin();
            for (auto g = s->graphs.begin(); g != s->graphs.end(); ++g)
                if (g->second.used < old->second.used) old = g;
            // an evicted graph may still be running on a stream
            ZG_HIP(hipDeviceSynchronize());
            (void)hipGraphExecDestroy(old->second.exec);
            s->graphs.erase(old);
        }
        hipGraph_t graph = nullptr;
        ZG_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
        const int rc = step(s, B, tokens, logits, greedy, commit, st);
        const hipError_t e = hipStreamEndCapture(st, &graph);
        if (rc) {
            if (e == hipSuccess && graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        ZG_HIP(e);
        hipGraphExec_t exec = nullptr;
        const hipError_t e2 = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        ZG_HIP(e2);
        it = s->graphs.emplace(key, zg_session::GraphEntry{exec, 0}).first;
    }
    it->second.used = ++s->graph_clock;
    ZG_HIP(hipGraphLaunch(it->second.exec, st));
    return ZG_COMPLETED;
}

// Poison: every row's device state is unknown after a failed launch.
void poison(zg_session* s) {
    std::fill(s->row_bad.begin(), s->row_bad.end(), 1);
    s->poisoned = true;
}

// A row whose state was just rewritten from a known source is trusted again;
// the session is usable when no row is left unknown.
void clear_poison(zg_session* s, size_t row) {
    s->row_bad[row] = 0;
    s->poisoned = std::find(s->row_bad.begin(), s->row_bad.end(), 1) != s->row_bad.end();
}

// Host mirrors of positions and GDN halves re-read from the device (after
// asynchronous steps, whose commits the host cannot see, or a failed step).
int pull_positions(zg_session* s, hipStream_t st) {
    zg_ctx* ctx = s->m->ctx;
    const size_t B = s->max_batch;
    ZG_HIP(hipMemcpyAsync(s->pos.data(), s->d_pos, B * sizeof(int), hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(s->cur.data(), s->d_cur, B * sizeof(int), hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

// Before any host-synchronous entry: steps queued on a caller's stream have
// finished and the host mirrors are the device's.
int settle(zg_session* s) {
    if (!s->async_steps) return ZG_COMPLETED;
    zg_ctx* ctx = s->m->ctx;
    ZG_HIP(hipEventSynchronize(s->dev_ev));
    s->async_steps = false;
    return pull_positions(s, ctx->stream);
}

// The status word of the steps since the last check.  A failed step did
// not publish (its commit is gated on this word), so the session keeps the
// state before it: the word is cleared, the host mirrors are re-read from
// the device unless the host copy is the newer one (pos_dirty: a reset,
// copy, restore, import or batched prefill since the last upload, which
// the device positions have not seen), and the error is returned.
int read_status(zg_session* s, hipStream_t st) {
    zg_ctx* ctx = s->m->ctx;
    int status = 0;
    ZG_HIP(hipMemcpyAsync(&status, s->d_status, sizeof(int), hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (status) {
        ZG_HIP(hipMemsetAsync(s->d_status, 0, sizeof(int), st));
        if (!s->pos_dirty) {
            int rc = pull_positions(s, st);
            if (rc) return rc;
        }
        s->pending_rows = 0;
        if (status & 2) return fail(ctx, ZG_E_MALFORMED, "decode step contains an out-of-vocabulary token id");
        if (status & 1) return fail(ctx, ZG_E_STATE, "nonfinite layer computation");
        if (status & 8) return fail(ctx, ZG_E_STATE, "degenerate attention softmax");
        if (status & 16)
            return fail(ctx, ZG_E_LIMIT,
                        "an activation exceeds the f16 range of the batched projections (zg_prefill and steps of at "
                        "most 4 rows compute in f32)");
        return fail(ctx, ZG_E_STATE, "decoder produced nonfinite logits");
    }
    return ZG_COMPLETED;
}

// Device positions follow the host copy: steps advance both (the last
// launch of a step, so device-driven decode loops never wait on the host);
// reset, import and random fill mark them dirty and the next step uploads
// them once.
int sync_positions(zg_session* s, hipStream_t st) {
    if (!s->pos_dirty) return ZG_COMPLETED;
    zg_ctx* ctx = s->m->ctx;
    const size_t B = s->max_batch;
    std::vector<int> p(B), t(B);
    for (size_t b = 0; b < B; ++b) {
        p[b] = s->pos[b];
        t[b] = s->pos[b] + 1;
    }
    ZG_HIP(hipMemcpyAsync(s->d_pos, p.data(), B * sizeof(int), hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(s->d_ntok, t.data(), B * sizeof(int), hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(s->d_cur, s->cur.data(), B * sizeof(int), hipMemcpyHostToDevice, st));
    // pageable source: make the copy complete before the vectors go away
    ZG_HIP(hipStreamSynchronize(st));
    s->pos_dirty = false;
    return ZG_COMPLETED;
}

int check_rows(zg_session* s, size_t rows) {
    zg_ctx* ctx = s->m->ctx;
    if (s->poisoned) return fail(ctx, ZG_E_STATE, "session poisoned by a failed launch: reset or import state");
    if (rows == 0 || rows > s->max_batch) return fail(ctx, ZG_E_LIMIT, "row count exceeds the session batch");
    for (size_t b = 0; b < rows; ++b)
        if ((size_t)s->pos[b] >= s->max_ctx) return fail(ctx, ZG_E_LIMIT, "model context capacity exhausted");
    return ZG_COMPLETED;
}

// Slot of the ring holding x[pos - 3 + k] (k = 0, 1, 2) at a row's position.
inline size_t ring_slot(int pos, int k) { return (size_t)((pos + 1 + k) & 3); }

// A device copy of one row's published state: per GDN layer the conv ring
// and the published GDN half, and with_kv the K and V rows [0, pos) of each
// attention layer.  Restored into half 0 of a row.
struct RowImage {
    void* dev = nullptr;
    size_t bytes = 0;
    int pos = 0;
    bool with_kv = false;
};

size_t kv_row_bytes(const zg_session* s) { return s->max_ctx * kvw(s->m->g) * (s->kv_bf16 ? 2 : 4); }

int save_row(zg_session* s, size_t row, bool with_kv, RowImage* img) {
    zg_ctx* ctx = s->m->ctx;
    const zg_geometry& g = s->m->g;
    const size_t esz = s->kv_bf16 ? 2 : 4, kvb = (size_t)s->pos[row] * kvw(g) * esz;
    img->pos = s->pos[row];
    img->with_kv = with_kv;
    img->bytes = s->ring.size() * (ring_floats(g) + rec_floats(g)) * 4 + (with_kv ? s->kc.size() * 2 * kvb : 0);
    ZG_HIP(hipMalloc(&img->dev, std::max<size_t>(img->bytes, 256)));
    char* at = (char*)img->dev;
    hipStream_t st = ctx->stream;
    for (size_t i = 0; i < s->ring.size(); ++i) {
        ZG_HIP(hipMemcpyAsync(at, s->ring[i] + row * ring_floats(g), ring_floats(g) * 4, hipMemcpyDeviceToDevice, st));
        at += ring_floats(g) * 4;
        ZG_HIP(hipMemcpyAsync(at, rec_half(s, i, row, s->cur[row]), rec_floats(g) * 4, hipMemcpyDeviceToDevice, st));
        at += rec_floats(g) * 4;
    }
    if (with_kv && kvb)
        for (size_t i = 0; i < s->kc.size(); ++i)
            for (void* cache : {s->kc[i], s->vc[i]}) {
                ZG_HIP(hipMemcpyAsync(at, (char*)cache + row * kv_row_bytes(s), kvb, hipMemcpyDeviceToDevice, st));
                at += kvb;
            }
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

// The row takes the image's state and position (its GDN state in half 0).
// Without KV the row keeps its cache, whose prefix [0, pos) the image's
// position must not exceed the row's own at save time.
int load_row(zg_session* s, size_t row, const RowImage& img) {
    zg_ctx* ctx = s->m->ctx;
    const zg_geometry& g = s->m->g;
    const size_t esz = s->kv_bf16 ? 2 : 4, kvb = (size_t)img.pos * kvw(g) * esz;
    const char* at = (const char*)img.dev;
    hipStream_t st = ctx->stream;
    for (size_t i = 0; i < s->ring.size(); ++i) {
        ZG_HIP(hipMemcpyAsync(s->ring[i] + row * ring_floats(g), at, ring_floats(g) * 4, hipMemcpyDeviceToDevice, st));
        at += ring_floats(g) * 4;
        ZG_HIP(hipMemcpyAsync(rec_half(s, i, row, 0), at, rec_floats(g) * 4, hipMemcpyDeviceToDevice, st));
        at += rec_floats(g) * 4;
    }
    if (img.with_kv && kvb)
        for (size_t i = 0; i < s->kc.size(); ++i)
            for (void* cache : {s->kc[i], s->vc[i]}) {
                ZG_HIP(hipMemcpyAsync((char*)cache + row * kv_row_bytes(s), at, kvb, hipMemcpyDeviceToDevice, st));
                at += kvb;
            }
    ZG_HIP(hipStreamSynchronize(st));
    s->pos[row] = img.pos;
    s->cur[row] = 0;
    s->pos_dirty = true;
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

void free_image(RowImage& img) {
    if (img.dev) (void)hipFree(img.dev);
    img.dev = nullptr;
}

std::atomic<uint64_t> g_model_serial{1};

}  // namespace

struct zg_snapshot {
    uint64_t model_serial = 0;
    int device = 0;
    int kv_bf16 = 0;
    RowImage img;
};

namespace {}  // namespace

extern "C" {

int zg_model_admit(int profile, const zg_geometry* g, const zg_tensor_desc* tensors, size_t n, char* msg,
                   size_t msg_len) {
    std::string why;
    const int rc = admit_model(profile, g, tensors, n, &why);
    if (msg && msg_len) {
        const size_t k = std::min(why.size(), msg_len - 1);
        memcpy(msg, why.data(), k);
        msg[k] = 0;
    }
    return rc;
}

int zg_model_load(zg_ctx* ctx, uint64_t source_id, const zg_geometry* g, const zg_tensor_desc* tensors, size_t n,
                  zg_model** out) {
    if (!ctx || !g || !tensors || !out) return fail(ctx, ZG_E_MALFORMED, "invalid model load arguments");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    *out = nullptr;
    if (source_id == 0) return fail(ctx, ZG_E_MALFORMED, "unbound source identity cannot own a resident model");
    {
        std::string why;
        const int rc = admit_model(ZG_PROFILE_GGUF_SOURCE_V1, g, tensors, n, &why);
        if (rc) return fail(ctx, rc, why);
    }
    auto m = new zg_model();
    m->ctx = ctx;
    m->source = source_id;
    m->serial = g_model_serial.fetch_add(1);
    m->g = *g;
    const uint64_t H = g->hidden, F = g->ffn, V = g->vocab, W = (uint64_t)g->gdn_heads * g->gdn_dim;
    const uint64_t QD = (uint64_t)g->q_heads * g->head_dim, KD = (uint64_t)g->kv_heads * g->head_dim;
    int rc = load_single(m, tensors, n, "token_embd.weight", H, V, zg::PRO_RMS, &m->embd);
    if (!rc) rc = load_vector(m, tensors, n, "output_norm.weight", H, &m->out_norm);
    m->layers.resize(g->layers);
    for (unsigned i = 0; i < g->layers && !rc; ++i) {
        LayerW& L = m->layers[i];
        // config.rs:146-167: full attention where (i + 1) % interval == 0
        L.full = ((i + 1) % g->full_attention_interval) == 0;
        rc = load_vector(m, tensors, n, lname(i, "attn_norm.weight"), H, &L.attn_norm);
        if (!rc) rc = load_vector(m, tensors, n, lname(i, "post_attention_norm.weight"), H, &L.post_norm);
        if (!rc)
            rc = load_stack(m, tensors, n, {lname(i, "ffn_gate.weight"), lname(i, "ffn_up.weight")}, H, {F, F},
                            lname(i, "ffn_gate_up"), zg::PRO_RMS, &L.ffn_gu);
        if (!rc)
            rc = load_single(m, tensors, n, lname(i, "ffn_down.weight"), F, H, zg::PRO_SILU_MUL, &L.ffn_down);
        if (rc) break;
        if (L.full) {
            rc = load_stack(m, tensors, n,
                            {lname(i, "attn_q.weight"), lname(i, "attn_k.weight"), lname(i, "attn_v.weight")}, H,
                            {2 * QD, KD, KD}, lname(i, "attn_qkv_in"), zg::PRO_RMS, &L.in_proj);
            if (!rc)
                rc = load_single(m, tensors, n, lname(i, "attn_output.weight"), QD, H, zg::PRO_PLAIN, &L.out_proj);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "attn_q_norm.weight"), g->head_dim, &L.q_norm);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "attn_k_norm.weight"), g->head_dim, &L.k_norm);
            m->n_attn++;
        } else {
            rc = load_stack(m, tensors, n,
                            {lname(i, "attn_qkv.weight"), lname(i, "attn_gate.weight"), lname(i, "ssm_alpha.weight"),
                             lname(i, "ssm_beta.weight")},
                            H, {3 * W, W, g->gdn_heads, g->gdn_heads}, lname(i, "gdn_in"), zg::PRO_RMS, &L.in_proj);
            if (!rc) rc = load_single(m, tensors, n, lname(i, "ssm_out.weight"), W, H, zg::PRO_GATED, &L.out_proj);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "ssm_conv1d.weight"), 4 * 3 * W, &L.conv_w);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "ssm_norm.weight"), g->gdn_dim, &L.ssm_norm);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "ssm_a"), g->gdn_heads, &L.ssm_a);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "ssm_dt.bias"), g->gdn_heads, &L.ssm_dt);
            m->n_gdn++;
        }
    }
    if (rc) {
        zg_model_destroy(m);
        return rc;
    }
    *out = m;
    return ZG_COMPLETED;
}

void zg_model_destroy(zg_model* m) {
    if (!m) return;
    zg_ctx* ctx = m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    for (void* p : m->vecs) (void)hipFree(p);
    for (zg_weight* w : m->refs) {
        w->model_refs -= 1;
        if (w->model_refs == 0 && !w->api_pinned) zgc::drop_weight(ctx, w);
    }
    delete m;
}

int zg_session_create(zg_model* m, size_t max_batch, size_t max_context, int kv_dtype, zg_session** out) {
    if (!m || !out) return ZG_E_MALFORMED;
    zg_ctx* ctx = m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    *out = nullptr;
    const zg_geometry& g = m->g;
    if (max_batch == 0 || max_batch > 64 || max_context == 0 || max_context > g.max_context)
        return fail(ctx, ZG_E_LIMIT, "session batch must be 1..64 and context within the model's");
    if (kv_dtype != ZG_BF16 && kv_dtype != ZG_F32) return fail(ctx, ZG_E_MALFORMED, "KV cache dtype must be BF16 or F32");
    if (max_batch > 1) {
        // the batched rows' 32-row kernel reads Q4_K weights in its MFMA
        // tile order; the 16-row kernel (K a multiple of 1024 up to 6144)
        // reads the weight's own layout, and zg_prefill_batched builds the
        // prompt GEMM's tiles when it first needs them
        std::vector<zg_weight*> ws = {m->embd};
        for (auto& L : m->layers) {
            ws.insert(ws.end(), {L.out_proj, L.ffn_down});
            for (const Part& p : L.in_proj) ws.push_back(p.w);
            for (const Part& p : L.ffn_gu) ws.push_back(p.w);
        }
        for (zg_weight* w : ws)
            if (w && w->dw.type == zg::kQ4_K && !w->dw.qs_t && !zg::xh16_layout(max_batch, w->dw.K)) {
                const hipError_t e = zg::ensure_mfma_tiles(w->dw, ctx->stream);
                if (e != hipSuccess) return fail(ctx, ZG_E_RESOURCE, "MFMA tile layout of a Q4_K weight");
            }
        if (hipStreamSynchronize(ctx->stream) != hipSuccess) return fail(ctx, ZG_E_DEVICE, "tile layout build");
    }
    auto s = new zg_session();
    s->m = m;
    s->max_batch = max_batch;
    s->max_ctx = max_context;
    s->kv_bf16 = kv_dtype == ZG_BF16;
    s->pos.assign(max_batch, 0);
    s->row_bad.assign(max_batch, 0);
    const char* env = getenv("ZG_GRAPHS");
    s->use_graphs = !(env && env[0] == '0');
    const size_t B = max_batch, H = g.hidden, F = g.ffn, V = g.vocab, W = (size_t)g.gdn_heads * g.gdn_dim;
    const size_t QD = (size_t)g.q_heads * g.head_dim;
    s->y0w = std::max({4 * W + 2 * (size_t)g.gdn_heads, 2 * QD + 2 * kvw(g), 2 * F});
    int rc = 0;
    auto A = [&](void** p, size_t bytes) {
        if (!rc) rc = dalloc(s, p, bytes);
    };
    s->cur.assign(max_batch, 0);
    if (hipEventCreateWithFlags(&s->dev_ev, hipEventDisableTiming) != hipSuccess) {
        delete s;
        return fail(ctx, ZG_E_DEVICE, "session event");
    }
    A((void**)&s->d_pos, B * 4);
    A((void**)&s->d_ntok, B * 4);
    A((void**)&s->d_cur, B * 4);
    A((void**)&s->d_status, 4);
    A((void**)&s->d_tokens, B * 4);
    A((void**)&s->d_greedy, B * 4);
    A((void**)&s->tickets, B * 4);
    // greedy partials: argmax_step's, or one per workgroup of the one-row LM head
    const size_t nparts = std::max<size_t>(zg::argmax_partials(B), 2048);
    A((void**)&s->pmax, nparts * 4);
    A((void**)&s->att_stats, B * g.q_heads * 2 * 4);
    A(&s->xh, zg::batched_scratch_bytes(B, std::max({H, F, W, QD})));
    if (B > 1) A((void**)&s->parts, 8 * ((B + 31) / 32 * 32) * H * sizeof(float));
    if (B > 1) A(&s->xh3, zg::batched_scratch_bytes(B, H));
    if (B > 1) A((void**)&s->rss, (B + 31) / 32 * 32 * ((H + 15) / 16) * sizeof(double));
    if (B > 1) A(&s->xh2, zg::batched_scratch_bytes(B, F));
    A((void**)&s->pidx, nparts * 4);
    A((void**)&s->x, B * H * 4);
    A((void**)&s->y0, B * s->y0w * 4);
    A((void**)&s->core, B * W * 4);
    A((void**)&s->gated, W * 4);
    A((void**)&s->ao, B * QD * 4);
    A((void**)&s->logits, B * V * 4);
    A((void**)&s->scores, B * g.q_heads * max_context * 4);
    if (m->all_q4k) {
        // the projections are tolerance-bound already: attention takes the
        // split-T form; models on exact codecs keep the reference's order
        // end to end
        size_t bytes = 0;
        for (size_t r = 1; r <= B; ++r)
            if (zg::attn_split_supported(r, (int)g.q_heads, (int)g.kv_heads, max_context))
                bytes = std::max(bytes, zg::attn_split_part_bytes(r, (int)g.q_heads, (int)g.kv_heads, max_context));
        if (bytes) {
            A((void**)&s->att_part, bytes);
            A((void**)&s->rope, max_context * 32 * 2 * sizeof(float));
            if (!rc && zg::rope_table(s->rope, max_context, powf(10000000.0f, -2.0f / 64.0f), ctx->stream) !=
                           hipSuccess)
                rc = ZG_E_DEVICE;
        }
    }
    s->layer_slot.resize(g.layers);
    for (size_t i = 0; i < m->layers.size() && !rc; ++i) {
        if (m->layers[i].full) {
            s->layer_slot[i] = (int)s->kc.size();
            void *k = nullptr, *v = nullptr;
            const size_t bytes = B * max_context * kvw(g) * (s->kv_bf16 ? 2 : 4);
            A(&k, bytes);
            A(&v, bytes);
            s->kc.push_back(k);
            s->vc.push_back(v);
        } else {
            s->layer_slot[i] = (int)s->ring.size();
            float *c = nullptr, *r = nullptr;
            A((void**)&c, B * ring_floats(g) * 4);
            A((void**)&r, B * 2 * rec_floats(g) * 4);  // published half + draft half per row
            s->ring.push_back(c);
            s->rec.push_back(r);
        }
    }
    if (rc) {
        zg_session_destroy(s);
        return rc;
    }
    *out = s;
    return ZG_COMPLETED;
}

void zg_session_destroy(zg_session* s) {
    if (!s) return;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    for (auto& kv : s->graphs) (void)hipGraphExecDestroy(kv.second.exec);
    for (void* p : s->allocs) (void)hipFree(p);
    for (void* p : s->pf) (void)hipFree(p);
    if (s->dev_ev) (void)hipEventDestroy(s->dev_ev);
    delete s;
}

int zg_session_reset(zg_session* s) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    const zg_geometry& g = s->m->g;
    const size_t B = s->max_batch;
    int rc = settle(s);
    if (rc) return rc;
    for (float* c : s->ring) ZG_HIP(hipMemsetAsync(c, 0, B * ring_floats(g) * 4, ctx->stream));
    for (float* r : s->rec) ZG_HIP(hipMemsetAsync(r, 0, B * 2 * rec_floats(g) * 4, ctx->stream));
    const size_t kvb = B * s->max_ctx * kvw(g) * (s->kv_bf16 ? 2 : 4);
    for (size_t i = 0; i < s->kc.size(); ++i) {
        ZG_HIP(hipMemsetAsync(s->kc[i], 0, kvb, ctx->stream));
        ZG_HIP(hipMemsetAsync(s->vc[i], 0, kvb, ctx->stream));
    }
    ZG_HIP(hipMemsetAsync(s->d_status, 0, 4, ctx->stream));
    ZG_HIP(hipMemsetAsync(s->tickets, 0, B * 4, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    std::fill(s->pos.begin(), s->pos.end(), 0);
    std::fill(s->cur.begin(), s->cur.end(), 0);
    s->pos_dirty = true;
    std::fill(s->row_bad.begin(), s->row_bad.end(), 0);
    s->poisoned = false;
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

// Row retirement: the row's conv history, GDN state and KV cache back to
// zero and its position to 0; the other rows are untouched.
int zg_session_reset_row(zg_session* s, size_t row) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (row >= s->max_batch) return fail(ctx, ZG_E_LIMIT, "row outside the session batch");
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    int rc = settle(s);  // work queued on a caller's stream lands first
    if (rc) return rc;
    for (float* c : s->ring) ZG_HIP(hipMemsetAsync(c + row * ring_floats(g), 0, ring_floats(g) * 4, st));
    for (float* r : s->rec) ZG_HIP(hipMemsetAsync(r + row * 2 * rec_floats(g), 0, 2 * rec_floats(g) * 4, st));
    const size_t rowb = s->max_ctx * kvw(g) * (s->kv_bf16 ? 2 : 4);
    for (size_t i = 0; i < s->kc.size(); ++i) {
        ZG_HIP(hipMemsetAsync((char*)s->kc[i] + row * rowb, 0, rowb, st));
        ZG_HIP(hipMemsetAsync((char*)s->vc[i] + row * rowb, 0, rowb, st));
    }
    ZG_HIP(hipStreamSynchronize(st));
    s->pos[row] = 0;
    s->cur[row] = 0;
    s->pos_dirty = true;
    clear_poison(s, row);
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

// Row admission by copy: row dst takes row src's whole state (conv history,
// GDN state, the KV cache up to src's position) and position.  With
// zg_session_reset_row this keeps the active rows of a continuous batch
// dense (retire row r: copy the last active row into r, reset the last),
// and it forks a prefilled prompt into several rows.
int zg_session_copy_row(zg_session* s, size_t dst, size_t src) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (dst >= s->max_batch || src >= s->max_batch) return fail(ctx, ZG_E_LIMIT, "row outside the session batch");
    if (dst == src) return ZG_COMPLETED;
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    int rc = settle(s);
    if (rc) return rc;
    for (float* c : s->ring)
        ZG_HIP(hipMemcpyAsync(c + dst * ring_floats(g), c + src * ring_floats(g), ring_floats(g) * 4,
                              hipMemcpyDeviceToDevice, st));
    // src's published half becomes dst's half 0
    for (size_t i = 0; i < s->rec.size(); ++i)
        ZG_HIP(hipMemcpyAsync(rec_half(s, i, dst, 0), rec_half(s, i, src, s->cur[src]), rec_floats(g) * 4,
                              hipMemcpyDeviceToDevice, st));
    const size_t esz = s->kv_bf16 ? 2 : 4;
    const size_t rowb = s->max_ctx * kvw(g) * esz;
    const size_t used = (size_t)s->pos[src] * kvw(g) * esz;
    const size_t stale = (size_t)s->pos[dst] * kvw(g) * esz;
    for (size_t i = 0; i < s->kc.size(); ++i) {
        for (void* cache : {s->kc[i], s->vc[i]}) {
            char* base = (char*)cache;
            if (used) ZG_HIP(hipMemcpyAsync(base + dst * rowb, base + src * rowb, used, hipMemcpyDeviceToDevice, st));
            if (stale > used) ZG_HIP(hipMemsetAsync(base + dst * rowb + used, 0, stale - used, st));
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    s->pos[dst] = s->pos[src];
    s->cur[dst] = 0;
    s->pos_dirty = true;
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

int zg_session_position(const zg_session* s, size_t row) {
    if (!s || row >= s->max_batch) return -1;
    return s->pos[row];
}

namespace {

// One step of rows [0, rows) from host tokens; with `commit` it publishes
// (QwenDenseCpu::forward), else it leaves a proposal (next_logits).
int host_step(zg_session* s, size_t rows, const uint32_t* tokens, float* logits, uint32_t* greedy, bool commit) {
    zg_ctx* ctx = s->m->ctx;
    int rc = settle(s);
    if (rc) return rc;
    if ((rc = check_rows(s, rows))) return rc;
    for (size_t b = 0; b < rows; ++b)
        if (tokens[b] >= s->m->g.vocab) return fail(ctx, ZG_E_MALFORMED, "decode step contains an out-of-vocabulary token id");
    hipStream_t st = ctx->stream;
    s->pending_rows = 0;
    if ((rc = sync_positions(s, st))) return rc;
    ZG_HIP(hipMemcpyAsync(s->d_tokens, tokens, rows * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipStreamSynchronize(st));
    const bool want = logits || greedy;
    if ((rc = run_step(s, rows, s->d_tokens, want ? s->logits : nullptr, want ? s->d_greedy : nullptr, commit, st))) {
        poison(s);  // a launch failed: the device state is unknown
        return rc;
    }
    if ((rc = read_status(s, st))) return rc;  // nothing was published
    if (commit) {
        for (size_t b = 0; b < rows; ++b) {
            s->pos[b] += 1;
            s->cur[b] ^= 1;
        }
    } else {
        s->pending_rows = rows;
    }
    if (logits) ZG_HIP(hipMemcpyAsync(logits, s->logits, rows * s->m->g.vocab * 4, hipMemcpyDeviceToHost, st));
    if (greedy) ZG_HIP(hipMemcpyAsync(greedy, s->d_greedy, rows * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

}  // namespace

int zg_decode_step(zg_session* s, size_t rows, const uint32_t* tokens, float* logits, uint32_t* greedy) {
    if (!s || !tokens) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    return host_step(s, rows, tokens, logits, greedy, true);
}

int zg_session_propose(zg_session* s, size_t rows, const uint32_t* tokens, float* logits, uint32_t* greedy) {
    if (!s || !tokens) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    return host_step(s, rows, tokens, logits, greedy, false);
}

int zg_session_commit(zg_session* s) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = settle(s);
    if (rc) return rc;
    if (s->pending_rows == 0) return fail(ctx, ZG_E_STATE, "session holds no prepared proposal");
    const size_t rows = s->pending_rows;
    zg::StepCommit sc;
    sc.pos = s->d_pos;
    sc.ntok = s->d_ntok;
    sc.cur = s->d_cur;
    ZG_HIP(zg::commit_step(sc, s->d_status, rows, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    for (size_t b = 0; b < rows; ++b) {
        s->pos[b] += 1;
        s->cur[b] ^= 1;
    }
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

// Per-token prefill, atomic over the whole call (prefill_transaction,
// lib.rs:1114-1187): the rows' published state is saved on the device
// first and restored if any token fails.
int zg_prefill(zg_session* s, size_t rows, size_t n, const uint32_t* tokens, float* logits) {
    if (!s || !tokens || n == 0) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = settle(s);
    if (rc) return rc;
    if ((rc = check_rows(s, rows))) return rc;
    for (size_t b = 0; b < rows; ++b)
        if ((size_t)s->pos[b] + n > s->max_ctx) return fail(ctx, ZG_E_LIMIT, "prompt exceeds the session context");
    for (size_t i = 0; i < rows * n; ++i)
        if (tokens[i] >= s->m->g.vocab) return fail(ctx, ZG_E_MALFORMED, "prompt contains an out-of-vocabulary token id");
    std::vector<RowImage> saved(rows);
    for (size_t b = 0; b < rows && !rc; ++b) rc = save_row(s, b, false, &saved[b]);
    std::vector<uint32_t> col(rows);
    for (size_t t = 0; t < n && !rc; ++t) {
        for (size_t b = 0; b < rows; ++b) col[b] = tokens[b * n + t];
        rc = host_step(s, rows, col.data(), t + 1 == n ? logits : nullptr, nullptr, true);
    }
    if (rc) {
        const std::string msg = last_message(ctx);
        for (size_t b = 0; b < rows; ++b)
            if (saved[b].dev && load_row(s, b, saved[b])) poison(s);
        zgc::fail(ctx, rc, msg);
    }
    for (RowImage& img : saved) free_image(img);
    return rc;
}

// Batched prefill of one row: embed the n tokens, run every layer over all of
// them (batched MFMA projections, chunked GDN prefill, causal attention with
// the KV append), and the LM head on the last.  Same result as n decode
// steps of that row up to the order of summation (end-to-end tolerance).
namespace {

int prefill_batched_body(zg_session* s, size_t row, size_t n, const uint32_t* tokens, float* logits) {
    zg_model* m = s->m;
    zg_ctx* ctx = m->ctx;
    const zg_geometry& g = m->g;
    if ((size_t)s->pos[row] + n > s->max_ctx) return fail(ctx, ZG_E_LIMIT, "prompt exceeds the session context");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= g.vocab) return fail(ctx, ZG_E_MALFORMED, "prompt contains an out-of-vocabulary token id");
    // the chunked GDN prefill is built for 128-wide heads with the model's
    // 1e-6 norm epsilon; the attention kernels for 256-wide heads, <= 4
    // query heads per KV head
    if (g.gdn_dim != 128 || g.head_dim != 256 || g.eps != 1e-6f || g.kv_heads == 0 || g.q_heads % g.kv_heads ||
        g.q_heads / g.kv_heads > 4)
        return fail(ctx, ZG_E_UNSUPPORTED, "batched prefill geometry not supported: use zg_prefill");
    std::vector<zg_weight*> ws;
    for (auto& L : m->layers) {
        if (L.in_proj.size() != 1 || L.ffn_gu.size() != 1)
            return fail(ctx, ZG_E_UNSUPPORTED, "batched prefill needs Q4_K projections: use zg_prefill");
        ws.insert(ws.end(), {L.in_proj[0].w, L.out_proj, L.ffn_gu[0].w, L.ffn_down});
    }
    for (zg_weight* w : ws)
        if (!w || w->dw.type != zg::kQ4_K)
            return fail(ctx, ZG_E_UNSUPPORTED, "batched prefill needs Q4_K projections: use zg_prefill");
    hipStream_t st = ctx->stream;
    // the device positions take the host's (a status failure below re-reads
    // them, and must find every other row as the host has it)
    int rc0 = sync_positions(s, st);
    if (rc0) return rc0;
    for (zg_weight* w : ws)
        if (!w->dw.qs_t) ZG_HIP(zg::ensure_mfma_tiles(w->dw, st));
    const size_t H = g.hidden, F = g.ffn, W = (size_t)g.gdn_heads * g.gdn_dim, GH = g.gdn_heads;
    const size_t QD = (size_t)g.q_heads * g.head_dim;
    const size_t mpad = (n + 31) / 32 * 32;
    const size_t ldp = s->y0w;
    // the prompt GEMM addresses each operand with 32-bit byte offsets
    for (zg_weight* w : ws)
        if (zg::prompt_gemm_bytes(n, w->dw.K, w->dw.N) >= ((uint64_t)1 << 32))
            return fail(ctx, ZG_E_LIMIT, "prompt too long for the batched prefill (an operand of its projections "
                                         "would reach 4 GiB): split it over several calls");
    enum { X, P, Q, K, V, BETA, LOGD, CORE, QB, OB, XH, XH2, CHUNK, TOK, ATTP, RPARTS, NBUF };
    // the split residual projections' partial sums: a split is taken only
    // while the tiles give at most 256 workgroups of 64 x 256 outputs, so two
    // runs of those (or four of a quarter as many) bound it
    const size_t kSplitParts = 2 * 256 * 64 * 256;
    if (n > s->pf_cap) {
        ZG_HIP(hipStreamSynchronize(st));
        for (void* p : s->pf) (void)hipFree(p);
        s->pf.assign(NBUF, nullptr);
        s->pf_cap = 0;
        const size_t bytes[NBUF] = {mpad * H * 4, mpad * ldp * 4, n * W * 4, n * W * 4, n * W * 4, n * GH * 4,
                                    n * GH * 4, mpad * W * 4, n * QD * 4, mpad * QD * 4,
                                    zg::batched_scratch_bytes(n, std::max({H, F, W, QD})),
                                    zg::batched_scratch_bytes(n, F), zg::gdn_chunk_scratch_bytes(n, GH), n * 4,
                                    zg::attn_prefill_part_bytes(n, (int)g.q_heads), kSplitParts * 4};
        for (int i = 0; i < NBUF; ++i) {
            ZG_HIP(hipMalloc(&s->pf[i], std::max<size_t>(bytes[i], 256)));
            ZG_HIP(hipMemsetAsync(s->pf[i], 0, std::max<size_t>(bytes[i], 256), st));  // stream-ordered
        }
        s->pf_cap = n;
    }
    float* x = (float*)s->pf[X];
    float* pj = (float*)s->pf[P];
    uint32_t* dtok = (uint32_t*)s->pf[TOK];
    const int pos0 = s->pos[row];
    ZG_HIP(hipMemcpyAsync(dtok, tokens, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipStreamSynchronize(st));
    ZG_HIP(zg::embed(m->embd->dw, dtok, x, n, s->d_status, st));
    auto gemm = [&](zg_weight* w, int pro, const float* xin, size_t ldx, const float* x2, size_t ldx2,
                    const float* gamma, int epi, float* y, size_t ldy, void* xh_out = nullptr,
                    const void* xh_in = nullptr) {
        zg::FusedGemvArgs f;
        f.M = (int)n;
        f.pro = pro;
        f.epi = epi;
        f.x = xin;
        f.ldx = ldx;
        f.x2 = x2;
        f.ldx2 = ldx2;
        f.gamma = gamma;
        f.eps = g.eps;
        f.group = (int)g.gdn_dim;
        f.y = y;
        f.ldy = ldy;
        f.status = s->d_status;
        f.xh_out = xh_out;
        f.xh_in = xh_in;
        if (epi == zg::EPI_RESID && ldy == H) {
            f.prompt_parts = (float*)s->pf[RPARTS];
            f.prompt_parts_n = kSplitParts;
        }
        return zg::batched_gemv(w->dw, f, s->pf[XH], st);
    };
    for (size_t i = 0; i < m->layers.size(); ++i) {
        LayerW& L = m->layers[i];
        const int slot = s->layer_slot[i];
        if (!L.full) {
            ZG_HIP(gemm(L.in_proj[0].w, zg::PRO_RMS, x, H, nullptr, 0, L.attn_norm, zg::EPI_STORE, pj, ldp));
            float* ring = s->ring[slot] + row * 3 * W * 4;
            float* state = rec_half(s, (size_t)slot, row, s->cur[row]);
            ZG_HIP(zg::gdn_prefill_conv(pj, ldp, n, W, GH, L.conv_w, ring, pos0, L.ssm_dt, L.ssm_a, (float*)s->pf[Q],
                                        (float*)s->pf[K], (float*)s->pf[V], (float*)s->pf[BETA],
                                        (float*)s->pf[LOGD], st));
            ZG_HIP(zg::gdn_chunk_prefill((const float*)s->pf[Q], (const float*)s->pf[K], (const float*)s->pf[V],
                                         (const float*)s->pf[BETA], (const float*)s->pf[LOGD], n, GH, state,
                                         (float*)s->pf[CORE], (float*)s->pf[CHUNK], false, false, st));
            ZG_HIP(gemm(L.out_proj, zg::PRO_GATED, (const float*)s->pf[CORE], W, pj + 3 * W, ldp, L.ssm_norm,
                        zg::EPI_RESID, x, H));
        } else {
            ZG_HIP(gemm(L.in_proj[0].w, zg::PRO_RMS, x, H, nullptr, 0, L.attn_norm, zg::EPI_STORE, pj, ldp));
            zg::AttnPrefillArgs a;
            a.P = pj;
            a.ldp = ldp;
            a.n = n;
            a.nq = (int)g.q_heads;
            a.nkv = (int)g.kv_heads;
            a.pos0 = pos0;
            a.kv_bf16 = s->kv_bf16;
            a.qnorm = L.q_norm;
            a.knorm = L.k_norm;
            a.eps = g.eps;
            a.theta_scale = powf(10000000.0f, -2.0f / 64.0f);
            a.scale = 1.0f / sqrtf((float)g.head_dim);
            const size_t esz = s->kv_bf16 ? 2 : 4;
            a.kcache = (char*)s->kc[slot] + row * s->max_ctx * kvw(g) * esz;
            a.vcache = (char*)s->vc[slot] + row * s->max_ctx * kvw(g) * esz;
            a.Q = (float*)s->pf[QB];
            a.out = (float*)s->pf[OB];
            a.status = s->d_status;
            a.part = (float*)s->pf[ATTP];
            a.rope = s->rope;  // (null unless the session holds the split-T attention buffers)
            ZG_HIP(zg::attn_prefill(a, st));
            ZG_HIP(gemm(L.out_proj, zg::PRO_PLAIN, (const float*)s->pf[OB], QD, nullptr, 0, nullptr, zg::EPI_RESID, x,
                        H));
        }
        const zg::DeviceWeight& gu = L.ffn_gu[0].w->dw;
        if (zg::batched_glu_supported(gu.type, gu.K, gu.N)) {
            ZG_HIP(gemm(L.ffn_gu[0].w, zg::PRO_RMS, x, H, nullptr, 0, L.post_norm, zg::EPI_GLU, pj, ldp, s->pf[XH2]));
            ZG_HIP(gemm(L.ffn_down, zg::PRO_PLAIN, pj, ldp, nullptr, 0, nullptr, zg::EPI_RESID, x, H, nullptr,
                        s->pf[XH2]));
        } else {
            ZG_HIP(gemm(L.ffn_gu[0].w, zg::PRO_RMS, x, H, nullptr, 0, L.post_norm, zg::EPI_STORE, pj, ldp));
            ZG_HIP(gemm(L.ffn_down, zg::PRO_SILU_MUL, pj, ldp, pj + F, ldp, nullptr, zg::EPI_RESID, x, H));
        }
    }
    if (!logits) {
        int rc = read_status(s, st);
        if (rc) return rc;
        s->pos[row] += (int)n;
        s->pos_dirty = true;
        return ZG_COMPLETED;
    }
    // LM head on the last prompt token (tied embedding, output norm)
    zg::FusedGemvArgs f;
    f.M = 1;
    f.pro = zg::PRO_RMS;
    f.epi = zg::EPI_STORE;
    f.x = x + (n - 1) * H;
    f.ldx = H;
    f.gamma = m->out_norm;
    f.eps = g.eps;
    f.y = s->logits;
    f.ldy = g.vocab;
    f.status = s->d_status;
    ZG_HIP(zg::fused_gemv(m->embd->dw, f, st));
    int rc = read_status(s, st);
    if (rc) return rc;
    ZG_HIP(hipMemcpyAsync(logits, s->logits, g.vocab * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    s->pos[row] += (int)n;
    s->pos_dirty = true;
    return ZG_COMPLETED;
}

}  // namespace

// Atomic like prefill_transaction (lib.rs:1114-1187): the row's conv ring
// and GDN state are saved on the device first and put back if the prompt
// fails (its KV rows lie past the published position).
int zg_prefill_batched(zg_session* s, size_t row, size_t n, const uint32_t* tokens, float* logits) {
    if (!s || !tokens || n == 0) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (s->poisoned) return fail(ctx, ZG_E_STATE, "session poisoned by a failed launch: reset or import state");
    if (row >= s->max_batch) return fail(ctx, ZG_E_LIMIT, "row outside the session batch");
    int rc = settle(s);
    if (rc) return rc;
    s->pending_rows = 0;
    RowImage saved;
    if ((rc = save_row(s, row, false, &saved))) return rc;
    rc = prefill_batched_body(s, row, n, tokens, logits);
    if (rc) {
        const std::string msg = last_message(ctx);
        if (load_row(s, row, saved)) poison(s);
        zgc::fail(ctx, rc, msg);
    }
    free_image(saved);
    return rc;
}

int zg_decode_step_device(zg_session* s, size_t rows, const uint32_t* d_tokens, float* d_logits, uint32_t* d_greedy,
                          void* stream) {
    if (!s || !d_tokens) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = check_rows(s, rows);
    if (rc) return rc;
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    s->pending_rows = 0;
    if ((rc = sync_positions(s, st))) return rc;
    if ((rc = run_step(s, rows, d_tokens, d_logits ? d_logits : (d_greedy ? s->logits : nullptr), d_greedy, true,
                       st))) {
        poison(s);
        return rc;
    }
    ZG_HIP(hipEventRecord(s->dev_ev, st));
    s->async_steps = true;
    // optimistic host mirrors (the device commits only a clean step; settle
    // and zg_session_check re-read them)
    for (size_t b = 0; b < rows; ++b) {
        s->pos[b] += 1;
        s->cur[b] ^= 1;
    }
    return ZG_COMPLETED;
}

int zg_session_check(zg_session* s, void* stream) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    if (s->async_steps) {
        ZG_HIP(hipEventSynchronize(s->dev_ev));
        s->async_steps = false;
    }
    int rc = read_status(s, st);
    if (rc) return rc;
    return pull_positions(s, st);
}

size_t zg_state_floats(const zg_session* s, size_t row) {
    if (!s || row >= s->max_batch) return 0;
    const zg_geometry& g = s->m->g;
    return s->m->n_gdn * (conv_floats(g) + rec_floats(g)) + s->m->n_attn * 2 * (size_t)s->pos[row] * kvw(g);
}

int zg_state_export(zg_session* s, size_t row, float* out, size_t n) {
    if (!s || !out) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = settle(s);
    if (rc) return rc;
    if (row >= s->max_batch || n != zg_state_floats(s, row)) return fail(ctx, ZG_E_MALFORMED, "state length mismatch");
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    const int P = s->pos[row];
    const size_t T = (size_t)P, kw = kvw(g), C = (size_t)g.gdn_heads * g.gdn_dim * 3;
    rc = ensure(ctx, ctx->scratch, std::max<size_t>(T * kw * 4, 256));
    if (rc) return rc;
    std::vector<float> ring(ring_floats(g));
    size_t at = 0;
    for (size_t i = 0; i < s->m->layers.size(); ++i) {
        const int slot = s->layer_slot[i];
        if (!s->m->layers[i].full) {
            // history [channel][oldest..newest] (lib.rs:79-80) from the ring
            ZG_HIP(hipMemcpy(ring.data(), s->ring[slot] + row * ring_floats(g), ring_floats(g) * 4, hipMemcpyDeviceToHost));
            for (size_t c = 0; c < C; ++c)
                for (int k = 0; k < 3; ++k) out[at + c * 3 + k] = ring[c * 4 + ring_slot(P, k)];
            at += conv_floats(g);
            ZG_HIP(hipMemcpy(out + at, rec_half(s, (size_t)slot, row, s->cur[row]), rec_floats(g) * 4,
                             hipMemcpyDeviceToHost));
            at += rec_floats(g);
        } else {
            for (void* cache : {s->kc[slot], s->vc[slot]}) {
                if (T) {
                    if (s->kv_bf16) {
                        ZG_HIP(zg::convert_kv((const uint16_t*)cache + row * s->max_ctx * kw, ctx->scratch.ptr, T * kw, true, st));
                        ZG_HIP(hipMemcpyAsync(out + at, ctx->scratch.ptr, T * kw * 4, hipMemcpyDeviceToHost, st));
                        ZG_HIP(hipStreamSynchronize(st));
                    } else {
                        ZG_HIP(hipMemcpy(out + at, (const float*)cache + row * s->max_ctx * kw, T * kw * 4,
                                         hipMemcpyDeviceToHost));
                    }
                }
                at += T * kw;
            }
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

namespace {

// The row's device state from a host image in the export order; on error
// the row may be partly written (the caller poisons the session).
int import_row(zg_session* s, size_t row, const float* in, int position) {
    zg_ctx* ctx = s->m->ctx;
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    const size_t T = (size_t)position, kw = kvw(g), C = (size_t)g.gdn_heads * g.gdn_dim * 3;
    std::vector<float> ring(ring_floats(g));
    size_t at = 0;
    for (size_t i = 0; i < s->m->layers.size(); ++i) {
        const int slot = s->layer_slot[i];
        if (!s->m->layers[i].full) {
            std::fill(ring.begin(), ring.end(), 0.0f);
            for (size_t c = 0; c < C; ++c)
                for (int k = 0; k < 3; ++k) ring[c * 4 + ring_slot(position, k)] = in[at + c * 3 + k];
            ZG_HIP(hipMemcpy(s->ring[slot] + row * ring_floats(g), ring.data(), ring_floats(g) * 4, hipMemcpyHostToDevice));
            at += conv_floats(g);
            ZG_HIP(hipMemcpy(rec_half(s, (size_t)slot, row, 0), in + at, rec_floats(g) * 4, hipMemcpyHostToDevice));
            at += rec_floats(g);
        } else {
            for (void* cache : {s->kc[slot], s->vc[slot]}) {
                if (T) {
                    if (s->kv_bf16) {
                        ZG_HIP(hipMemcpyAsync(ctx->scratch.ptr, in + at, T * kw * 4, hipMemcpyHostToDevice, st));
                        ZG_HIP(zg::convert_kv(ctx->scratch.ptr, (uint16_t*)cache + row * s->max_ctx * kw, T * kw, false, st));
                        ZG_HIP(hipStreamSynchronize(st));
                    } else {
                        ZG_HIP(hipMemcpy((float*)cache + row * s->max_ctx * kw, in + at, T * kw * 4,
                                         hipMemcpyHostToDevice));
                    }
                }
                at += T * kw;
            }
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

}  // namespace

// Either the row takes the image (state, position, published half 0) or,
// on a refusal or an allocation failure, nothing changes; a device copy
// that fails midway leaves the row partly written, which poisons the
// session until the row is reset, restored or imported again.
int zg_state_import(zg_session* s, size_t row, const float* in, size_t n, int position) {
    if (!s || !in) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (row >= s->max_batch || position < 0 || (size_t)position > s->max_ctx)
        return fail(ctx, ZG_E_MALFORMED, "invalid state import row or position");
    int rc = settle(s);
    if (rc) return rc;
    const int saved = s->pos[row];
    s->pos[row] = position;  // zg_state_floats sizes the KV part by the row's position
    const size_t want = zg_state_floats(s, row);
    s->pos[row] = saved;
    if (n != want || !all_finite(in, n))
        return fail(ctx, ZG_E_MALFORMED, "state import length mismatch or nonfinite state");
    const size_t T = (size_t)position, kw = kvw(s->m->g);
    if ((rc = ensure(ctx, ctx->scratch, std::max<size_t>(T * kw * 4, 256)))) return rc;
    if ((rc = import_row(s, row, in, position))) {
        poison(s);
        return rc;
    }
    s->pos[row] = position;
    s->cur[row] = 0;
    s->pos_dirty = true;
    clear_poison(s, row);
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

int zg_session_fill_random(zg_session* s, size_t rows, size_t prefix, uint64_t seed) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (rows == 0 || rows > s->max_batch || prefix >= s->max_ctx)
        return fail(ctx, ZG_E_LIMIT, "random prefix exceeds the session");
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    int rc = settle(s);
    if (rc) return rc;
    uint64_t k = seed * 0x9e3779b97f4a7c15ull;
    const size_t kw = kvw(g);
    for (size_t i = 0; i < s->ring.size(); ++i) {
        ZG_HIP(zg::fill_normal(s->ring[i], rows * ring_floats(g), false, ++k, 0.5f, st));
        for (size_t b = 0; b < rows; ++b) ZG_HIP(zg::fill_normal(rec_half(s, i, b, 0), rec_floats(g), false, ++k, 0.02f, st));
    }
    for (size_t i = 0; i < s->kc.size(); ++i) {
        for (size_t b = 0; b < rows; ++b) {
            const size_t off = b * s->max_ctx * kw * (s->kv_bf16 ? 2 : 4);
            ZG_HIP(zg::fill_normal((char*)s->kc[i] + off, prefix * kw, s->kv_bf16, ++k, 1.0f, st));
            ZG_HIP(zg::fill_normal((char*)s->vc[i] + off, prefix * kw, s->kv_bf16, ++k, 1.0f, st));
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    for (size_t b = 0; b < rows; ++b) {
        s->pos[b] = (int)prefix;
        s->cur[b] = 0;
        clear_poison(s, b);
    }
    s->pos_dirty = true;
    s->pending_rows = 0;
    return ZG_COMPLETED;
}

int zg_session_snapshot(zg_session* s, size_t row, zg_snapshot** out) {
    if (!s || !out) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    *out = nullptr;
    if (row >= s->max_batch) return fail(ctx, ZG_E_LIMIT, "row outside the session batch");
    int rc = settle(s);
    if (rc) return rc;
    auto snap = new zg_snapshot();
    snap->model_serial = s->m->serial;
    snap->device = ctx->device;
    snap->kv_bf16 = s->kv_bf16;
    if ((rc = save_row(s, row, true, &snap->img))) {
        free_image(snap->img);
        delete snap;
        return rc;
    }
    *out = snap;
    return ZG_COMPLETED;
}

int zg_session_restore(zg_session* s, size_t row, const zg_snapshot* snap) {
    if (!s || !snap) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (row >= s->max_batch) return fail(ctx, ZG_E_LIMIT, "row outside the session batch");
    if (snap->model_serial != s->m->serial || snap->kv_bf16 != s->kv_bf16 || snap->device != ctx->device)
        return fail(ctx, ZG_E_STATE, "foreign snapshot: another model, device or KV cache type");
    if ((size_t)snap->img.pos > s->max_ctx) return fail(ctx, ZG_E_LIMIT, "snapshot exceeds the session context");
    int rc = settle(s);
    if (rc) return rc;
    if ((rc = load_row(s, row, snap->img))) {
        poison(s);
        return rc;
    }
    clear_poison(s, row);
    return ZG_COMPLETED;
}

size_t zg_snapshot_bytes(const zg_snapshot* snap) { return snap ? snap->img.bytes : 0; }
int zg_snapshot_position(const zg_snapshot* snap) { return snap ? snap->img.pos : -1; }

void zg_snapshot_destroy(zg_snapshot* snap) {
    if (!snap) return;
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipSetDevice(snap->device);
    free_image(snap->img);
    (void)hipSetDevice(dev);
    delete snap;
}

}  // extern "C"
