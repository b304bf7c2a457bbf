// Boundary B: resident Qwen3.5 hybrid model + decode sessions, and the GDN /
// attention boundary-A regions.  See zg_model.hip for the per-step schedule.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "zg_context.hpp"

using namespace zgc;

namespace {

struct LayerW {
    bool full = false;
    zg_weight *qkv = nullptr, *gate = nullptr, *alpha = nullptr, *beta = nullptr, *ssm_out = nullptr;
    zg_weight *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
    zg_weight *ffn_gate = nullptr, *ffn_up = nullptr, *ffn_down = nullptr;
    float *attn_norm = nullptr, *post_norm = nullptr, *conv_w = nullptr, *ssm_norm = nullptr, *ssm_a = nullptr,
          *ssm_dt = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

}  // namespace

struct zg_model {
    zg_ctx* ctx = nullptr;
    uint64_t source = 0;
    zg_geometry g{};
    std::vector<LayerW> layers;
    zg_weight* embd = nullptr;
    float* out_norm = nullptr;
    std::vector<void*> vecs;  // device copies of F32 parameter vectors
    size_t n_gdn = 0, n_attn = 0;
};

struct zg_session {
    zg_model* m = nullptr;
    size_t max_batch = 0, max_ctx = 0;
    int kv_bf16 = 1;
    std::vector<int> pos;  // host copy of each row's next position
    bool poisoned = false;
    bool pos_dirty = true;  // device positions must be re-uploaded from pos
    // device buffers
    std::vector<void*> allocs;
    int *d_pos = nullptr, *d_ntok = nullptr, *d_status = nullptr;
    uint32_t *d_tokens = nullptr, *d_greedy = nullptr;
    float *x = nullptr, *y0 = nullptr, *y1 = nullptr, *y2 = nullptr, *y3 = nullptr, *mixed = nullptr, *core = nullptr,
          *gated = nullptr, *out = nullptr, *logits = nullptr, *qr = nullptr, *scores = nullptr, *probs = nullptr;
    void* prep = nullptr;
    size_t prep_bytes = 0, y0w = 0, y1w = 0, y2w = 0, gatedw = 0;
    std::vector<float*> conv, rec;   // per GDN layer
    std::vector<void*> kc, vc;       // per attention layer
    std::vector<int> layer_slot;     // layer -> index into conv/rec or kc/vc
    // prepared-activation memo for one step
    const void* prep_src = nullptr;
    const float* prep_gamma = nullptr;
    int prep_type = -1;
    size_t prep_rows = 0;
};

namespace {

const zg_tensor_desc* find_tensor(const zg_tensor_desc* t, size_t n, const std::string& name) {
    for (size_t i = 0; i < n; ++i)
        if (t[i].name && name == t[i].name) return &t[i];
    return nullptr;
}

std::string lname(unsigned i, const char* suffix) { return "blk." + std::to_string(i) + "." + suffix; }

int load_matrix(zg_model* m, const zg_tensor_desc* ts, size_t n, const std::string& name, uint64_t K, uint64_t N,
                zg_weight** out) {
    zg_ctx* ctx = m->ctx;
    const zg_tensor_desc* t = find_tensor(ts, n, name);
    if (!t) return fail(ctx, ZG_E_MALFORMED, "missing tensor " + name);
    if (t->shape0 != K || t->shape1 != N)
        return fail(ctx, ZG_E_MALFORMED, "tensor " + name + " geometry differs from the model configuration");
    int rc = check_matrix(ctx, t->ggml_type, K, N, t->data, t->nbytes);
    if (rc == ZG_UNSUPPORTED) return fail(ctx, ZG_E_UNSUPPORTED, "tensor " + name + ": " + ctx->err);
    if (rc) return rc;
    return lookup_or_register(ctx, m->source, name.c_str(), t->ggml_type, K, N, t->data, t->nbytes, out);
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

int dalloc(zg_session* s, void** p, size_t bytes) {
    zg_ctx* ctx = s->m->ctx;
    ZG_HIP(hipMalloc(p, bytes < 256 ? 256 : bytes));
    ZG_HIP(hipMemset(*p, 0, bytes < 256 ? 256 : bytes));
    s->allocs.push_back(*p);
    return ZG_COMPLETED;
}

size_t conv_floats(const zg_geometry& g) { return (size_t)g.gdn_heads * g.gdn_dim * 3 * 3; }
size_t rec_floats(const zg_geometry& g) { return (size_t)g.gdn_heads * g.gdn_dim * g.gdn_dim; }
size_t kvw(const zg_geometry& g) { return (size_t)g.kv_heads * g.head_dim; }

// Prepare the activation of `src` for weight w (RMS with gamma when given),
// reusing the previous preparation when source, gamma, codec and rows match.
int project(zg_session* s, zg_weight* w, const float* src, const float* gamma, float* y, size_t B, hipStream_t st) {
    zg_ctx* ctx = s->m->ctx;
    if (!(s->prep_src == src && s->prep_gamma == gamma && s->prep_type == w->dw.type && s->prep_rows == B)) {
        ZG_HIP(zg::act_prepare_for(w->dw.type, src, 0, B, w->dw.K, gamma, s->m->g.eps, s->prep, st));
        s->prep_src = src;
        s->prep_gamma = gamma;
        s->prep_type = w->dw.type;
        s->prep_rows = B;
    }
    ZG_HIP(zg::gemv(w->dw, B, s->prep, y, st));
    return ZG_COMPLETED;
}

void invalidate_prep(zg_session* s) { s->prep_src = nullptr; }

// One decode step for rows [0, B): tokens already in s->d_tokens, positions
// in s->d_pos / s->d_ntok.  Logits land in s->logits, greedy ids in
// s->d_greedy.  Asynchronous on st.
int step(zg_session* s, size_t B, const uint32_t* tokens, float* logits, uint32_t* greedy, hipStream_t st) {
    zg_model* m = s->m;
    zg_ctx* ctx = m->ctx;
    const zg_geometry& g = m->g;
    const size_t H = g.hidden, F = g.ffn, W = (size_t)g.gdn_heads * g.gdn_dim;
    int rc;
    invalidate_prep(s);
    ZG_HIP(zg::embed(m->embd->dw, tokens, s->x, B, s->d_status, st));
    for (size_t i = 0; i < m->layers.size(); ++i) {
        LayerW& L = m->layers[i];
        const int slot = s->layer_slot[i];
        if (!L.full) {
            if ((rc = project(s, L.qkv, s->x, L.attn_norm, s->y0, B, st))) return rc;
            if ((rc = project(s, L.gate, s->x, L.attn_norm, s->y1, B, st))) return rc;
            if ((rc = project(s, L.alpha, s->x, L.attn_norm, s->y2, B, st))) return rc;
            if ((rc = project(s, L.beta, s->x, L.attn_norm, s->y3, B, st))) return rc;
            ZG_HIP(zg::gdn_conv(s->y0, L.conv_w, s->conv[slot], s->mixed, 3 * W, B, 1, 3 * W, 3 * W * 3, 3 * W, st));
            ZG_HIP(zg::gdn_recurrent(true, s->mixed, s->mixed + W, s->mixed + 2 * W, 3 * W, s->y2, s->y3, g.gdn_heads,
                                     L.ssm_dt, L.ssm_a, g.eps, 1.0f / sqrtf((float)g.gdn_dim), nullptr, s->rec[slot],
                                     s->core, W, g.gdn_heads, g.gdn_dim, B, st));
            // grouped RMS over heads with ssm_norm, then normalized * silu(z)
            ZG_HIP(zg::rms_groups(s->core, L.ssm_norm, g.gdn_dim, B * g.gdn_heads, g.eps, s->gated, st));
            ZG_HIP(zg::silu(s->y1, s->gated, B * W, s->gated, st));
            if ((rc = project(s, L.ssm_out, s->gated, nullptr, s->out, B, st))) return rc;
        } else {
            if ((rc = project(s, L.wq, s->x, L.attn_norm, s->y0, B, st))) return rc;
            if ((rc = project(s, L.wk, s->x, L.attn_norm, s->y1, B, st))) return rc;
            if ((rc = project(s, L.wv, s->x, L.attn_norm, s->y2, B, st))) return rc;
            zg::AttnArgs a;
            a.B = (int)B;
            a.nq = (int)g.q_heads;
            a.nkv = (int)g.kv_heads;
            a.d = (int)g.head_dim;
            a.rotate = 64;
            a.tmax = (int)s->max_ctx;
            a.kv_bf16 = s->kv_bf16;
            a.do_prep = 1;
            a.qproj = s->y0;
            a.q_stride = 2 * (size_t)g.q_heads * g.head_dim;  // compact GEMV output of attn_q
            a.kproj = s->y1;
            a.vproj = s->y2;
            a.kv_stride = kvw(g);
            a.qnorm = L.q_norm;
            a.knorm = L.k_norm;
            a.pos = s->d_pos;
            a.ntok = s->d_ntok;
            a.theta_scale = powf(10000000.0f, -2.0f / 64.0f);
            a.eps = g.eps;
            a.scale = 1.0f / sqrtf((float)g.head_dim);
            a.qr = s->qr;
            a.qr_stride = (size_t)g.q_heads * g.head_dim;
            a.kcache = s->kc[slot];
            a.vcache = s->vc[slot];
            a.cache_row_stride = s->max_ctx * kvw(g);
            a.scores = s->scores;
            a.probs = s->probs;
            a.score_stride = (size_t)g.q_heads * s->max_ctx;
            int maxpos = 0;
            for (size_t b = 0; b < B; ++b) maxpos = std::max(maxpos, s->pos[b] + 1);
            a.tmax = maxpos;
            a.gate = s->y0;
            a.gate_stride = 2 * (size_t)g.q_heads * g.head_dim;
            a.out = s->gated;
            a.out_stride = (size_t)g.q_heads * g.head_dim;
            ZG_HIP(zg::attention(a, st));
            if ((rc = project(s, L.wo, s->gated, nullptr, s->out, B, st))) return rc;
        }
        ZG_HIP(zg::residual_add(s->x, s->out, B * H, s->d_status, st));
        if ((rc = project(s, L.ffn_gate, s->x, L.post_norm, s->y0, B, st))) return rc;
        if ((rc = project(s, L.ffn_up, s->x, L.post_norm, s->y1, B, st))) return rc;
        ZG_HIP(zg::silu(s->y0, s->y1, B * F, s->gated, st));
        if ((rc = project(s, L.ffn_down, s->gated, nullptr, s->out, B, st))) return rc;
        ZG_HIP(zg::residual_add(s->x, s->out, B * H, s->d_status, st));
    }
    if (logits || greedy) {
        if ((rc = project(s, m->embd, s->x, m->out_norm, logits ? logits : s->logits, B, st))) return rc;
        if (greedy) ZG_HIP(zg::argmax(logits ? logits : s->logits, g.vocab, B, greedy, s->d_status, st));
    }
    return ZG_COMPLETED;
}

int read_status(zg_session* s, hipStream_t st) {
    zg_ctx* ctx = s->m->ctx;
    int status = 0;
    ZG_HIP(hipMemcpyAsync(&status, s->d_status, sizeof(int), hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (status) {
        ZG_HIP(hipMemsetAsync(s->d_status, 0, sizeof(int), st));
        ZG_HIP(hipStreamSynchronize(st));
        s->poisoned = true;
        if (status & 2) return fail(ctx, ZG_E_MALFORMED, "decode step contains an out-of-vocabulary token id");
        if (status & 1) return fail(ctx, ZG_E_STATE, "nonfinite layer computation");
        return fail(ctx, ZG_E_STATE, "decoder produced nonfinite logits");
    }
    return ZG_COMPLETED;
}

// Device positions follow the host copy: steps advance both (a one-wave
// kernel on the stream, so device-driven decode loops never wait on the
// host); reset, import and random fill mark them dirty and the next step
// uploads them once.
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
    // pageable source: make the copy complete before the vectors go away
    ZG_HIP(hipStreamSynchronize(st));
    s->pos_dirty = false;
    return ZG_COMPLETED;
}

int advance(zg_session* s, size_t rows, hipStream_t st) {
    zg_ctx* ctx = s->m->ctx;
    ZG_HIP(zg::advance_positions(s->d_pos, s->d_ntok, rows, st));
    for (size_t b = 0; b < rows; ++b) s->pos[b] += 1;
    return ZG_COMPLETED;
}

int check_rows(zg_session* s, size_t rows) {
    zg_ctx* ctx = s->m->ctx;
    if (s->poisoned) return fail(ctx, ZG_E_STATE, "session poisoned by a failed step: reset or import state");
    if (rows == 0 || rows > s->max_batch) return fail(ctx, ZG_E_LIMIT, "row count exceeds the session batch");
    for (size_t b = 0; b < rows; ++b)
        if ((size_t)s->pos[b] >= s->max_ctx) return fail(ctx, ZG_E_LIMIT, "model context capacity exhausted");
    return ZG_COMPLETED;
}

}  // namespace

extern "C" {

int zg_model_load(zg_ctx* ctx, uint64_t source_id, const zg_geometry* g, const zg_tensor_desc* tensors, size_t n,
                  zg_model** out) {
    if (!ctx || !g || !tensors || !out) return fail(ctx, ZG_E_MALFORMED, "invalid model load arguments");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    *out = nullptr;
    if (source_id == 0) return fail(ctx, ZG_E_MALFORMED, "unbound source identity cannot own a resident model");
    if (g->layers == 0 || g->layers > 4096 || g->full_attention_interval == 0 || g->gdn_dim != 128 ||
        g->head_dim != 256 || g->q_heads == 0 || g->q_heads > 8 || g->kv_heads == 0 || g->q_heads % g->kv_heads ||
        g->q_heads / g->kv_heads > 4 || g->gdn_heads == 0 || g->gdn_heads > 64 || !(g->eps > 0.0f) ||
        g->max_context == 0 || g->hidden % 256 || g->ffn % 256)
        return fail(ctx, ZG_E_UNSUPPORTED, "model geometry outside the resident decode path (gdn_dim 128, head_dim 256)");
    auto m = new zg_model();
    m->ctx = ctx;
    m->source = source_id;
    m->g = *g;
    const uint64_t H = g->hidden, F = g->ffn, V = g->vocab, W = (uint64_t)g->gdn_heads * g->gdn_dim;
    const uint64_t QD = (uint64_t)g->q_heads * g->head_dim, KD = (uint64_t)g->kv_heads * g->head_dim;
    int rc = load_matrix(m, tensors, n, "token_embd.weight", H, V, &m->embd);
    if (!rc) rc = load_vector(m, tensors, n, "output_norm.weight", H, &m->out_norm);
    m->layers.resize(g->layers);
    for (unsigned i = 0; i < g->layers && !rc; ++i) {
        LayerW& L = m->layers[i];
        // config.rs:146-167: full attention where (i + 1) % interval == 0
        L.full = ((i + 1) % g->full_attention_interval) == 0;
        rc = load_vector(m, tensors, n, lname(i, "attn_norm.weight"), H, &L.attn_norm);
        if (!rc) rc = load_vector(m, tensors, n, lname(i, "post_attention_norm.weight"), H, &L.post_norm);
        if (!rc) rc = load_matrix(m, tensors, n, lname(i, "ffn_gate.weight"), H, F, &L.ffn_gate);
        if (!rc) rc = load_matrix(m, tensors, n, lname(i, "ffn_up.weight"), H, F, &L.ffn_up);
        if (!rc) rc = load_matrix(m, tensors, n, lname(i, "ffn_down.weight"), F, H, &L.ffn_down);
        if (rc) break;
        if (L.full) {
            rc = load_matrix(m, tensors, n, lname(i, "attn_q.weight"), H, 2 * QD, &L.wq);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "attn_k.weight"), H, KD, &L.wk);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "attn_v.weight"), H, KD, &L.wv);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "attn_output.weight"), QD, H, &L.wo);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "attn_q_norm.weight"), g->head_dim, &L.q_norm);
            if (!rc) rc = load_vector(m, tensors, n, lname(i, "attn_k_norm.weight"), g->head_dim, &L.k_norm);
            m->n_attn++;
        } else {
            rc = load_matrix(m, tensors, n, lname(i, "attn_qkv.weight"), H, 3 * W, &L.qkv);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "attn_gate.weight"), H, W, &L.gate);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "ssm_alpha.weight"), H, g->gdn_heads, &L.alpha);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "ssm_beta.weight"), H, g->gdn_heads, &L.beta);
            if (!rc) rc = load_matrix(m, tensors, n, lname(i, "ssm_out.weight"), W, H, &L.ssm_out);
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
    (void)hipStreamSynchronize(ctx->stream);
    for (void* p : m->vecs) (void)hipFree(p);
    zg_source_release(ctx, m->source);
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
    auto s = new zg_session();
    s->m = m;
    s->max_batch = max_batch;
    s->max_ctx = max_context;
    s->kv_bf16 = kv_dtype == ZG_BF16;
    s->pos.assign(max_batch, 0);
    const size_t B = max_batch, H = g.hidden, F = g.ffn, V = g.vocab, W = (size_t)g.gdn_heads * g.gdn_dim;
    const size_t QD = (size_t)g.q_heads * g.head_dim;
    s->y0w = std::max({3 * W, 2 * QD, F});
    s->y1w = std::max({W, F, kvw(g)});
    s->y2w = std::max<size_t>(g.gdn_heads, kvw(g));
    s->gatedw = std::max({W, F, QD});
    size_t prep = 0;
    for (size_t K : {H, F, W, QD}) prep = std::max(prep, zg::prepared_bytes(ZG_Q4_K, B, K));
    for (size_t K : {H, F, W, QD}) prep = std::max(prep, zg::prepared_bytes(ZG_Q8_0, B, K));
    for (size_t K : {H, F, W, QD}) prep = std::max(prep, zg::prepared_bytes(ZG_F32, B, K));
    s->prep_bytes = prep;
    int rc = 0;
    auto A = [&](void** p, size_t bytes) {
        if (!rc) rc = dalloc(s, p, bytes);
    };
    A((void**)&s->d_pos, B * 4);
    A((void**)&s->d_ntok, B * 4);
    A((void**)&s->d_status, 4);
    A((void**)&s->d_tokens, B * 4);
    A((void**)&s->d_greedy, B * 4);
    A((void**)&s->x, B * H * 4);
    A((void**)&s->y0, B * s->y0w * 4);
    A((void**)&s->y1, B * s->y1w * 4);
    A((void**)&s->y2, B * s->y2w * 4);
    A((void**)&s->y3, B * g.gdn_heads * 4);
    A((void**)&s->mixed, B * 3 * W * 4);
    A((void**)&s->core, B * W * 4);
    A((void**)&s->gated, B * s->gatedw * 4);
    A((void**)&s->out, B * H * 4);
    A((void**)&s->logits, B * V * 4);
    A((void**)&s->qr, B * QD * 4);
    A((void**)&s->scores, B * g.q_heads * max_context * 4);
    A((void**)&s->probs, B * g.q_heads * max_context * 4);
    A(&s->prep, prep);
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
            s->layer_slot[i] = (int)s->conv.size();
            float *c = nullptr, *r = nullptr;
            A((void**)&c, B * conv_floats(g) * 4);
            A((void**)&r, B * rec_floats(g) * 4);
            s->conv.push_back(c);
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
    (void)hipStreamSynchronize(ctx->stream);
    for (void* p : s->allocs) (void)hipFree(p);
    delete s;
}

int zg_session_reset(zg_session* s) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    const zg_geometry& g = s->m->g;
    const size_t B = s->max_batch;
    for (float* c : s->conv) ZG_HIP(hipMemsetAsync(c, 0, B * conv_floats(g) * 4, ctx->stream));
    for (float* r : s->rec) ZG_HIP(hipMemsetAsync(r, 0, B * rec_floats(g) * 4, ctx->stream));
    const size_t kvb = B * s->max_ctx * kvw(g) * (s->kv_bf16 ? 2 : 4);
    for (size_t i = 0; i < s->kc.size(); ++i) {
        ZG_HIP(hipMemsetAsync(s->kc[i], 0, kvb, ctx->stream));
        ZG_HIP(hipMemsetAsync(s->vc[i], 0, kvb, ctx->stream));
    }
    ZG_HIP(hipMemsetAsync(s->d_status, 0, 4, ctx->stream));
    ZG_HIP(hipStreamSynchronize(ctx->stream));
    std::fill(s->pos.begin(), s->pos.end(), 0);
    s->pos_dirty = true;
    s->poisoned = false;
    return ZG_COMPLETED;
}

int zg_session_position(const zg_session* s, size_t row) {
    if (!s || row >= s->max_batch) return -1;
    return s->pos[row];
}

int zg_decode_step(zg_session* s, size_t rows, const uint32_t* tokens, float* logits, uint32_t* greedy) {
    if (!s || !tokens) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = check_rows(s, rows);
    if (rc) return rc;
    for (size_t b = 0; b < rows; ++b)
        if (tokens[b] >= s->m->g.vocab) return fail(ctx, ZG_E_MALFORMED, "decode step contains an out-of-vocabulary token id");
    hipStream_t st = ctx->stream;
    if ((rc = sync_positions(s, st))) return rc;
    ZG_HIP(hipMemcpyAsync(s->d_tokens, tokens, rows * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipStreamSynchronize(st));
    const bool want = logits || greedy;
    if ((rc = step(s, rows, s->d_tokens, want ? s->logits : nullptr, want ? s->d_greedy : nullptr, st))) {
        s->poisoned = true;
        return rc;
    }
    if ((rc = advance(s, rows, st))) return rc;
    if ((rc = read_status(s, st))) return rc;
    if (logits) ZG_HIP(hipMemcpyAsync(logits, s->logits, rows * s->m->g.vocab * 4, hipMemcpyDeviceToHost, st));
    if (greedy) ZG_HIP(hipMemcpyAsync(greedy, s->d_greedy, rows * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

int zg_prefill(zg_session* s, size_t rows, size_t n, const uint32_t* tokens, float* logits) {
    if (!s || !tokens || n == 0) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    std::vector<uint32_t> col(rows);
    for (size_t t = 0; t < n; ++t) {
        for (size_t b = 0; b < rows; ++b) col[b] = tokens[b * n + t];
        int rc = zg_decode_step(s, rows, col.data(), t + 1 == n ? logits : nullptr, nullptr);
        if (rc) return rc;
    }
    return ZG_COMPLETED;
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
    if ((rc = sync_positions(s, st))) return rc;
    if ((rc = step(s, rows, d_tokens, d_logits ? d_logits : (d_greedy ? s->logits : nullptr), d_greedy, st))) {
        s->poisoned = true;
        return rc;
    }
    return advance(s, rows, st);
}

int zg_session_check(zg_session* s, void* stream) {
    if (!s) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    return read_status(s, stream ? (hipStream_t)stream : ctx->stream);
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
    if (row >= s->max_batch || n != zg_state_floats(s, row)) return fail(ctx, ZG_E_MALFORMED, "state length mismatch");
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    const size_t T = (size_t)s->pos[row], kw = kvw(g);
    int rc = ensure(ctx, ctx->scratch, std::max<size_t>(T * kw * 4, 256));
    if (rc) return rc;
    size_t at = 0;
    for (size_t i = 0; i < s->m->layers.size(); ++i) {
        const int slot = s->layer_slot[i];
        if (!s->m->layers[i].full) {
            ZG_HIP(hipMemcpyAsync(out + at, s->conv[slot] + row * conv_floats(g), conv_floats(g) * 4, hipMemcpyDeviceToHost, st));
            at += conv_floats(g);
            ZG_HIP(hipMemcpyAsync(out + at, s->rec[slot] + row * rec_floats(g), rec_floats(g) * 4, hipMemcpyDeviceToHost, st));
            at += rec_floats(g);
        } else {
            for (void* cache : {s->kc[slot], s->vc[slot]}) {
                if (T) {
                    if (s->kv_bf16) {
                        ZG_HIP(zg::convert_kv((const uint16_t*)cache + row * s->max_ctx * kw, ctx->scratch.ptr, T * kw, true, st));
                        ZG_HIP(hipMemcpyAsync(out + at, ctx->scratch.ptr, T * kw * 4, hipMemcpyDeviceToHost, st));
                        ZG_HIP(hipStreamSynchronize(st));
                    } else {
                        ZG_HIP(hipMemcpyAsync(out + at, (const float*)cache + row * s->max_ctx * kw, T * kw * 4,
                                              hipMemcpyDeviceToHost, st));
                    }
                }
                at += T * kw;
            }
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

int zg_state_import(zg_session* s, size_t row, const float* in, size_t n, int position) {
    if (!s || !in) return ZG_E_MALFORMED;
    zg_ctx* ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (row >= s->max_batch || position < 0 || (size_t)position > s->max_ctx)
        return fail(ctx, ZG_E_MALFORMED, "invalid state import row or position");
    const int saved = s->pos[row];
    s->pos[row] = position;
    if (n != zg_state_floats(s, row) || !all_finite(in, n)) {
        s->pos[row] = saved;
        return fail(ctx, ZG_E_MALFORMED, "state import length mismatch or nonfinite state");
    }
    const zg_geometry& g = s->m->g;
    hipStream_t st = ctx->stream;
    const size_t T = (size_t)position, kw = kvw(g);
    int rc = ensure(ctx, ctx->scratch, std::max<size_t>(T * kw * 4, 256));
    if (rc) return rc;
    size_t at = 0;
    for (size_t i = 0; i < s->m->layers.size(); ++i) {
        const int slot = s->layer_slot[i];
        if (!s->m->layers[i].full) {
            ZG_HIP(hipMemcpyAsync(s->conv[slot] + row * conv_floats(g), in + at, conv_floats(g) * 4, hipMemcpyHostToDevice, st));
            at += conv_floats(g);
            ZG_HIP(hipMemcpyAsync(s->rec[slot] + row * rec_floats(g), in + at, rec_floats(g) * 4, hipMemcpyHostToDevice, st));
            at += rec_floats(g);
        } else {
            for (void* cache : {s->kc[slot], s->vc[slot]}) {
                if (T) {
                    if (s->kv_bf16) {
                        ZG_HIP(hipMemcpyAsync(ctx->scratch.ptr, in + at, T * kw * 4, hipMemcpyHostToDevice, st));
                        ZG_HIP(zg::convert_kv(ctx->scratch.ptr, (uint16_t*)cache + row * s->max_ctx * kw, T * kw, false, st));
                        ZG_HIP(hipStreamSynchronize(st));
                    } else {
                        ZG_HIP(hipMemcpyAsync((float*)cache + row * s->max_ctx * kw, in + at, T * kw * 4,
                                              hipMemcpyHostToDevice, st));
                    }
                }
                at += T * kw;
            }
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    s->pos_dirty = true;
    s->poisoned = false;
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
    uint64_t k = seed * 0x9e3779b97f4a7c15ull;
    const size_t kw = kvw(g);
    for (size_t i = 0; i < s->conv.size(); ++i) {
        ZG_HIP(zg::fill_normal(s->conv[i], rows * conv_floats(g), false, ++k, 0.5f, st));
        ZG_HIP(zg::fill_normal(s->rec[i], rows * rec_floats(g), false, ++k, 0.02f, st));
    }
    for (size_t i = 0; i < s->kc.size(); ++i) {
        for (size_t b = 0; b < rows; ++b) {
            const size_t off = b * s->max_ctx * kw * (s->kv_bf16 ? 2 : 4);
            ZG_HIP(zg::fill_normal((char*)s->kc[i] + off, prefix * kw, s->kv_bf16, ++k, 1.0f, st));
            ZG_HIP(zg::fill_normal((char*)s->vc[i] + off, prefix * kw, s->kv_bf16, ++k, 1.0f, st));
        }
    }
    ZG_HIP(hipStreamSynchronize(st));
    for (size_t b = 0; b < rows; ++b) s->pos[b] = (int)prefix;
    s->pos_dirty = true;
    s->poisoned = false;
    return ZG_COMPLETED;
}

// ----------------------------------------------------- boundary-A regions

int zg_gdn_conv(zg_ctx* ctx, const float* activation, const float* weights, const float* history, size_t channels,
                float* raw_out, float* history_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!activation || !weights || !history || !raw_out || !history_out || channels == 0 ||
        !all_finite(activation, channels) || !all_finite(weights, channels * 4) || !all_finite(history, channels * 3))
        return fail(ctx, ZG_E_MALFORMED, "GDN causal convolution source geometry/nonfinite input");
    const size_t oa = 0, ow = align256(channels * 4), oh = ow + align256(channels * 16), oo = oh + align256(channels * 12);
    int rc = ensure(ctx, ctx->scratch, oo + align256(channels * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    ZG_HIP(hipMemcpyAsync(b + oa, activation, channels * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ow, weights, channels * 16, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oh, history, channels * 12, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::gdn_conv((const float*)(b + oa), (const float*)(b + ow), (float*)(b + oh), (float*)(b + oo), channels, 1,
                        0, 0, 0, 0, st));
    ZG_HIP(hipMemcpyAsync(raw_out, b + oo, channels * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(history_out, b + oh, channels * 12, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(raw_out, channels) || !all_finite(history_out, channels * 3))
        return fail(ctx, ZG_E_STATE, "physical GDN convolution returned incomplete/nonfinite source state");
    return ZG_COMPLETED;
}

int zg_gdn_coefficients(zg_ctx* ctx, const float* alpha, const float* beta, const float* dt, const float* a,
                        size_t heads, float scale, float* gain_out, float* beta_out, float* softplus_out,
                        float* gate_raw_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!alpha || !beta || !dt || !a || !gain_out || !beta_out || !softplus_out || !gate_raw_out || heads == 0 ||
        !all_finite(alpha, heads) || !all_finite(beta, heads) || !all_finite(dt, heads) || !all_finite(a, heads) ||
        !std::isfinite(scale) || scale <= 0.0f)
        return fail(ctx, ZG_E_MALFORMED, "invalid source GDN coefficient inputs");
    const size_t stride = align256(heads * 4);
    int rc = ensure(ctx, ctx->scratch, 8 * stride);
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const float* ins[4] = {alpha, beta, dt, a};
    for (int i = 0; i < 4; ++i) ZG_HIP(hipMemcpyAsync(b + i * stride, ins[i], heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::gdn_coefficients((const float*)b, (const float*)(b + stride), (const float*)(b + 2 * stride),
                                (const float*)(b + 3 * stride), heads, (float*)(b + 4 * stride), (float*)(b + 5 * stride),
                                (float*)(b + 6 * stride), (float*)(b + 7 * stride), st));
    float* outs[4] = {gain_out, beta_out, softplus_out, gate_raw_out};
    for (int i = 0; i < 4; ++i)
        ZG_HIP(hipMemcpyAsync(outs[i], b + (4 + i) * stride, heads * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    for (int i = 0; i < 4; ++i)
        if (!all_finite(outs[i], heads)) return fail(ctx, ZG_E_STATE, "incomplete/nonfinite source GDN coefficients");
    return ZG_COMPLETED;
}

int zg_gdn_recurrent(zg_ctx* ctx, size_t width, size_t heads, const float* q, const float* k, const float* v,
                     const float* coefficients, const float* state, float* output, float* state_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!q || !k || !v || !coefficients || !state || !output || !state_out || width == 0 || heads == 0)
        return fail(ctx, ZG_E_MALFORMED, "invalid source GDN recurrent geometry or FP32 inputs");
    const size_t n = heads * width, ns = n * width;
    if (!all_finite(q, n) || !all_finite(k, n) || !all_finite(v, n) || !all_finite(state, ns) ||
        !all_finite(coefficients, heads * 3))
        return fail(ctx, ZG_E_MALFORMED, "invalid source GDN recurrent geometry or FP32 inputs");
    if (width != 128) return fail(ctx, ZG_UNSUPPORTED, "GDN recurrence offered for head width 128");
    std::vector<float> gain(heads), beta(heads), scale(heads);
    for (size_t h = 0; h < heads; ++h) {
        gain[h] = coefficients[3 * h];
        beta[h] = coefficients[3 * h + 1];
        scale[h] = coefficients[3 * h + 2];
    }
    const size_t oq = 0, ok = align256(n * 4), ov = ok + align256(n * 4), oc = ov + align256(n * 4),
                 os = oc + 3 * align256(heads * 4), oo = os + align256(ns * 4);
    int rc = ensure(ctx, ctx->scratch, oo + align256(n * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    ZG_HIP(hipMemcpyAsync(b + oq, q, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ok, k, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ov, v, n * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oc, gain.data(), heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oc + align256(heads * 4), beta.data(), heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + oc + 2 * align256(heads * 4), scale.data(), heads * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + os, state, ns * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::gdn_recurrent(false, (const float*)(b + oq), (const float*)(b + ok), (const float*)(b + ov), 0,
                             (const float*)(b + oc), (const float*)(b + oc + align256(heads * 4)), 0, nullptr, nullptr,
                             0.0f, 0.0f, (const float*)(b + oc + 2 * align256(heads * 4)), (float*)(b + os),
                             (float*)(b + oo), 0, heads, width, 1, st));
    ZG_HIP(hipMemcpyAsync(output, b + oo, n * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(state_out, b + os, ns * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(output, n) || !all_finite(state_out, ns))
        return fail(ctx, ZG_E_STATE, "incomplete/nonfinite GDN recurrent proposal");
    return ZG_COMPLETED;
}

int zg_rope_kv(zg_ctx* ctx, const float* query, const float* key, const float* value, size_t head_width,
               size_t query_heads, size_t kv_heads, size_t rotate, size_t position, float theta_scale, float* query_out,
               float* key_out, float* value_out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!query || !key || !value || !query_out || !key_out || !value_out || head_width == 0 || query_heads == 0 ||
        kv_heads == 0 || query_heads % kv_heads || rotate == 0 || rotate > head_width || rotate % 2 ||
        position > 2147483647u || !std::isfinite(theta_scale) || theta_scale <= 0.0f || theta_scale > 1.0f ||
        !all_finite(query, query_heads * head_width) || !all_finite(key, kv_heads * head_width) ||
        !all_finite(value, kv_heads * head_width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source RoPE/KV geometry or FP32 input");
    if (head_width > 256 || rotate > 128) return fail(ctx, ZG_UNSUPPORTED, "RoPE offered for head width <= 256");
    const size_t nq = query_heads * head_width, nk = kv_heads * head_width;
    // The prep kernel reads q from a [q | gate] layout (stride 2*head_width);
    // lay the query out that way.
    std::vector<float> qpad(2 * nq, 0.0f);
    for (size_t h = 0; h < query_heads; ++h)
        std::memcpy(qpad.data() + h * 2 * head_width, query + h * head_width, head_width * 4);
    const size_t oq = 0, ok = align256(2 * nq * 4), ov = ok + align256(nk * 4), op = ov + align256(nk * 4),
                 oqr = op + 256, oko = oqr + align256(nq * 4), ovo = oko + align256(nk * 4);
    int rc = ensure(ctx, ctx->scratch, ovo + align256(nk * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const int p = (int)position;
    ZG_HIP(hipMemcpyAsync(b + oq, qpad.data(), 2 * nq * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ok, key, nk * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + ov, value, nk * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + op, &p, 4, hipMemcpyHostToDevice, st));
    zg::AttnArgs a;
    a.B = 1;
    a.nq = (int)query_heads;
    a.nkv = (int)kv_heads;
    a.d = (int)head_width;
    a.rotate = (int)rotate;
    a.do_prep = 1;
    a.prep_only = 1;
    a.norm = 0;
    a.qproj = (const float*)(b + oq);
    a.q_stride = 2 * nq;
    a.kproj = (const float*)(b + ok);
    a.vproj = (const float*)(b + ov);
    a.kv_stride = nk;
    a.pos = (const int*)(b + op);
    a.theta_scale = theta_scale;
    a.qr = (float*)(b + oqr);
    a.qr_stride = nq;
    a.kout = (float*)(b + oko);
    a.vout = (float*)(b + ovo);
    ZG_HIP(zg::rope_prep(a, st));
    ZG_HIP(hipMemcpyAsync(query_out, b + oqr, nq * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(key_out, b + oko, nk * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipMemcpyAsync(value_out, b + ovo, nk * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    if (!all_finite(query_out, nq) || !all_finite(key_out, nk))
        return fail(ctx, ZG_E_STATE, "incomplete/nonfinite RoPE proposal");
    return ZG_COMPLETED;
}

// QK + softmax + PV regions share one driver over f32 host keys/values.
static int attention_region(zg_ctx* ctx, const float* query, const float* keys, const float* values, size_t tokens,
                            size_t head_width, size_t query_heads, size_t kv_heads, float scale, float* dots,
                            float* scores, float* probs, float* out) {
    const size_t nq = query_heads * head_width, kw = kv_heads * head_width, ns = query_heads * tokens;
    const size_t oq = 0, ok = align256(nq * 4), ov = ok + align256(tokens * kw * 4), on = ov + align256(values ? tokens * kw * 4 : 4),
                 od = on + 256, osc = od + align256(ns * 4), opr = osc + align256(ns * 4),
                 oo = opr + align256(ns * 4);
    int rc = ensure(ctx, ctx->scratch, oo + align256(nq * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const int T = (int)tokens;
    ZG_HIP(hipMemcpyAsync(b + oq, query, nq * 4, hipMemcpyHostToDevice, st));
    if (keys) ZG_HIP(hipMemcpyAsync(b + ok, keys, tokens * kw * 4, hipMemcpyHostToDevice, st));
    if (values) ZG_HIP(hipMemcpyAsync(b + ov, values, tokens * kw * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + on, &T, 4, hipMemcpyHostToDevice, st));
    if (probs && !keys) ZG_HIP(hipMemcpyAsync(b + opr, probs, ns * 4, hipMemcpyHostToDevice, st));
    zg::AttnArgs a;
    a.B = 1;
    a.nq = (int)query_heads;
    a.nkv = (int)kv_heads;
    a.d = (int)head_width;
    a.tmax = T;
    a.kv_bf16 = 0;
    a.qr = (float*)(b + oq);
    a.qr_stride = nq;
    a.kcache = b + ok;
    a.vcache = b + ov;
    a.cache_row_stride = tokens * kw;
    a.ntok = (const int*)(b + on);
    a.scale = scale;
    a.dots = (float*)(b + od);
    a.scores = (float*)(b + osc);
    a.probs = (float*)(b + opr);
    a.score_stride = ns;
    a.out = out ? (float*)(b + oo) : nullptr;
    a.out_stride = nq;
    ZG_HIP(zg::attention_parts(a, keys != nullptr, keys != nullptr, out != nullptr, st));
    if (dots) ZG_HIP(hipMemcpyAsync(dots, b + od, ns * 4, hipMemcpyDeviceToHost, st));
    if (scores) ZG_HIP(hipMemcpyAsync(scores, b + osc, ns * 4, hipMemcpyDeviceToHost, st));
    if (probs && keys) ZG_HIP(hipMemcpyAsync(probs, b + opr, ns * 4, hipMemcpyDeviceToHost, st));
    if (out) ZG_HIP(hipMemcpyAsync(out, b + oo, nq * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    return ZG_COMPLETED;
}

int zg_attention_qk(zg_ctx* ctx, const float* query, const float* keys, size_t tokens, size_t head_width,
                    size_t query_heads, size_t kv_heads, float scale, float* dots, float* scores) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!query || !keys || !dots || !scores || head_width == 0 || query_heads == 0 || kv_heads == 0 ||
        query_heads % kv_heads || tokens == 0 || !std::isfinite(scale) || scale <= 0.0f ||
        !all_finite(query, query_heads * head_width) || !all_finite(keys, tokens * kv_heads * head_width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source attention QK region");
    if (head_width != 256 || query_heads / kv_heads > 4)
        return fail(ctx, ZG_UNSUPPORTED, "attention offered for head width 256, GQA group <= 4");
    const size_t ns = query_heads * tokens;
    std::vector<float> probs(ns);
    int rc = attention_region(ctx, query, keys, nullptr, tokens, head_width, query_heads, kv_heads, scale, dots, scores,
                              probs.data(), nullptr);
    if (rc) return rc;
    for (size_t i = 0; i < ns; ++i)
        if (!std::isfinite(dots[i]) || scores[i] != dots[i] * scale)
            return fail(ctx, ZG_E_STATE, "incomplete/nonfinite QK proposal or wrong source scale");
    return ZG_COMPLETED;
}

int zg_attention_softmax(zg_ctx* ctx, const float* scores, size_t heads, size_t width, float* probabilities) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!scores || !probabilities || heads == 0 || width == 0 || !all_finite(scores, heads * width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source attention softmax region");
    const size_t ns = heads * width;
    const size_t osc = 0, on = align256(ns * 4), opr = on + 256;
    int rc = ensure(ctx, ctx->scratch, opr + align256(ns * 4));
    if (rc) return rc;
    char* b = (char*)ctx->scratch.ptr;
    hipStream_t st = ctx->stream;
    const int T = (int)width;
    ZG_HIP(hipMemcpyAsync(b + osc, scores, ns * 4, hipMemcpyHostToDevice, st));
    ZG_HIP(hipMemcpyAsync(b + on, &T, 4, hipMemcpyHostToDevice, st));
    ZG_HIP(zg::softmax_rows((const float*)(b + osc), ns, (const int*)(b + on), (float*)(b + opr), heads, 1, st));
    ZG_HIP(hipMemcpyAsync(probabilities, b + opr, ns * 4, hipMemcpyDeviceToHost, st));
    ZG_HIP(hipStreamSynchronize(st));
    for (size_t i = 0; i < ns; ++i)
        if (!std::isfinite(probabilities[i]) || probabilities[i] < 0.0f || probabilities[i] > 1.0f)
            return fail(ctx, ZG_E_STATE, "invalid source softmax probability");
    return ZG_COMPLETED;
}

int zg_attention_value(zg_ctx* ctx, const float* probabilities, const float* values, size_t tokens, size_t head_width,
                       size_t query_heads, size_t kv_heads, float* out) {
    if (!ctx) return ZG_E_MALFORMED;
    std::lock_guard<std::recursive_mutex> g(ctx->mu);
    (void)hipSetDevice(ctx->device);
    if (!probabilities || !values || !out || head_width == 0 || query_heads == 0 || kv_heads == 0 ||
        query_heads % kv_heads || tokens == 0 || !all_finite(values, tokens * kv_heads * head_width))
        return fail(ctx, ZG_E_MALFORMED, "invalid source attention value region");
    for (size_t i = 0; i < query_heads * tokens; ++i)
        if (!std::isfinite(probabilities[i]) || std::signbit(probabilities[i]) || probabilities[i] > 1.0f)
            return fail(ctx, ZG_E_MALFORMED, "invalid source attention value region");
    if (head_width != 256 || query_heads / kv_heads > 4)
        return fail(ctx, ZG_UNSUPPORTED, "attention offered for head width 256, GQA group <= 4");
    std::vector<float> dummy(query_heads * head_width);
    int rc = attention_region(ctx, dummy.data(), nullptr, values, tokens, head_width, query_heads, kv_heads, 1.0f,
                              nullptr, nullptr, const_cast<float*>(probabilities), out);
    if (rc) return rc;
    if (!all_finite(out, query_heads * head_width))
        return fail(ctx, ZG_E_STATE, "incomplete/nonfinite source attention value proposal");
    return ZG_COMPLETED;
}

}  // extern "C"
