"""Pins the oracle's whole-token forward (zgo_forward_token) with an
independent float64 restatement of the reference's schedule.

`forward64` below is written from model-qwen35/src/forward.rs:451-755 (the
layer order, the [q | gate] per-head split, the GQA head map h / group,
norm * silu(z) for the GDN output gate, sigmoid(gate) * attention),
lib.rs:1552-1577 (RoPE pairs (i, i + 32), angle = position * theta^i),
lib.rs:324-362 (softplus / sigmoid gates), the closed-form GDN update
S <- g S (I - beta k k^T) + beta v k^T, o = S q / sqrt(d), and the Q4_K
decode rule of artifacts/src/codecs/q4.rs:39-70.  It calls no oracle
function and keeps every value in float64, so it shares no rounding and no
code with the oracle; the oracle's f32 logits must match it to 1e-4
relative on F32- and Q4_K-weighted models over several positions.

Each plausible misreading is planted in the float64 forward and shown to
fail the same check: swapped [q | gate] halves, silu applied to the norm
instead of z, the GQA head map h % kv_heads, and RoPE on adjacent pairs.
"""
import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import gguf, qwen35

G = dict(hidden=256, layers=4, ffn=512, vocab=600, gdn_heads=2, gdn_dim=128, q_heads=4, kv_heads=2, head_dim=256,
         full_attention_interval=4, max_context=64, eps=1e-6)
TOL = 1e-4


def _f16(b):
    return np.ascontiguousarray(b).view(np.float16).astype(np.float64).reshape(-1)


def dequant(ty, data, rows, cols):
    """[rows, cols] float64 weights (GGML ne0 = cols)."""
    raw = np.ascontiguousarray(data, np.uint8)
    if ty == gguf.F32:
        return raw.view(np.float32).astype(np.float64).reshape(rows, cols)
    assert ty == gguf.Q4_K
    b = raw.reshape(-1, 144)
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    p = b[:, 4:16].astype(np.int64)
    v = b[:, 16:144]
    out = np.empty((b.shape[0], 256))
    for g in range(8):
        if g < 4:
            sc, mn = p[:, g] & 63, p[:, g + 4] & 63
        else:
            sc = (p[:, g + 4] & 15) | ((p[:, g - 4] >> 6) << 4)
            mn = (p[:, g + 4] >> 4) | ((p[:, g] >> 6) << 4)
        q = v[:, (g // 2) * 32:(g // 2) * 32 + 32]
        q = (q >> 4) if g % 2 else (q & 15)
        out[:, g * 32:(g + 1) * 32] = (d * sc)[:, None] * q - (dmin * mn)[:, None]
    return out.reshape(rows, cols)


def silu(x):
    return x / (1.0 + np.exp(-x))


def rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


class Forward64:
    def __init__(self, g, t, mistake=None):
        self.g, self.mistake = g, mistake
        self.W = {}
        for name, (ty, s0, s1, data) in t.items():
            if ty == gguf.F32 and s1 == 1 and not name.endswith("ssm_conv1d.weight"):
                self.W[name] = np.ascontiguousarray(data).view(np.float32).astype(np.float64)
            else:
                self.W[name] = dequant(ty, data, s1, s0)
        H, W = g["gdn_heads"], g["gdn_heads"] * g["gdn_dim"]
        kinds = qwen35.layer_kinds(g)
        self.conv = {i: np.zeros((3 * W, 3)) for i, k in enumerate(kinds) if k == "linear_attention"}
        self.S = {i: np.zeros((H, g["gdn_dim"], g["gdn_dim"])) for i, k in enumerate(kinds) if k == "linear_attention"}
        self.K = {i: [] for i, k in enumerate(kinds) if k == "full_attention"}
        self.V = {i: [] for i, k in enumerate(kinds) if k == "full_attention"}
        self.pos = 0

    def w(self, i, name):
        return self.W[f"blk.{i}.{name}"]

    def gdn(self, i, x):
        g = self.g
        H, d = g["gdn_heads"], g["gdn_dim"]
        W = H * d
        qkv = self.w(i, "attn_qkv.weight") @ x
        z = self.w(i, "attn_gate.weight") @ x
        alpha = self.w(i, "ssm_alpha.weight") @ x
        beta_p = self.w(i, "ssm_beta.weight") @ x
        taps = self.w(i, "ssm_conv1d.weight").reshape(3 * W, 4)  # [channel][tap], newest last
        hist = self.conv[i]
        raw = (hist * taps[:, :3]).sum(1) + qkv * taps[:, 3]
        self.conv[i] = np.concatenate([hist[:, 1:], qkv[:, None]], 1)
        mixed = silu(raw)
        q, k, v = mixed[:W].reshape(H, d), mixed[W:2 * W].reshape(H, d), mixed[2 * W:].reshape(H, d)
        q = q / np.sqrt((q * q).sum(1, keepdims=True) + g["eps"])
        k = k / np.sqrt((k * k).sum(1, keepdims=True) + g["eps"])
        a = self.w(i, "ssm_a")
        sp = np.log1p(np.exp(alpha + self.w(i, "ssm_dt.bias")))
        gain = np.exp(sp * a)
        beta = 1.0 / (1.0 + np.exp(-beta_p))
        out = np.empty((H, d))
        for h in range(H):
            S = self.S[i][h]  # [value][key]
            S = gain[h] * S @ (np.eye(d) - beta[h] * np.outer(k[h], k[h])) + beta[h] * np.outer(v[h], k[h])
            self.S[i][h] = S
            out[h] = S @ q[h] / np.sqrt(d)
        gamma = self.w(i, "ssm_norm.weight")
        normed = np.stack([rms(out[h], gamma, g["eps"]) for h in range(H)]).reshape(-1)
        gated = silu(normed) * z if self.mistake == "silu_on_norm" else normed * silu(z)
        return self.w(i, "ssm_out.weight") @ gated

    def rope(self, heads):
        g = self.g
        ts = 10_000_000.0 ** (-2.0 / 64.0)
        out = heads.copy()
        for r in range(heads.shape[0]):
            for i in range(32):
                ang = self.pos * ts ** i
                if self.mistake == "rope_adjacent":
                    a_i, b_i = 2 * i, 2 * i + 1
                else:
                    a_i, b_i = i, i + 32
                a, b = heads[r, a_i], heads[r, b_i]
                out[r, a_i] = a * np.cos(ang) - b * np.sin(ang)
                out[r, b_i] = a * np.sin(ang) + b * np.cos(ang)
        return out

    def attention(self, i, x):
        g = self.g
        nq, nkv, d = g["q_heads"], g["kv_heads"], g["head_dim"]
        qg = (self.w(i, "attn_q.weight") @ x).reshape(nq, 2, d)
        q, gate = (qg[:, 1], qg[:, 0]) if self.mistake == "swap_qgate" else (qg[:, 0], qg[:, 1])
        k = (self.w(i, "attn_k.weight") @ x).reshape(nkv, d)
        v = (self.w(i, "attn_v.weight") @ x).reshape(nkv, d)
        q = np.stack([rms(q[h], self.w(i, "attn_q_norm.weight"), g["eps"]) for h in range(nq)])
        k = np.stack([rms(k[h], self.w(i, "attn_k_norm.weight"), g["eps"]) for h in range(nkv)])
        q, k = self.rope(q), self.rope(k)
        self.K[i].append(k)
        self.V[i].append(v)
        Ks, Vs = np.stack(self.K[i]), np.stack(self.V[i])  # [T][kv][d]
        out = np.empty((nq, d))
        for h in range(nq):
            kv = h % nkv if self.mistake == "gqa_mod" else h // (nq // nkv)
            s = Ks[:, kv] @ q[h] / np.sqrt(d)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[h] = p @ Vs[:, kv]
        gated = (out * (1.0 / (1.0 + np.exp(-gate)))).reshape(-1)
        return self.w(i, "attn_output.weight") @ gated

    def forward(self, token):
        g = self.g
        x = self.W["token_embd.weight"][token].copy()
        for i, kind in enumerate(qwen35.layer_kinds(g)):
            h = rms(x, self.w(i, "attn_norm.weight"), g["eps"])
            x = x + (self.gdn(i, h) if kind == "linear_attention" else self.attention(i, h))
            h = rms(x, self.w(i, "post_attention_norm.weight"), g["eps"])
            act = (self.w(i, "ffn_up.weight") @ h) * silu(self.w(i, "ffn_gate.weight") @ h)
            x = x + self.w(i, "ffn_down.weight") @ act
        self.pos += 1
        return self.W["token_embd.weight"] @ rms(x, self.W["output_norm.weight"], g["eps"])


def _worst(kind, seed, mistake=None, steps=6):
    t = qwen35.synthetic_tensors(G, kind, seed=seed)
    ref = O.Model(G, t).session()
    f = Forward64(G, t, mistake)
    toks = np.random.default_rng(seed).integers(0, G["vocab"], steps)
    worst = 0.0
    for tok in toks:
        a, b = f.forward(int(tok)), ref.forward(int(tok)).astype(np.float64)
        worst = max(worst, float(np.max(np.abs(a - b)) / np.max(np.abs(b))))
    return worst


@pytest.mark.parametrize("kind", [gguf.F32, gguf.Q4_K])
def test_oracle_forward_matches_float64_restatement(kind):
    worst = _worst(kind, 70 + kind)
    print(f"kind={kind}: worst relative logit difference {worst:.2e}")
    assert worst <= TOL


@pytest.mark.parametrize("mistake", ["swap_qgate", "silu_on_norm", "gqa_mod", "rope_adjacent"])
def test_planted_mistakes_are_caught(mistake):
    worst = _worst(gguf.F32, 70 + gguf.F32, mistake)
    print(f"{mistake}: worst relative logit difference {worst:.2e}")
    assert worst > 100 * TOL
