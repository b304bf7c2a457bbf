"""Writes tests/golden/prefill_8192_oracle.npz: the CPU oracle's token-by-token
prefill (QwenDenseCpu::prefill_transaction, model-qwen35/src/lib.rs:
1119-1187, restated in oracle/zg_oracle.c) of an 8192-token prompt through
a 4-layer model of the 2B widths (3 GDN layers, 1 attention layer, bf16 KV
cache), with glibc's transcendentals as the reference's Rust f32 functions
use.  Stored: the last token's logits and greedy id, and a fixed subsample
of the exported state (reference domain order, lib.rs:112-150) -- per GDN
layer every 37th conv-history value and every 97th recurrent-state value,
the attention layer's keys and values of the last 8 positions in full and
every 1009th before them.  The prompt and weights come from seeded
generators (numpy PCG64), so tests/test_prefill_gpu.py rebuilds them.

    python tests/golden/make_prefill_8192.py      (about 15 minutes on 8 cores)
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

N_PROMPT = 8192
GEOMETRY = dict(hidden=2048, layers=4, ffn=6144, vocab=1000, gdn_heads=16, gdn_dim=128, q_heads=8, kv_heads=2,
                head_dim=256, full_attention_interval=4, max_context=N_PROMPT + 64, eps=1e-6)
WEIGHT_SEED, TOKEN_SEED = 88, 8192


def prompt():
    return np.random.default_rng(TOKEN_SEED).integers(0, GEOMETRY["vocab"], N_PROMPT).astype(np.uint32)


def state_index(g, n):
    """Indices of the stored state subsample in the export of a row at
    position n (per GDN layer conv [3W][3] then state [H][128][128]; the
    attention layer keys then values [n][kv_heads * head_dim])."""
    W = g["gdn_heads"] * g["gdn_dim"]
    conv, rec = 3 * W * 3, g["gdn_heads"] * g["gdn_dim"] ** 2
    kw = g["kv_heads"] * g["head_dim"]
    idx, at = [], 0
    for i in range(g["layers"]):
        if (i + 1) % g["full_attention_interval"] == 0:
            for _ in range(2):  # keys, values
                head = np.arange(0, (n - 8) * kw, 1009)
                tail = np.arange((n - 8) * kw, n * kw)
                idx += [at + head, at + tail]
                at += n * kw
        else:
            idx += [at + np.arange(0, conv, 37)]
            at += conv
            idx += [at + np.arange(0, rec, 97)]
            at += rec
    return np.concatenate(idx).astype(np.int64), at


def main():
    import zg_oracle as O
    from zerogravity_amd import gguf, qwen35
    t = qwen35.synthetic_tensors(GEOMETRY, gguf.Q4_K, seed=WEIGHT_SEED)
    toks = prompt()
    t0 = time.time()
    with O.libm_mode(O.LIBM_GLIBC):
        o = O.Model(GEOMETRY, t).session(kv_bf16=True)
        for i, tok in enumerate(toks[:-1]):
            o.forward(int(tok), need_logits=False)
            if i % 1024 == 0:
                print(f"{i} tokens, {time.time() - t0:.0f} s", flush=True)
        logits = o.forward(int(toks[-1]))
        state = o.state()
    idx, total = state_index(GEOMETRY, N_PROMPT)
    assert total == state.size, (total, state.size)
    np.savez_compressed(os.path.join(HERE, "prefill_8192_oracle.npz"), logits=logits.astype(np.float32),
                        greedy=np.array([O.greedy(logits)], np.int64), state_idx=idx,
                        state=state[idx].astype(np.float32))
    print(f"done in {time.time() - t0:.0f} s: greedy {O.greedy(logits)}, {idx.size} state values")


if __name__ == "__main__":
    main()
