"""GPU parity of the batched prefill (zg_prefill_batched) against the CPU
oracle's token-by-token prefill.

Reference: QwenDenseCpu::prefill_transaction (model-qwen35/src/lib.rs:
1119-1187) runs forward_token once per prompt token.  The batched path
computes the same functions layer by layer over the whole prompt: Q4_K
projections as f16 MFMA GEMMs, the GDN layers through the chunked WY/UT
prefill (gdn/chunk.rs), causal attention with an online softmax appending
to the KV cache.  The order of summation differs, so the bar is the
end-to-end one: last-token logits within 2e-2 max-abs with the same greedy
token, the recurrent and KV state close enough that greedy decoding that
continues from it picks the oracle's tokens.
"""
import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import gguf, qwen35
from zerogravity_amd import regions as R

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]
LOGIT_TOL = 2e-2

TINY = dict(hidden=512, layers=4, ffn=512, vocab=1000, gdn_heads=2, gdn_dim=128, q_heads=2, kv_heads=1,
            head_dim=256, full_attention_interval=4, max_context=4096, eps=1e-6)
WIDE = dict(hidden=2048, layers=4, ffn=6144, vocab=1000, gdn_heads=16, gdn_dim=128, q_heads=8, kv_heads=2,
            head_dim=256, full_attention_interval=4, max_context=4096, eps=1e-6)


def _tokens(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.uint32)


def rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.fixture(scope="module")
def kern():
    k = R.HipMatVecKernel(0)
    yield k


@pytest.fixture(scope="module")
def tiny():
    return qwen35.synthetic_tensors(TINY, gguf.Q4_K, seed=12)


def _oracle_prefill(o, toks):
    for t in toks[:-1]:
        o.forward(int(t), need_logits=False)
    return o.forward(int(toks[-1]))


def _greedy_tail(s, o, lg, ref, steps):
    """Continue greedy decoding of row 0 on both sides from the prefill's
    logits."""
    worst = float(np.max(np.abs(lg - ref)))
    tok = int(np.argmax(ref))
    assert int(np.argmax(lg)) == tok
    for i in range(steps):
        got = s.forward(tok)
        want = o.forward(tok)
        worst = max(worst, float(np.max(np.abs(got - want))))
        assert int(np.argmax(got)) == int(np.argmax(want)), i
        tok = int(np.argmax(want))
    return worst


@pytest.mark.parametrize("n,kv", [(1, L.F32), (17, L.BF16), (70, L.F32), (130, L.BF16)])
def test_prefill_batched_matches_token_prefill(kern, tiny, n, kv):
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=1, max_context=256, kv_dtype=kv)
    o = O.Model(TINY, tiny).session(kv_bf16=kv == L.BF16)
    toks = _tokens(100 + n, n, TINY["vocab"])
    lg = s.prefill_batched(toks)
    ref = _oracle_prefill(o, toks)
    assert s.positions()[0] == n
    sg, so = s.state(), o.state()
    assert sg.size == so.size
    e_state = rel_err(sg, so)
    worst = _greedy_tail(s, o, lg, ref, 8)
    print(f"batched prefill n={n} kv={kv}: logits/decode max-abs {worst:.3e}, state rel {e_state:.2e}")
    assert worst <= LOGIT_TOL
    assert e_state <= 1e-2
    m.close()


def test_prefill_batched_in_pieces_and_rows(kern, tiny):
    """Two prompt pieces back to back (the second starts mid-chunk at
    position 45, reading the conv ring and KV cache the first left), on row 1
    of a two-row session; row 0 is left untouched."""
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=2, max_context=256, kv_dtype=L.F32)
    toks = _tokens(5, 100, TINY["vocab"])
    s.prefill_batched(toks[:45], row=1, logits=False)
    lg = s.prefill_batched(toks[45:], row=1)
    assert s.positions() == [0, 100]
    o = O.Model(TINY, tiny).session()
    ref = _oracle_prefill(o, toks)
    st = s.state(row=1)
    assert rel_err(st, o.state()) <= 1e-2
    assert np.all(s.state(row=0) == 0)
    worst = float(np.max(np.abs(lg - ref)))
    print(f"batched prefill 45+55 on row 1: logits max-abs {worst:.3e}")
    assert worst <= LOGIT_TOL and int(np.argmax(lg)) == int(np.argmax(ref))
    m.close()


def test_prefill_batched_refusals(kern, tiny):
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=1, max_context=32, kv_dtype=L.F32)
    for bad, code in ((np.zeros(0, np.uint32), L.E_MALFORMED), (np.array([TINY["vocab"]], np.uint32), L.E_MALFORMED),
                      (np.zeros(33, np.uint32), L.E_LIMIT)):
        with pytest.raises(L.ZgError) as e:
            s.prefill_batched(bad)
        assert e.value.code == code
    with pytest.raises(L.ZgError) as e:
        s.prefill_batched(np.zeros(1, np.uint32), row=1)
    assert e.value.code == L.E_LIMIT
    assert s.positions() == [0]
    m.close()
    t8 = qwen35.synthetic_tensors(TINY, gguf.Q8_0, seed=3)
    m8 = qwen35.QwenModelHip(TINY, t8, kernel=kern)
    s8 = m8.session(max_batch=1, max_context=32, kv_dtype=L.F32)
    with pytest.raises(L.ZgError) as e:
        s8.prefill_batched(np.zeros(4, np.uint32))
    assert e.value.code == L.E_UNSUPPORTED
    m8.close()


@pytest.mark.parametrize("kv", [L.BF16, L.F32])
def test_prefill_batched_2b_shapes(kern, kv):
    """The 2B layer shapes (16 GDN heads, 8 query / 2 KV heads, FFN 6144) over
    a 150-token prompt: three GDN chunks, the last ragged; both cache types
    (4 query heads per KV head: the attention kernel loads the next key block
    ahead in either)."""
    t = qwen35.synthetic_tensors(WIDE, gguf.Q4_K, seed=21)
    m = qwen35.QwenModelHip(WIDE, t, kernel=kern)
    s = m.session(max_batch=1, max_context=256, kv_dtype=kv)
    o = O.Model(WIDE, t).session(kv_bf16=kv == L.BF16)
    toks = _tokens(9, 150, WIDE["vocab"])
    lg = s.prefill_batched(toks)
    ref = _oracle_prefill(o, toks)
    e_state = rel_err(s.state(), o.state())
    worst = _greedy_tail(s, o, lg, ref, 4)
    print(f"batched prefill 2B shapes n=150 kv={kv}: logits/decode max-abs {worst:.3e}, state rel {e_state:.2e}")
    assert worst <= LOGIT_TOL
    assert e_state <= 1e-2
    m.close()


def test_prefill_batched_repeatable_and_tracks_token_prefill(kern):
    """A long prompt on a fresh session (the call that allocates and clears
    the prompt buffers) and again after reset give bit-identical logits and
    state; both track the device's token-by-token prefill."""
    t = qwen35.synthetic_tensors(WIDE, gguf.Q4_K, seed=4)
    m = qwen35.QwenModelHip(WIDE, t, kernel=kern)
    n = 4000
    s = m.session(max_batch=1, max_context=4096, kv_dtype=L.BF16)
    toks = _tokens(31, n, WIDE["vocab"])
    lg0 = s.prefill_batched(toks)
    st0 = s.state()
    s.reset()
    lg1 = s.prefill_batched(toks)
    assert np.array_equal(lg0.view(np.uint32), lg1.view(np.uint32))
    assert np.array_equal(st0.view(np.uint32), s.state().view(np.uint32))
    s.reset()
    lt = s.prefill_transaction(toks)
    worst = float(np.max(np.abs(lt - lg0)))
    print(f"batched vs token-by-token prefill n={n}: logits max-abs {worst:.3e}")
    assert worst <= LOGIT_TOL and int(np.argmax(lt)) == int(np.argmax(lg0))
    m.close()


@pytest.mark.parametrize("n", [400, 600, 2048])
def test_prefill_batched_prompt_gemm_matches_oracle(kern, n):
    """From 256 prompt rows every projection runs through the register-
    blocked prompt GEMM (zg_gemm.hip: Q4_K dequantized in registers, f16
    MFMA, f32 accumulation; SwiGLU on the f32 gate/up sums, rounded once to
    f16 for the down projection).  The lengths cover the residual
    projections' split over K (four runs at 400 rows, two at 600 and at
    2048 for K >= 4096) and the prompt attention's key chunks (below 256
    tile workgroups).  At the 2B layer shapes against the
    oracle's token-by-token prefill with glibc transcendentals (the
    reference's): last logits within 2e-2 max-abs, the same greedy token,
    state within 1e-2 relative, and the first decoded token after it the
    same; the result is bit-identical on a repeat."""
    t = qwen35.synthetic_tensors(WIDE, gguf.Q4_K, seed=8)
    m = qwen35.QwenModelHip(WIDE, t, kernel=kern)
    s = m.session(max_batch=1, max_context=n + 16, kv_dtype=L.BF16)
    toks = _tokens(77 + n, n, WIDE["vocab"])
    lg0 = s.prefill_batched(toks)
    st0 = s.state()
    s.reset()
    lg1 = s.prefill_batched(toks)
    assert np.array_equal(lg0.view(np.uint32), lg1.view(np.uint32))
    assert np.array_equal(st0.view(np.uint32), s.state().view(np.uint32))
    with O.libm_mode(O.LIBM_GLIBC):
        o = O.Model(WIDE, t).session(kv_bf16=True)
        ref = _oracle_prefill(o, toks)
        e_state = rel_err(st0, o.state())
        worst = float(np.max(np.abs(lg0 - ref)))
        print(f"prompt-GEMM prefill n={n}: logits max-abs {worst:.3e} vs the oracle, state rel {e_state:.2e}")
        assert worst <= LOGIT_TOL and int(np.argmax(lg0)) == int(np.argmax(ref))
        assert e_state <= 1e-2
        tok = int(np.argmax(ref))
        assert int(np.argmax(s.forward(tok))) == int(np.argmax(o.forward(tok)))
    m.close()


def test_prefill_batched_8192_matches_oracle(kern):
    """The longest prompt the bench times: 8192 tokens at the 2B widths (4
    layers, bf16 KV) through zg_prefill_batched -- prompt GEMM, chunked GDN
    prefill over 128 chunks, prompt attention -- against the oracle's
    token-by-token prefill of the same seeded model and prompt with glibc's
    transcendentals (lib.rs:1119-1187; the expected values are the committed
    fixture tests/golden/prefill_8192_oracle.npz, written by
    tests/golden/make_prefill_8192.py because the oracle needs minutes for
    this prompt): last logits within 2e-2 max-abs, the same greedy token,
    the state (a fixed subsample of the export) within 1e-2 relative."""
    import os
    import sys
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    sys.path.insert(0, here)
    import make_prefill_8192 as G
    ref = np.load(os.path.join(here, "prefill_8192_oracle.npz"))
    t = qwen35.synthetic_tensors(G.GEOMETRY, gguf.Q4_K, seed=G.WEIGHT_SEED)
    m = qwen35.QwenModelHip(G.GEOMETRY, t, kernel=kern)
    s = m.session(max_batch=1, max_context=G.GEOMETRY["max_context"], kv_dtype=L.BF16)
    lg = s.prefill_batched(G.prompt())
    assert s.position == G.N_PROMPT
    st = s.state()
    idx, total = G.state_index(G.GEOMETRY, G.N_PROMPT)
    assert st.size == total and np.array_equal(idx, ref["state_idx"])
    worst = float(np.max(np.abs(lg - ref["logits"])))
    e_state = rel_err(st[idx], ref["state"])
    print(f"batched prefill n=8192: logits max-abs {worst:.3e} vs the oracle, state rel {e_state:.2e}")
    assert worst <= LOGIT_TOL
    assert int(np.argmax(lg)) == int(ref["greedy"][0])
    assert e_state <= 1e-2
    m.close()
