"""Boundary B semantics on the device: publication, snapshots, shared
weights, threading and the device greedy readout.

The reference publishes a decode step only at commit and a prefill only if
every token succeeds (QwenDenseCpu::next_logits / commit /
prefill_transaction, model-qwen35/src/lib.rs:1057-1070, 1114-1187,
1211-1225), restores sessions from snapshots (gpu/src/
resident_inference.rs:2766, 3258), keys resident weights by their source
(core/src/accelerator.rs:22-68), is Send + Sync (accelerator.rs:682) and
reads greedy tokens with greedy_finite (core/src/numerics.rs:124-162).

A failing step is forced from the model's data: layer 0's ssm_norm gamma has
one element of 3.4e38, so the gated RMSNorm output overflows to infinity
when the normalised GDN output times silu(z) at that element exceeds 1 in
magnitude, and the residual stream becomes nonfinite (ZG_E_STATE).  That
depends on the token and the state; which tokens fail at a given state is
found by proposing them, which publishes nothing.
"""
import threading

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import gguf, qwen35
from zerogravity_amd import regions as R

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]

TINY = dict(hidden=512, layers=4, ffn=512, vocab=1000, gdn_heads=2, gdn_dim=128, q_heads=2, kv_heads=1,
            head_dim=256, full_attention_interval=4, max_context=4096, eps=1e-6)


@pytest.fixture(scope="module")
def kern():
    return R.HipMatVecKernel(0)


@pytest.fixture(scope="module")
def tiny():
    return qwen35.synthetic_tensors(TINY, gguf.Q4_K, seed=31)


@pytest.fixture(scope="module")
def fragile():
    """The tiny Q4_K model with one ssm_norm element of 3.4e38 in layer 0."""
    t = dict(qwen35.synthetic_tensors(TINY, gguf.Q4_K, seed=32))
    ty, s0, s1, data = t["blk.0.ssm_norm.weight"]
    gamma = np.frombuffer(data.tobytes(), np.float32).copy()
    gamma[5] = 3.4e38
    t["blk.0.ssm_norm.weight"] = (ty, s0, s1, gamma.view(np.uint8))
    return t


def _probe(sess, want_ok, start):
    """The first token from `start` whose step at the session's current
    state succeeds (want_ok) or fails with ZG_E_STATE; proposals publish
    nothing, so probing leaves the session as it was."""
    for i in range(TINY["vocab"]):
        tok = (start + i) % TINY["vocab"]
        try:
            sess.next_logits([tok])
            ok = True
        except L.ZgError as e:
            assert e.code == L.E_STATE, e
            ok = False
        if ok == want_ok:
            return tok
    pytest.skip("no such token at this state")


def test_failed_step_and_prefill_publish_nothing(kern, fragile):
    m = qwen35.QwenModelHip(TINY, fragile, kernel=kern)
    s = m.session(max_batch=1, max_context=256, kv_dtype=L.F32)
    hist = []
    for i in range(3):  # a prompt of tokens that pass, each published by commit
        hist.append(_probe(s, True, 37 * i))
        s.next_logits([hist[-1]])
        s.commit()
    assert s.position == 3
    before = s.state()
    # a failing decode step: nothing moves
    bad = _probe(s, False, 0)
    with pytest.raises(L.ZgError) as e:
        s.forward(bad)
    assert e.value.code == L.E_STATE
    assert s.position == 3
    assert np.array_equal(s.state().view(np.uint32), before.view(np.uint32))
    # the session goes on as one that never saw the failed token
    ref = m.session(max_batch=1, max_context=256, kv_dtype=L.F32)
    for tok in hist:
        ref.forward(tok)
    t3 = _probe(s, True, 500)
    assert np.array_equal(s.forward(t3).view(np.uint32), ref.forward(t3).view(np.uint32))
    # a prompt whose third token fails at its position
    snap = s.snapshot(0)
    at4 = s.state()
    t4 = _probe(s, True, 100)
    s.forward(t4)
    t5 = _probe(s, True, 200)
    s.forward(t5)
    bad2 = _probe(s, False, 300)
    s.restore(snap, 0)
    assert s.position == 4
    assert np.array_equal(s.state().view(np.uint32), at4.view(np.uint32))
    with pytest.raises(L.ZgError):
        s.prefill_transaction([t4, t5, bad2, t3])
    assert s.position == 4
    assert np.array_equal(s.state().view(np.uint32), at4.view(np.uint32))
    # batched prefill: rolls back as well (its f16 projections overflow on
    # every token of this model, so here it always fails)
    with pytest.raises(L.ZgError):
        s.prefill_batched([t4, t5, bad2])
    assert s.position == 4
    assert np.array_equal(s.state().view(np.uint32), at4.view(np.uint32))
    # and the session still decodes exactly as the one that saw no failure
    assert np.array_equal(s.forward(t4).view(np.uint32), ref.forward(t4).view(np.uint32))
    snap.close()
    m.close()


def test_failed_batched_prefill_keeps_other_rows(kern, fragile):
    """A batched prefill that fails on one row (its f16 projections overflow
    on every token of this model) leaves the other rows as the host has
    them, including a row imported since the last step, whose host position
    and published GDN half are newer than the device's copies."""
    m = qwen35.QwenModelHip(TINY, fragile, kernel=kern)
    donor = m.session(max_batch=1, max_context=256, kv_dtype=L.F32)
    for i in range(2):
        donor.forward(_probe(donor, True, 53 * i + 7))
    image = donor.state()
    s = m.session(max_batch=2, max_context=256, kv_dtype=L.F32)
    for i in range(3):  # row 0 steps: its position and published half move on the device
        s.forward(_probe(s, True, 91 * i + 5))
    s.load_state(image, 2, row=0)
    with pytest.raises(L.ZgError):
        s.prefill_batched([1, 2, 3], row=1)
    assert s.positions() == [2, 0]
    assert np.array_equal(s.state(0).view(np.uint32), image.view(np.uint32))
    # row 0 decodes as the donor does
    t = _probe(donor, True, 400)
    assert np.array_equal(s.forward(t).view(np.uint32), donor.forward(t).view(np.uint32))
    m.close()


def test_batched_prefill_refuses_32bit_operands(kern):
    """An operand of the prompt GEMM reaching 4 GiB (here the f16 activation
    tiles of the FFN down projection, 262144 rows x K = 8192) is ZG_E_LIMIT
    before any projection runs; the session is untouched."""
    g = dict(TINY, ffn=8192, max_context=262400)
    m = qwen35.QwenModelHip(g, qwen35.synthetic_tensors(g, gguf.Q4_K, seed=33), kernel=kern)
    s = m.session(max_batch=1, max_context=262400, kv_dtype=L.BF16)
    with pytest.raises(L.ZgError) as e:
        s.prefill_batched(np.ones(262144, np.uint32))
    assert e.value.code == L.E_LIMIT
    assert s.position == 0
    assert np.all(s.state() == 0.0)
    s.forward(1)
    assert s.position == 1
    m.close()


def test_propose_and_commit(kern, tiny):
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=2, max_context=64, kv_dtype=L.F32)
    ref = m.session(max_batch=2, max_context=64, kv_dtype=L.F32)
    toks = np.random.default_rng(3).integers(0, TINY["vocab"], (6, 2)).astype(np.uint32)
    with pytest.raises(L.ZgError) as e:
        s.commit()  # nothing proposed
    assert e.value.code == L.E_STATE
    for i in range(6):
        before = s.state(0)
        lg, gr = s.next_logits(toks[i], greedy=True)
        # a proposal publishes nothing, and proposing again recomputes the same draft
        assert s.positions() == [i, i]
        assert np.array_equal(s.state(0).view(np.uint32), before.view(np.uint32))
        again = s.next_logits(toks[i])
        assert np.array_equal(lg.view(np.uint32), again.view(np.uint32))
        s.commit()
        with pytest.raises(L.ZgError):
            s.commit()  # already published
        r_lg, r_gr = ref.step(toks[i], greedy=True)
        assert np.array_equal(lg.view(np.uint32), r_lg.view(np.uint32)), i
        assert np.array_equal(gr, r_gr)
        assert list(gr) == [int(np.argmax(row)) for row in lg]
    assert s.positions() == [6, 6]
    # any other step drops a pending proposal
    s.next_logits(toks[0])
    s.step(toks[1])
    with pytest.raises(L.ZgError):
        s.commit()
    m.close()


def test_snapshot_restore_and_fork(kern, tiny):
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=2, max_context=64, kv_dtype=L.BF16)
    toks = np.random.default_rng(4).integers(0, TINY["vocab"], 12).astype(np.uint32)
    for t in toks[:5]:
        s.forward(int(t))
    snap = s.snapshot(0)
    assert snap.position == 5
    first = [s.forward(int(t)) for t in toks[5:9]]
    s.restore(snap, 0)
    assert s.position == 5
    again = [s.forward(int(t)) for t in toks[5:9]]
    for a, b in zip(first, again):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # restored into another session of the same model: the same next step
    other = m.session(max_batch=2, max_context=64, kv_dtype=L.BF16)
    other.restore(snap, 0)
    assert np.array_equal(other.forward(int(toks[5])).view(np.uint32), first[0].view(np.uint32))
    # forked into row 1 beside an unrelated row 0 (a two-row step)
    fork = m.session(max_batch=2, max_context=64, kv_dtype=L.BF16)
    fork.restore(snap, 1)
    assert fork.positions() == [0, 5]
    lg, _ = fork.step([int(toks[0]), int(toks[5])])
    # two rows take the batched f16 MFMA kernels, one row the int8
    # matrix-core GEMV: the f16 and int16 activation codings agree to a few
    # 1e-3
    assert float(np.max(np.abs(lg[1] - first[0]))) <= 5e-3
    # a snapshot of another model, or of another KV type, is foreign
    m2 = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    with pytest.raises(L.ZgError) as e:
        m2.session(max_batch=1, max_context=64, kv_dtype=L.BF16).restore(snap, 0)
    assert e.value.code == L.E_STATE
    with pytest.raises(L.ZgError) as e:
        m.session(max_batch=1, max_context=64, kv_dtype=L.F32).restore(snap, 0)
    assert e.value.code == L.E_STATE
    with pytest.raises(L.ZgError) as e:
        m.session(max_batch=1, max_context=4, kv_dtype=L.BF16).restore(snap, 0)
    assert e.value.code == L.E_LIMIT
    snap.close()
    m2.close()
    m.close()


def test_models_sharing_a_source_keep_their_weights(kern, tiny):
    """Two models loaded from one source share its resident weights;
    destroying one leaves the other's intact (each holds a reference)."""
    a = qwen35.QwenModelHip(TINY, tiny, kernel=kern, source_id=777001)
    sa = a.session(max_batch=1, max_context=32, kv_dtype=L.F32)
    toks = [5, 77, 301, 999]
    want = [sa.forward(t) for t in toks]
    b = qwen35.QwenModelHip(TINY, tiny, kernel=kern, source_id=777001)
    sb = b.session(max_batch=1, max_context=32, kv_dtype=L.F32)
    sa.close()
    a.close()
    kern.ctx.check(L.lib().zg_source_release(kern.ctx.h, 777001))  # handles released; b still holds its weights
    got = [sb.forward(t) for t in toks]
    for x, y in zip(want, got):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    b.close()


def test_threads_share_a_context(kern):
    """Four threads run region GEMVs on one context while a fifth fails on
    purpose; every result is the single-thread one and each thread reads
    its own failure text."""
    rng = np.random.default_rng(9)
    w = qwen35.synth.random_matrix(rng, gguf.Q8_0, 384, 1024)
    xs = [rng.standard_normal(1024).astype(np.float32) for _ in range(4)]
    want = [O.matvec(gguf.Q8_0, w.reshape(-1), 384, 1024, x) for x in xs]
    errors, texts = [], {}
    mine = kern.ctx.error()

    def worker(i):
        try:
            for _ in range(20):
                res = kern.try_execute(R.MatVecRegion(R.SourceIdentity(55), "thr", gguf.Q8_0, 1024, 384,
                                                      w.reshape(-1), xs[i]))
                assert np.array_equal(res.values.view(np.uint32), want[i].view(np.uint32))
        except Exception as e:  # reported to the main thread
            errors.append(e)

    def failer():
        bad = np.zeros(4, np.float32)
        for _ in range(20):
            rc = L.lib().zg_rms_norm(kern.ctx.h, bad.ctypes.data, bad.ctypes.data, 0, 1e-6, bad.ctypes.data)
            assert rc < 0
            texts["failer"] = kern.ctx.error()

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(4)] + [threading.Thread(target=failer)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    assert texts["failer"] == "invalid grouped RMS normalization dimensions"
    assert kern.ctx.error() == mine  # the failures of another thread do not replace this thread's text


def test_reset_waits_for_queued_device_steps(kern, tiny):
    import torch
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=2, max_context=64, kv_dtype=L.F32)
    st = torch.cuda.Stream()
    toks = torch.tensor([3, 4], dtype=torch.int32, device="cuda")
    greedy = torch.empty(2, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        for _ in range(8):
            kern.ctx.check(L.lib().zg_decode_step_device(s.h, 2, toks.data_ptr(), None, greedy.data_ptr(),
                                                         st.cuda_stream))
    s.reset()  # no host synchronisation before: the queued steps must land first
    assert s.positions() == [0, 0]
    st0 = s.state(0)
    assert st0.size > 0 and not np.any(st0)
    fresh = m.session(max_batch=1, max_context=64, kv_dtype=L.F32)
    assert np.array_equal(s.forward(7).view(np.uint32), fresh.forward(7).view(np.uint32))
    m.close()


def test_device_steps_with_many_buffers(kern, tiny):
    """A caller that hands new buffers every step gets a new captured graph
    each time; the cache stays bounded and every step stays correct."""
    import torch
    m = qwen35.QwenModelHip(TINY, tiny, kernel=kern)
    s = m.session(max_batch=1, max_context=64, kv_dtype=L.F32)
    ref = m.session(max_batch=1, max_context=64, kv_dtype=L.F32)
    tok = 11
    keep = []  # distinct buffers every step
    for i in range(24):
        d_tok = torch.tensor([tok], dtype=torch.int32, device="cuda")
        d_out = torch.empty(1, dtype=torch.int32, device="cuda")
        keep += [d_tok, d_out]
        torch.cuda.synchronize()
        kern.ctx.check(L.lib().zg_decode_step_device(s.h, 1, d_tok.data_ptr(), None, d_out.data_ptr(), None))
        kern.ctx.check(L.lib().zg_session_check(s.h, None))
        got = int(d_out.cpu()[0])
        want = int(ref.step([tok], greedy=True)[1][0])
        assert got == want, i
        tok = got
    assert s.position == 24
    m.close()


def test_device_greedy_matches_greedy_finite(kern):
    rng = np.random.default_rng(5)
    V, rows = 151936, 6
    lg = rng.standard_normal((rows, V)).astype(np.float32)
    # ties across the 64 partial blocks and within one: the first index wins
    per = ((V + 63) // 64 + 3) & ~3
    lg[0, [7 * per + 3, 2 * per + 9, 40 * per]] = 50.0
    lg[1, [per - 1, per]] = 60.0              # the two sides of a block boundary
    lg[2, [V - 1, V - 2]] = 70.0
    lg[3, 100] = -0.0
    lg[3] = np.minimum(lg[3], -1.0)
    lg[3, 100], lg[3, 50] = 0.0, -0.0         # a signed-zero tie: the first one wins
    lg[4] = 1.25                              # all equal
    out = np.empty(rows, np.uint32)
    kern.ctx.check(L.lib().zg_greedy(kern.ctx.h, lg.ctypes.data, rows, V, out.ctypes.data))
    for r in range(rows):
        assert int(out[r]) == O.greedy(lg[r]), r
    assert list(out[:5]) == [2 * per + 9, per - 1, V - 2, 50, 0]
    for bad in (np.nan, np.inf, -np.inf):
        x = lg[:2].copy()
        x[1, 12345] = bad
        rc = L.lib().zg_greedy(kern.ctx.h, x.ctypes.data, 2, V, out.ctypes.data)
        assert rc == L.E_STATE, bad
    assert L.lib().zg_greedy(kern.ctx.h, lg.ctypes.data, 1, 0, out.ctypes.data) == L.E_LIMIT
    # the reference's own table (numerics.rs:146-162)
    for vals, want in (([-0.0, 0.0], 0), ([0.0, -0.0], 0), ([3.0, 3.0], 0), ([-2.0, 4.0, 4.0], 1)):
        v = np.array(vals, np.float32)
        kern.ctx.check(L.lib().zg_greedy(kern.ctx.h, v.ctypes.data, 1, v.size, out.ctypes.data))
        assert int(out[0]) == want
