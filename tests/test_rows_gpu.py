"""Continuous-batch row management on the device session: admission by
batched prefill into a row, retirement by zg_session_copy_row +
zg_session_reset_row (the active rows stay dense for the batched decode
step), and forking a prefilled prompt into another row.

Reference behaviour: each row of a cohort evolves as its own session
(resident_inference.rs:1101-1111, private per-row state); a row's logits
depend only on its own tokens.  Every row is therefore checked against the
oracle's own session for its request (the north star's 2e-2 end-to-end bar,
same greedy token; the oracle calls glibc's transcendentals as the
reference's f32 functions do) and against its own one-row device session
run on the same tokens.  One row takes the int8 matrix-core GEMV (int16
activation codes) and two or more rows of Q4_K weights the batched f16
MFMA kernels (the activation rounded to f16), so the device pair agrees to
the two codings' noise: up to ~6e-3 on these logits, within ROW_TOL (half
the end-to-end bar), far below the O(1) difference a leak between rows
would show; prefill logits of the same prompt run the same kernels and
agree bit for bit.
"""
import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import gguf, qwen35
from zerogravity_amd import regions as R

pytestmark = pytest.mark.gpu
ROW_TOL = 1e-2
LOGIT_TOL = 2e-2

TINY = dict(hidden=512, layers=4, ffn=512, vocab=1000, gdn_heads=2, gdn_dim=128, q_heads=2, kv_heads=1,
            head_dim=256, full_attention_interval=4, max_context=4096, eps=1e-6)


@pytest.fixture(scope="module")
def tensors():
    return qwen35.synthetic_tensors(TINY, gguf.Q4_K, seed=12)


@pytest.fixture(scope="module")
def model(tensors):
    kern = R.HipMatVecKernel(0)
    m = qwen35.QwenModelHip(TINY, tensors, kernel=kern)
    yield m
    m.close()


@pytest.fixture(scope="module")
def oracle(tensors):
    return O.Model(TINY, tensors)


def _toks(seed, n):
    return np.random.default_rng(seed).integers(0, TINY["vocab"], n).astype(np.uint32)


class Solo:
    """One request on its own one-row device session, with the oracle's
    session for the same request beside it."""

    def __init__(self, model, prompt, oracle=None):
        self.s = model.session(max_batch=1, max_context=256, kv_dtype=L.BF16)
        self.last = self.s.prefill_batched(prompt)
        self.o = None
        if oracle is not None:
            self.o = oracle.session(kv_bf16=True)
            with O.libm_mode(O.LIBM_GLIBC):
                for t in prompt:
                    self.ref = self.o.forward(int(t))
            check_oracle(self.last, self.ref)

    def step(self, tok):
        self.last = self.s.forward(tok)
        if self.o is not None:
            with O.libm_mode(O.LIBM_GLIBC):
                self.ref = self.o.forward(int(tok))
            check_oracle(self.last, self.ref)
        return self.last


def check_oracle(lg, ref):
    err = float(np.max(np.abs(lg - ref)))
    assert err <= LOGIT_TOL, err
    assert int(np.argmax(lg)) == O.greedy(ref)


def test_admit_decode_retire_compact(model, oracle):
    prompts = [_toks(1, 40), _toks(2, 9), _toks(3, 70)]
    s = model.session(max_batch=4, max_context=256, kv_dtype=L.BF16)
    solos = [Solo(model, p, oracle) for p in prompts]
    last = []
    for r, p in enumerate(prompts):
        last.append(s.prefill_batched(p, row=r))
        assert np.array_equal(last[r], solos[r].last)  # same kernels, same row arithmetic
    assert s.positions() == [40, 9, 70, 0]
    active = 3
    owner = [0, 1, 2]  # request held by each active row
    toks = [int(np.argmax(x)) for x in last]
    for step in range(6):
        if step == 3:
            # retire the request in row 1: row 2 moves into it
            active = s.retire(1, active)
            owner = [owner[0], owner[2]]
            toks = [toks[0], toks[2]]
            assert s.positions()[2] == 0 and np.all(s.state(row=2) == 0)
        lg, _ = s.step(np.array(toks, np.uint32))
        for r in range(active):
            solo = solos[owner[r]]
            ref = solo.step(toks[r])
            err = float(np.max(np.abs(lg[r] - ref)))
            assert err <= ROW_TOL, (step, r, err)
            assert int(np.argmax(lg[r])) == int(np.argmax(ref))
            check_oracle(lg[r], solo.ref)  # the retired row's successor too
        toks = [int(np.argmax(lg[r])) for r in range(active)]
    pos = s.positions()
    assert pos[0] == 40 + 6 and pos[1] == 70 + 6 and pos[2] == 0
    # admit a new request into the freed slot: the same logits as its own
    # session, and the oracle's for that prompt
    lg = s.prefill_batched(_toks(4, 33), row=2)
    admitted = Solo(model, _toks(4, 33), oracle)
    assert np.array_equal(lg, admitted.last)
    lg2, _ = s.step(np.array(toks + [int(np.argmax(lg))], np.uint32))
    check_oracle(lg2[2], admitted.o.forward(int(np.argmax(lg))))
    s.close()


def test_copy_row_forks_prompt_and_refuses_bad_rows(model):
    s = model.session(max_batch=3, max_context=128, kv_dtype=L.F32)
    s.prefill_batched(_toks(9, 50), row=0)
    s.copy_row(2, 0)
    assert s.positions() == [50, 0, 50]
    assert np.array_equal(s.state(row=2).view(np.uint32), s.state(row=0).view(np.uint32))
    # both copies continue identically from the same token
    lg, _ = s.step(np.array([5, 0, 5], np.uint32))
    assert np.array_equal(lg[0], lg[2])
    # a shorter row copied over a longer one (row 1 stepped above: retire it first)
    s.reset_row(1)
    s.prefill_batched(_toks(10, 7), row=1)
    s.copy_row(2, 1)
    assert s.positions()[2] == 7
    assert np.array_equal(s.state(row=2).view(np.uint32), s.state(row=1).view(np.uint32))
    s.copy_row(1, 1)
    for bad in ((3, 0), (0, 3)):
        with pytest.raises(L.ZgError) as e:
            s.copy_row(*bad)
        assert e.value.code == L.E_LIMIT
    with pytest.raises(L.ZgError) as e:
        s.reset_row(3)
    assert e.value.code == L.E_LIMIT
    s.reset_row(0)
    assert s.positions() == [0, 7, 7]
    assert np.all(s.state(row=0) == 0)
    s.close()
