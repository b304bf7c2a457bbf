"""The committed L=8192 prefill fixture (tests/golden/prefill_8192_oracle.npz)
is consistent with the script that wrote it: the stored state indices are
the ones state_index() selects for the geometry and prompt length, the
greedy token is the first maximum of the stored logits (the reference's
greedy rule, core/src/numerics.rs:126-140: the first maximum wins), and every
stored value is finite.  The GPU comparison against it is in
test_prefill_gpu.py."""
import os
import sys

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_prefill_8192 as G  # noqa: E402


def test_fixture_matches_its_script():
    ref = np.load(os.path.join(HERE, "prefill_8192_oracle.npz"))
    idx, total = G.state_index(G.GEOMETRY, G.N_PROMPT)
    assert np.array_equal(ref["state_idx"], idx)
    assert idx.min() >= 0 and idx.max() < total and np.all(np.diff(idx) > 0)
    lg = ref["logits"]
    assert lg.shape == (G.GEOMETRY["vocab"],) and np.all(np.isfinite(lg))
    assert int(ref["greedy"][0]) == int(np.argmax(lg))
    assert ref["state"].shape == idx.shape and np.all(np.isfinite(ref["state"]))


def test_prompt_is_reproducible():
    p = G.prompt()
    assert p.dtype == np.uint32 and p.size == G.N_PROMPT
    assert np.array_equal(p, G.prompt()) and int(p.max()) < G.GEOMETRY["vocab"]
