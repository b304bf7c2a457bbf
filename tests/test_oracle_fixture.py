"""The reference's only real-distribution GDN step vector, pinning the
oracle's recurrence and its two-stage L2.

tests/golden/pinned_cached_head0.f32le.bin is the data file the reference
test crates/zerogravity-cpu/src/numerics/torch_cpu/recurrent_tests.rs:14-76
reads (its SHA-256 is the one that test's comment records): head 0 of
layer 0, second token, of the original Qwen3.5 0.8B checkpoint, captured
from pinned Torch CPU.  Layout per recurrent_tests.rs:14-45: b"ZGCG128\\0",
the words 1, 1, 14, then 14 fields each as a word count and f32 words:
q, k, v (raw, bf16-exact), beta, decay (the multiplicative gain), the
previous state (key-major [k][v]), L2-normalised q and k, q / sqrt(128),
two intermediates, the f32 core output, its bf16 rounding, the new state.

Torch evaluates the update as separate multiplies and adds and its key-axis
sums in its own order (recurrent.rs:155-225); the GGUF recurrence the
oracle restates fuses the update and sums with the 32-accumulator tree
(model-qwen35/src/lib.rs:1446-1499).  So the check is at tolerance, not
bits: 1e-5 relative, the reference's own bound for its recurrence
(lib.rs:1998-2055).  A key-major state used without transposing it is
shown to fail.
"""
import hashlib
import math
import os

import numpy as np

import zg_oracle as O

PATH = os.path.join(os.path.dirname(__file__), "golden", "pinned_cached_head0.f32le.bin")
SHA256 = "78b2664bd9018b419ed1d1ea2d36f6a7fc01d615a0653cb962b2176fb9900065"
COUNTS = [128, 128, 128, 1, 1, 16384, 128, 128, 128, 128, 128, 128, 128, 16384]
TOL = 1e-5


def fields():
    raw = open(PATH, "rb").read()
    assert hashlib.sha256(raw).hexdigest() == SHA256
    assert raw[:8] == b"ZGCG128\0"
    words = np.frombuffer(raw[8:], "<u4")
    assert list(words[:3]) == [1, 1, 14]
    at, out = 3, []
    for n in COUNTS:
        assert words[at] == n
        out.append(words[at + 1:at + 1 + n].view("<f4").astype(np.float32))
        at += 1 + n
    assert at == words.size
    return out


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))


def test_fixture_l2_normalisation():
    f = fields()
    d = 128
    gamma = np.full(d, np.float32(1) / np.sqrt(np.float32(d)), np.float32)
    for raw, want in ((f[0], f[6]), (f[1], f[7])):
        got = O.grouped_rms_norm(raw, gamma, 1, np.float32(1e-6) / np.float32(d))
        assert rel(got, want) <= TOL, rel(got, want)
    # the scaled query the cached path multiplies with (q / sqrt(128))
    assert rel(f[6] / np.float32(math.sqrt(d)), f[8]) <= TOL


def test_fixture_recurrent_step():
    f = fields()
    d = 128
    q, k, v = f[0], f[1], f[2]
    beta, gain = float(f[3][0]), float(f[4][0])
    gamma = np.full(d, np.float32(1) / np.sqrt(np.float32(d)), np.float32)
    qn = O.grouped_rms_norm(q, gamma, 1, np.float32(1e-6) / np.float32(d))
    kn = O.grouped_rms_norm(k, gamma, 1, np.float32(1e-6) / np.float32(d))
    prev_vm = np.ascontiguousarray(f[5].reshape(d, d).T)  # key-major -> value-major [v][k]
    core, state_vm = O.gdn_recurrent_step(prev_vm.reshape(-1), qn, kn, v, gain, beta, 1 / math.sqrt(d))
    state_km = state_vm.reshape(d, d).T
    print(f"core rel {rel(core, f[11]):.2e} state rel {rel(state_km, f[13].reshape(d, d)):.2e}")
    assert rel(core, f[11]) <= TOL
    assert rel(state_km, f[13].reshape(d, d)) <= TOL
    # bf16 output: the core rounded to bf16 within one bf16 unit of the pinned words
    u = core.view(np.uint32)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).view(np.float32)
    assert np.all(np.abs(b - f[12]) <= np.abs(f[12]) * 2.0 ** -7)
    # the plausible mistake: the key-major state taken as value-major
    bad, _ = O.gdn_recurrent_step(np.ascontiguousarray(f[5]), qn, kn, v, gain, beta, 1 / math.sqrt(d))
    assert rel(bad, f[11]) > 100 * TOL
