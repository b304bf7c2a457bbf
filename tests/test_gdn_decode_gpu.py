"""GPU parity of the resident GDN decode step (zg_gdn_decode_device) against
the CPU oracle's per-operator chain on identical seeded inputs: causal conv
(cpu/src/ops/gdn.rs:7-44), SiLU, two-stage q/k L2 (forward.rs:564-576),
gates (lib.rs:339-362) and the recurrence (lib.rs:1446-1499).  Every step is
restated in the reference's operation order on both sides, so the core
outputs and states are required bit-identical, over several rows and
consecutive positions (the 4-slot conv ring wraps)."""
import math

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]
D = 128


@pytest.fixture(scope="module")
def ctx():
    c = L.Context(0)
    yield c
    c.close()


def _oracle_row(proj, conv_w, hist, state, dt, a, H, eps):
    W = H * D
    raw, hist = O.gdn_conv_step(proj[:3 * W], conv_w, hist)
    act = O.silu(raw)
    sc = np.full(D, np.float32(1.0) / np.sqrt(np.float32(D)), np.float32)
    qn = O.grouped_rms_norm(act[:W], sc, H, eps / D)
    kn = O.grouped_rms_norm(act[W:2 * W], sc, H, eps / D)
    v = act[2 * W:3 * W]
    gain, beta, _, _ = O.gdn_coefficients(proj[4 * W:4 * W + H], proj[4 * W + H:4 * W + 2 * H], dt, a,
                                          1 / math.sqrt(D))
    core = np.empty(W, np.float32)
    st = state.copy()
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        o, s2 = O.gdn_recurrent_step(st[h * D * D:(h + 1) * D * D], qn[sl], kn[sl], v[sl], float(gain[h]),
                                     float(beta[h]), 1 / math.sqrt(D))
        st[h * D * D:(h + 1) * D * D] = s2
        core[sl] = o
    return core, hist, st


@pytest.mark.parametrize("B,H", [(1, 16), (3, 4)])
def test_gdn_decode_device_matches_oracle(ctx, B, H):
    import torch
    rng = np.random.default_rng(40 + B)
    W = H * D
    stride = 4 * W + 2 * H
    conv_w = (0.5 * rng.standard_normal(3 * W * 4)).astype(np.float32)
    dt = (0.1 * rng.standard_normal(H)).astype(np.float32)
    a = (-np.exp(rng.standard_normal(H))).astype(np.float32)
    state = (0.02 * rng.standard_normal((B, H * D * D))).astype(np.float32)
    eps = 1e-6
    d_conv = torch.from_numpy(conv_w).cuda()
    d_dt, d_a = torch.from_numpy(dt).cuda(), torch.from_numpy(a).cuda()
    d_ring = torch.zeros(B * 3 * W * 4, device="cuda")
    d_state = torch.from_numpy(state.reshape(-1).copy()).cuda()
    d_core = torch.empty(B * W, device="cuda")
    hist = [np.zeros(3 * W * 3, np.float32) for _ in range(B)]
    ref_state = [state[b].copy() for b in range(B)]
    for step in range(6):
        proj = rng.standard_normal((B, stride)).astype(np.float32)
        d_proj = torch.from_numpy(proj).cuda()
        d_pos = torch.full((B,), step, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        ctx.check(L.lib().zg_gdn_decode_device(ctx.h, B, H, d_proj.data_ptr(), stride, d_conv.data_ptr(),
                                               d_ring.data_ptr(), d_pos.data_ptr(), d_dt.data_ptr(),
                                               d_a.data_ptr(), eps, d_state.data_ptr(), d_core.data_ptr(), None))
        torch.cuda.synchronize()
        core = d_core.cpu().numpy().reshape(B, W)
        st = d_state.cpu().numpy().reshape(B, -1)
        for b in range(B):
            ref_core, hist[b], ref_state[b] = _oracle_row(proj[b], conv_w, hist[b], ref_state[b], dt, a, H, eps)
            assert np.array_equal(core[b].view(np.uint32), ref_core.view(np.uint32)), (step, b)
            assert np.array_equal(st[b].view(np.uint32), ref_state[b].view(np.uint32)), (step, b)
    print(f"GDN decode B={B} H={H}: 6 steps bit-identical")
