"""Parity at the sizes the benchmark runs.

* Config 5: the 2B-shaped Q4_K model (24 layers, vocabulary 151936) decoding
  greedily from a seeded 2048-token state already in the bf16 KV cache and
  the GDN state, at B=1 and B=32, through zg_decode_step_device with the
  device's own greedy readout feeding the next step.  Held to the north
  star's end-to-end bar (logits within 2e-2 max-abs, identical greedy
  tokens) against the oracle calling glibc's transcendentals, as the
  reference's Rust f32 functions do (model-qwen35/src/lib.rs:1227-1254,
  forward.rs:451-755; greedy_finite, core/src/numerics.rs:124-140).
* Config 3: the resident GDN decode step at B = 8, 32 and 64 rows with 16
  heads, both kernels (a quarter head per workgroup; one head per workgroup
  with the gated RMSNorm into ssm_out's f16 tiles), bit-exact per row
  against the oracle's conv -> SiLU -> L2 -> gates -> recurrence chain
  (cpu/src/ops/gdn.rs:7-44, forward.rs:564-594, lib.rs:339-362,1446-1499).
"""
import math

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import gguf, qwen35
from zerogravity_amd import regions as R

pytestmark = pytest.mark.gpu
LOGIT_TOL = 2e-2
D = 128


def bf16_exact(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


# ------------------------------------------------------------ config 5

@pytest.fixture(scope="module")
def model_2b():
    g = dict(qwen35.QWEN35_2B, max_context=4096)
    t = qwen35.synthetic_tensors(g, gguf.Q4_K, seed=2027)
    return g, t


def _seeded_state(g, prefix, seed):
    """One row's state in the reference domain order (lib.rs:112-150): per
    GDN layer conv history [6144][3] ~ N(0, 0.5) and state [16][128][128] ~
    N(0, 0.02); per attention layer keys then values [prefix][512] ~ N(0, 1),
    bf16-exact so that the bf16 cache holds them unchanged."""
    rng = np.random.default_rng(seed)
    W = g["gdn_heads"] * g["gdn_dim"]
    kw = g["kv_heads"] * g["head_dim"]
    parts = []
    for kind in qwen35.layer_kinds(g):
        if kind == "linear_attention":
            parts.append((0.5 * rng.standard_normal(3 * W * 3)).astype(np.float32))
            parts.append((0.02 * rng.standard_normal(g["gdn_heads"] * D * D)).astype(np.float32))
        else:
            parts.append(bf16_exact(rng.standard_normal(prefix * kw)))
            parts.append(bf16_exact(rng.standard_normal(prefix * kw)))
    return np.concatenate(parts)


STEPS = 128  # 128 greedy steps
CHECKED = {1: (0,), 3: (0, 2), 32: (0, 4, 9, 13, 18, 22, 27, 31)}  # B=3: the batched f16 kernels below 16 rows
_RUNS = {}


def _device_run(model_2b, B):
    """The device's 128 greedy steps at B rows from the seeded 2048-token
    state, the device greedy feeding the next step (zg_decode_step_device);
    logits of the checked rows and every row's greedy token per step.  Run
    once per B and shared by the tests that check its rows."""
    if B in _RUNS:
        return _RUNS[B]
    import torch
    g, t = model_2b
    prefix, nstate = 2048, 8
    kern = R.HipMatVecKernel(0)
    m = qwen35.QwenModelHip(g, t, kernel=kern)
    s = m.session(max_batch=B, max_context=prefix + STEPS + 8, kv_dtype=L.BF16)
    states = [_seeded_state(g, prefix, 100 + i) for i in range(min(B, nstate))]
    for r in range(B):
        s.load_state(states[r % nstate], prefix, row=r)
    first = np.random.default_rng(B).integers(0, g["vocab"], B).astype(np.uint32)
    d_tok = torch.from_numpy(first.view(np.int32).copy()).cuda()
    d_logits = torch.empty((B, g["vocab"]), dtype=torch.float32, device="cuda")
    d_greedy = torch.empty(B, dtype=torch.int32, device="cuda")
    rows = list(CHECKED[B])
    logits = np.empty((STEPS, len(rows), g["vocab"]), np.float32)
    greedy = np.empty((STEPS, B), np.uint32)
    for step in range(STEPS):
        torch.cuda.synchronize()
        kern.ctx.check(L.lib().zg_decode_step_device(s.h, B, d_tok.data_ptr(), d_logits.data_ptr(),
                                                     d_greedy.data_ptr(), None))
        kern.ctx.check(L.lib().zg_session_check(s.h, None))
        logits[step] = d_logits[rows].cpu().numpy()
        greedy[step] = d_greedy.cpu().numpy().view(np.uint32)
        d_tok.copy_(d_greedy)
    assert s.positions() == [prefix + STEPS] * B
    m.close()
    kern.ctx.close()
    _RUNS[B] = dict(first=first, states=states, rows=rows, logits=logits, greedy=greedy)
    return _RUNS[B]


@pytest.mark.parametrize("B,checked", [(1, (0,)), (3, (0, 2)), (32, (0, 4)), (32, (9, 13)), (32, (18, 22)),
                                       (32, (27, 31))])
def test_config5_2b_q4k_decode_from_2048_prefix(model_2b, B, checked):
    """128 greedy steps, each checked row against its own oracle session
    (split over several tests so that each stays within the per-test time
    limit: the oracle decodes about 8 tokens/s on 16 cores).  The device
    decodes free-running (its greedy feeds its next step); the oracle takes
    the device's tokens, so every step compares the same history.  Every
    step: logits within 2e-2 max-abs, and the device's token is greedy_finite
    of its own logits.  The north star's greedy bar, identical tokens over
    32 steps, holds exactly for the first 32; beyond them a different token
    is allowed only at a near-tie, where the device's choice scores within
    the logit tolerance of the oracle's maximum (the per-op error of the f16
    batched projections can order two logits that close either way)."""
    g, t = model_2b
    run = _device_run(model_2b, B)
    oracle = O.Model(g, t)
    worst, ties = 0.0, []
    for r in checked:
        o = oracle.session(kv_bf16=True)
        o.load_state(run["states"][r % len(run["states"])], 2048)
        tok = int(run["first"][r])
        k = run["rows"].index(r)
        with O.libm_mode(O.LIBM_GLIBC):
            for step in range(STEPS):
                ref = o.forward(tok)
                lg = run["logits"][step, k]
                err = float(np.max(np.abs(lg - ref)))
                worst = max(worst, err)
                assert err <= LOGIT_TOL, (step, r, err)
                got = int(run["greedy"][step, r])
                assert got == O.greedy(lg)  # the device readout is greedy_finite of its own logits
                want = O.greedy(ref)
                if got != want:
                    margin = float(ref[want] - ref[got])
                    assert step >= 32 and margin <= LOGIT_TOL, (step, r, got, want, margin)
                    ties.append((step, r, margin))
                tok = got
    print(f"config 5 B={B}: {STEPS} greedy steps, rows {checked}, worst logit max-abs {worst:.3e}, "
          f"near-ties {ties}")


# ------------------------------------------------------------ config 3

def _oracle_gdn_row(proj, conv_w, hist, state, dt, a, H, eps):
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


def _tile_index(B, W):
    """f16 index of (row m, channel k) in the batched projections' A tiles:
    the 16-row decode kernel's layout for B < 256 rows and W a multiple of
    1024 up to 6144, else the 32-row layout (include/zg_hip.h)."""
    m = np.arange(B)[:, None]
    k = np.arange(W)[None, :]
    if B < 256 and W % 1024 == 0 and W <= 6144:
        op = 2 * ((k >> 5) & 1) + ((k >> 3) & 1)
        lane = (m & 15) + 16 * (((k >> 4) & 1) + 2 * ((k >> 6) & 1))
        return ((((m >> 4) * (W >> 7) + (k >> 7)) * 4 + op) * 64 + lane) * 8 + (k & 7)
    lane = ((k & 15) >> 3) * 32 + (m & 31)
    return ((((m >> 5) * (W >> 8) + (k >> 8)) * 16 + ((k & 255) >> 4)) * 64 + lane) * 8 + (k & 7)


@pytest.mark.usefixtures("exact_libm")
@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("B", [8, 32, 64])
def test_config3_gdn_decode_rows_bit_exact(B, gated):
    import torch
    ctx = L.Context(0)
    H, eps = 16, 1e-6
    W = H * D
    rng = np.random.default_rng(300 + B + 7 * gated)
    stride = 4 * W + 2 * H
    conv_w = (0.5 * rng.standard_normal(3 * W * 4)).astype(np.float32)
    dt = (0.1 * rng.standard_normal(H)).astype(np.float32)
    a = (-np.exp(0.5 * rng.standard_normal(H))).astype(np.float32)
    norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    state = (0.02 * rng.standard_normal((B, H * D * D))).astype(np.float32)
    d_conv, d_dt, d_a, d_norm = (torch.from_numpy(x).cuda() for x in (conv_w, dt, a, norm))
    d_ring = torch.zeros(B * 3 * W * 4, device="cuda")
    d_state = torch.from_numpy(state.reshape(-1).copy()).cuda()
    d_core = torch.empty(B * W, device="cuda")
    nt = L.lib().zg_gdn_decode_tiles_bytes(B, H)
    d_tiles = torch.zeros(nt // 2, dtype=torch.float16, device="cuda")
    hist = [np.zeros(3 * W * 3, np.float32) for _ in range(B)]
    ref_state = [state[b].copy() for b in range(B)]
    idx = _tile_index(B, W)
    for step in range(3):
        # BASELINE config 3 inputs: q/k/v pre-activations ~ N(0,1) (L2-normalised
        # in the step), beta = sigmoid(N(0,1)), decay from softplus(N(0,1))
        proj = rng.standard_normal((B, stride)).astype(np.float32)
        d_proj = torch.from_numpy(proj).cuda()
        d_pos = torch.full((B,), 2040 + step, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        if gated:
            rc = L.lib().zg_gdn_decode_gated_device(ctx.h, B, H, d_proj.data_ptr(), stride, d_conv.data_ptr(),
                                                    d_ring.data_ptr(), d_pos.data_ptr(), d_dt.data_ptr(),
                                                    d_a.data_ptr(), d_norm.data_ptr(), eps, d_state.data_ptr(),
                                                    d_core.data_ptr(), d_tiles.data_ptr(), None)
        else:
            rc = L.lib().zg_gdn_decode_device(ctx.h, B, H, d_proj.data_ptr(), stride, d_conv.data_ptr(),
                                              d_ring.data_ptr(), d_pos.data_ptr(), d_dt.data_ptr(), d_a.data_ptr(),
                                              eps, d_state.data_ptr(), d_core.data_ptr(), None)
        ctx.check(rc)
        torch.cuda.synchronize()
        core = d_core.cpu().numpy().reshape(B, W)
        st = d_state.cpu().numpy().reshape(B, -1)
        tiles = d_tiles.cpu().numpy()
        for b in range(B):
            ref_core, hist[b], ref_state[b] = _oracle_gdn_row(proj[b], conv_w, hist[b], ref_state[b], dt, a, H, eps)
            assert np.array_equal(core[b].view(np.uint32), ref_core.view(np.uint32)), (step, b)
            assert np.array_equal(st[b].view(np.uint32), ref_state[b].view(np.uint32)), (step, b)
            if gated:
                gn = O.grouped_rms_norm(ref_core, norm, H, eps)
                z = proj[b, 3 * W:4 * W]
                want = (gn * O.silu(z)).astype(np.float16)
                assert np.array_equal(tiles[idx[b]].view(np.uint16), want.view(np.uint16)), (step, b)
    print(f"GDN decode B={B} gated={gated}: 3 steps bit-identical per row")
    ctx.close()
