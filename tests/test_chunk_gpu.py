"""GPU parity of the chunked (WY/UT) GDN prefill against the CPU oracle.

The chunk reference is numerics/torch_cpu/gdn/chunk/core.rs:69-274 (one
chunk per call, key-major state, bf16-rounded outputs); the oracle restates
it (oracle/zg_oracle.c zgo_gdn_chunk_prefill) and is pinned against the
token-by-token recurrence in test_oracle_kat.py.  The device runs its
products on v_mfma_f32_16x16x4f32, whose four products per step accumulate
as a chain of fused multiply-adds in k order, so a product over k = 0..K-1
reproduces the reference's FMA chain (core.rs:277-310) exactly; the solves
follow gdn/chunk.rs:16-76 operation by operation.  State and outputs are
therefore required bit-identical to the oracle's; the 1e-3 relative bar of
the north star applies only against the token-by-token recurrence.

Inputs follow the prefill benchmark's synthetic distribution: q, k, v and
beta bf16-exact, beta = sigmoid(N(0,1)), log decay = -softplus(N(0,1)) *
exp(N(0,0.5)), prior state N(0, 0.02).
"""
import math

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import chunk as CH

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]
REL_TOL = 1e-3
D = 128


def bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


def inputs(seed, T, H, prior=True):
    rng = np.random.default_rng(seed)
    q = bf16(rng.standard_normal(T * H * D))
    k = bf16(rng.standard_normal(T * H * D))
    v = bf16(rng.standard_normal(T * H * D))
    beta = bf16(1.0 / (1.0 + np.exp(-rng.standard_normal(T * H))))
    logd = (-np.log1p(np.exp(rng.standard_normal(T * H))) * np.exp(0.5 * rng.standard_normal(T * H)))
    logd = np.minimum(logd, 0.0).astype(np.float32)
    st = (0.02 * rng.standard_normal(H * D * D)).astype(np.float32) if prior else None
    return q, k, v, beta, logd, st


def rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def key_major(st, H):
    return np.ascontiguousarray(st.reshape(H, D, D).transpose(0, 2, 1)).reshape(-1)


@pytest.fixture(scope="module")
def ctx():
    c = L.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


def test_chunk_zero_updates_preserve_prior_and_refuse_invalid(ctx):
    # chunk/tests/core.rs:5-71: zero q/k/v/beta/log-decay leave a prior of
    # 3.5 bit-identical and give +0 outputs; malformed inputs are refused.
    H, rows = 16, 17
    zeros = np.zeros(rows * H * D, np.float32)
    rates = np.zeros(rows * H, np.float32)
    state = np.full(H * D * D, 3.5, np.float32)

    def inp(**kw):
        base = dict(rows=rows, heads=H, query=zeros, key=zeros, value=zeros, beta=rates, log_decay=rates,
                    previous_state=state)
        base.update(kw)
        return CH.ChunkInputs(**base)

    out = CH.core(ctx, inp())
    assert np.all(out.output_bf16.view(np.uint32) == 0)
    assert np.array_equal(out.state, state)
    bad = [dict(rows=65), dict(heads=0), dict(previous_state=state[:-1]),
           dict(log_decay=np.full_like(rates, np.inf)), dict(log_decay=np.full_like(rates, 0.125)),
           dict(query=np.full_like(zeros, np.uint32(0x3F800001).view(np.float32))),
           dict(beta=np.zeros(1, np.float32)), dict(beta=np.full_like(rates, 2.0)),
           dict(log_decay=np.full_like(rates, -np.finfo(np.float32).max)), dict(heads=8, rows=34)]
    for b in bad:
        with pytest.raises(L.ZgError) as e:
            CH.core(ctx, inp(**b))
        assert e.value.code == L.E_MALFORMED, b
    assert np.all(state == 3.5)


@pytest.mark.parametrize("rows,H,prior", [(1, 16, False), (17, 16, True), (64, 16, True), (50, 32, True)])
def test_chunk_core_matches_oracle(ctx, rows, H, prior):
    q, k, v, beta, logd, st = inputs(100 + rows + H, rows, H, prior)
    res = CH.core(ctx, CH.ChunkInputs(rows, H, q, k, v, beta, logd, None if st is None else key_major(st, H)))
    out_r, st_r = O.gdn_chunk_prefill(q, k, v, beta, logd, H, D, 64, st)
    assert np.array_equal(res.state.view(np.uint32), key_major(st_r, H).view(np.uint32))
    assert np.array_equal(res.output_bf16.view(np.uint32), bf16(out_r).view(np.uint32))
    print(f"chunk core rows={rows} H={H} prior={prior}: state and bf16 outputs bit-identical")


def _device_prefill(ctx, torch, q, k, v, beta, logd, st, T, H):
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, k, v))
    db, dl = torch.from_numpy(beta).cuda(), torch.from_numpy(logd).cuda()
    ds = torch.from_numpy(st.copy()).cuda()
    do = torch.empty(T * H * D, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    CH.prefill_device(ctx, T, H, dq, dk, dv, db, dl, ds, do, None)
    torch.cuda.synchronize()
    return do.cpu().numpy(), ds.cpu().numpy()


@pytest.mark.parametrize("T", [1, 70, 130, 2048])
def test_prefill_device_matches_oracle(ctx, torch_cuda, T):
    H = 16
    q, k, v, beta, logd, st = inputs(7 + T, T, H, True)
    out, st_d = _device_prefill(ctx, torch_cuda, q, k, v, beta, logd, st, T, H)
    out_r, st_r = O.gdn_chunk_prefill(q, k, v, beta, logd, H, D, 64, st)
    print(f"prefill T={T} H={H}: out rel {rel_err(out, out_r):.2e} state rel {rel_err(st_d, st_r):.2e}")
    assert np.array_equal(st_d.view(np.uint32), st_r.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), out_r.view(np.uint32))


def _tokenwise_state(q, k, v, beta, logd, H, T):
    """Final state of the token-by-token recurrence (lib.rs:1446-1499) with
    the two-stage q/k L2 normalisation (forward.rs:564-576)."""
    sc = np.full(D, np.float32(1.0) / np.sqrt(np.float32(D)), np.float32)
    st = np.zeros(H * D * D, np.float32)
    scale = 1.0 / math.sqrt(D)
    for t in range(T):
        sl = slice(t * H * D, (t + 1) * H * D)
        qn = O.grouped_rms_norm(q[sl], sc, H, 1e-6 / D)
        kn = O.grouped_rms_norm(k[sl], sc, H, 1e-6 / D)
        for h in range(H):
            hs = slice(h * D, (h + 1) * D)
            _, s2 = O.gdn_recurrent_step(st[h * D * D:(h + 1) * D * D], qn[hs], kn[hs], v[sl][hs],
                                         float(np.exp(np.float32(logd[t * H + h]))), float(beta[t * H + h]), scale)
            st[h * D * D:(h + 1) * D * D] = s2
    return st


def test_prefill_final_state_matches_token_recurrence(ctx, torch_cuda):
    # Config 4's check at L = 2048, H = 16, S0 = 0: the chunked prefill's
    # final state equals the token-by-token recurrence's.
    T, H = 2048, 16
    q, k, v, beta, logd, _ = inputs(2048, T, H, False)
    st0 = np.zeros(H * D * D, np.float32)
    _, st_d = _device_prefill(ctx, torch_cuda, q, k, v, beta, logd, st0, T, H)
    st_t = _tokenwise_state(q, k, v, beta, logd, H, T)
    e = rel_err(st_d, st_t)
    print(f"prefill L={T} final state vs token recurrence: rel {e:.2e}")
    assert e <= REL_TOL, e


def test_prefill_long_state_properties(ctx, torch_cuda):
    # L = 8192 (config 4's long case): bit-identical to the oracle; two
    # halves run back to back give the same state and outputs as one call
    # (chunks are 64-aligned); the state stays finite and bounded.
    T, H = 8192, 16
    q, k, v, beta, logd, _ = inputs(8192, T, H, False)
    st0 = np.zeros(H * D * D, np.float32)
    out, st = _device_prefill(ctx, torch_cuda, q, k, v, beta, logd, st0, T, H)
    out_r, st_r = O.gdn_chunk_prefill(q, k, v, beta, logd, H, D, 64, st0)
    assert np.array_equal(st.view(np.uint32), st_r.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), out_r.view(np.uint32))
    half = T // 2
    a, b = slice(0, half * H * D), slice(half * H * D, T * H * D)
    o1, s1 = _device_prefill(ctx, torch_cuda, q[a], k[a], v[a], beta[:half * H], logd[:half * H], st0, half, H)
    o2, s2 = _device_prefill(ctx, torch_cuda, q[b], k[b], v[b], beta[half * H:], logd[half * H:], s1, half, H)
    assert np.array_equal(st, s2)
    assert np.array_equal(out, np.concatenate([o1, o2]))
    assert np.isfinite(out).all() and np.isfinite(st).all()
    assert float(np.abs(st).max()) < 1e3


def test_prefill_device_refuses_oversized_output(ctx):
    """(tokens + 64) * heads * 512 bytes of output at 4 GiB or more is
    refused on the host with ZG_E_LIMIT before any device memory is read
    (the output kernel's 32-bit buffer offsets, rows past the end included,
    must not wrap).  The buffers are allocated at the full size the call
    names (16 GiB in all), so a regression of the host check would compute
    in bounds and fail this test instead of faulting."""
    import torch
    tokens = (1 << 23) - 64  # (tokens + 64) * 1 head * 512 = 2^32
    qkv = [torch.empty(tokens * 128, dtype=torch.float32, device="cuda") for _ in range(3)]
    beta = torch.zeros(tokens, dtype=torch.float32, device="cuda")
    logd = torch.zeros(tokens, dtype=torch.float32, device="cuda")
    state = torch.zeros(128 * 128, dtype=torch.float32, device="cuda")
    out = torch.empty((tokens + 64) * 128, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    rc = L.lib().zg_gdn_chunk_prefill_device(ctx.h, tokens, 1, *[t.data_ptr() for t in qkv], beta.data_ptr(),
                                             logd.data_ptr(), state.data_ptr(), out.data_ptr(), None)
    assert rc == L.E_LIMIT
    assert "4 GiB" in ctx.error()
    del qkv, out
    torch.cuda.empty_cache()
