"""The decode step's fused projection forms through zg_gemv_device_fused,
against the oracle's operations in the reference's order: RMSNorm
(model-qwen35/src/lib.rs:263-284), the gated grouped RMSNorm times silu(z)
(forward.rs:586-594), the SwiGLU product (forward.rs:498), the residual add
(forward.rs:489,501), the tied embedding row (cpu/src/source.rs:214-222) and
greedy_finite (core/src/numerics.rs:126-140).  Q8_0 bit-identical; Q4_K
within 1e-3 relative (max |err| / max |ref| per row)."""
import zlib

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import regions as R
from zerogravity_amd import synth

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]
Q4K_REL = 1e-3
PRO_RMS, PRO_GATED, PRO_SILU_MUL, PRO_PLAIN = 0, 1, 2, 3
EPI_STORE, EPI_RESID, EPI_GLU = 0, 1, 2


@pytest.fixture(scope="module")
def kern():
    k = R.HipMatVecKernel(0)
    yield k
    k.ctx.close()


def _check(kind, got, ref):
    if kind == synth.Q8_0:
        assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32)), \
            float(np.max(np.abs(got - ref)))
    else:
        for m in range(ref.shape[0]):
            err = float(np.max(np.abs(got[m] - ref[m])) / np.max(np.abs(ref[m])))
            assert err <= Q4K_REL, (m, err)


def _fused(kern, h, M, pro, epi, x, x2, gamma, y, ldy, group=128, emb=None, tok=None, gmax=None, gidx=None):
    import torch
    p = lambda t: None if t is None else t.data_ptr()
    rc = L.lib().zg_gemv_device_fused(kern.ctx.h, h.h, M, pro, epi, x.data_ptr(), x.shape[-1], p(x2),
                                      0 if x2 is None else x2.shape[-1], p(gamma), 1e-6, group, y.data_ptr(), ldy,
                                      None if emb is None else emb.h, p(tok), p(gmax), p(gidx), None)
    if rc != L.UNSUPPORTED:
        kern.ctx.check(rc)
    torch.cuda.synchronize()
    return rc


@pytest.mark.parametrize("kind", [synth.Q8_0, synth.Q4_K])
@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("form", ["rms_store", "gated_resid", "plain_resid", "silu_mul_resid", "rms_glu"])
def test_fused_forms_match_oracle(kern, kind, M, form):
    import torch
    rng = np.random.default_rng(zlib.crc32(f"{kind}.{M}.{form}".encode()))
    K, N = 2048, 1024 if form != "rms_glu" else 2048
    w = synth.random_matrix(rng, kind, N, K)
    h = kern.register(700 + kind, f"fused.{kind}.{form}.{M}", kind, K, N, w.reshape(-1))
    x = rng.standard_normal((M, K)).astype(np.float32)
    x2 = rng.standard_normal((M, K)).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    pro = {"rms_store": PRO_RMS, "gated_resid": PRO_GATED, "plain_resid": PRO_PLAIN, "silu_mul_resid": PRO_SILU_MUL,
           "rms_glu": PRO_RMS}[form]
    epi = {"rms_store": EPI_STORE, "rms_glu": EPI_GLU}.get(form, EPI_RESID)
    g_use = gamma[:128] if pro == PRO_GATED else gamma
    wr = w.reshape(-1)
    refs = []
    for m in range(M):
        if pro == PRO_RMS:
            a = O.rms_norm(x[m], gamma, 1e-6)
        elif pro == PRO_GATED:
            a = O.silu(x2[m], mult=O.grouped_rms_norm(x[m], g_use, K // 128, 1e-6))
        elif pro == PRO_SILU_MUL:
            a = O.silu(x[m], mult=x2[m])
        else:
            a = x[m]
        if epi == EPI_GLU:
            full = O.matvec(kind, wr, N, K, a)
            refs.append(O.silu(full[:N // 2], mult=full[N // 2:]))
        else:
            v = O.matvec(kind, wr, N, K, a)
            refs.append(O.binary(0, y0[m], v) if epi == EPI_RESID else v)
    ref = np.stack(refs)
    dx, dx2 = torch.from_numpy(x).cuda(), torch.from_numpy(x2).cuda()
    dg = torch.from_numpy(g_use.copy()).cuda()
    ncol = N // 2 if epi == EPI_GLU else N
    dy = torch.from_numpy(y0[:, :ncol].copy() if epi == EPI_RESID else np.full((M, ncol), np.nan, np.float32)).cuda()
    rc = _fused(kern, h, M, pro, epi, dx, dx2 if pro in (PRO_GATED, PRO_SILU_MUL) else None,
                dg if pro in (PRO_RMS, PRO_GATED) else None, dy, ncol)
    if kind == synth.Q8_0 and epi == EPI_GLU:
        # the step fuses SwiGLU into Q4_K projections only (Q8_0 models run
        # the product in the down projection's prologue)
        assert rc == L.UNSUPPORTED
        return
    assert rc == L.COMPLETED
    _check(kind, dy.cpu().numpy(), ref)


PRO_GATED_PRE = 5


@pytest.mark.parametrize("kind", [synth.Q8_0, synth.Q4_K])
def test_fused_gated_pre_is_the_gated_form(kern, kind):
    """ZG_PRO_GATED_PRE, the one-row step's ssm_out (the GDN kernel forms
    (x * gamma) * silu(z) once, the projection applies the per-head 1/rms):
    with x2 holding that product formed by the same float operations (the
    oracle's silu is the device's bit for bit) the result is ZG_PRO_GATED's
    bit for bit, and within 1e-3 of the reference's order.  N = 2048 takes
    the 8-row tiles.  Other codecs and several rows are refused."""
    import torch
    rng = np.random.default_rng(1717)
    K, N = 2048, 2048
    w = synth.random_matrix(rng, kind, N, K)
    h = kern.register(730 + kind, f"fused.pre.{kind}", kind, K, N, w.reshape(-1))
    x = rng.standard_normal((1, K)).astype(np.float32)
    z = rng.standard_normal((1, K)).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    y0 = rng.standard_normal((1, N)).astype(np.float32)
    u = O.silu(z[0], mult=x[0] * np.tile(g, K // 128))[None]
    dx, dz, du, dg = (torch.from_numpy(a.copy()).cuda() for a in (x, z, u, g))
    if kind != synth.Q4_K:
        dy = torch.from_numpy(y0.copy()).cuda()
        assert _fused(kern, h, 1, PRO_GATED_PRE, EPI_RESID, dx, du, None, dy, N) == L.UNSUPPORTED
        return
    dy_g = torch.from_numpy(y0.copy()).cuda()
    assert _fused(kern, h, 1, PRO_GATED, EPI_RESID, dx, dz, dg, dy_g, N) == L.COMPLETED
    dy_p = torch.from_numpy(y0.copy()).cuda()
    assert _fused(kern, h, 1, PRO_GATED_PRE, EPI_RESID, dx, du, None, dy_p, N) == L.COMPLETED
    got_g, got_p = dy_g.cpu().numpy(), dy_p.cpu().numpy()
    assert np.array_equal(got_p.view(np.uint32), got_g.view(np.uint32))
    a = O.silu(z[0], mult=O.grouped_rms_norm(x[0], g, K // 128, 1e-6))
    ref = O.binary(0, y0[0], O.matvec(kind, w.reshape(-1), N, K, a))[None]
    _check(kind, got_p, ref)
    x3 = torch.from_numpy(np.repeat(x, 3, 0)).cuda()
    u3 = torch.from_numpy(np.repeat(u, 3, 0)).cuda()
    y3 = torch.from_numpy(np.repeat(y0, 3, 0)).cuda()
    assert _fused(kern, h, 3, PRO_GATED_PRE, EPI_RESID, x3, u3, None, y3, N) == L.UNSUPPORTED


def test_fused_embedding_prologue_and_greedy_partials(kern):
    """One row: the token's Q4_K embedding row dequantised in the prologue
    (stored at x bit-exactly) feeding an RMS projection, and an LM-head
    shaped projection leaving per-workgroup greedy partials whose
    combination is greedy_finite of the device's own logits."""
    import torch
    rng = np.random.default_rng(11)
    K, V, N = 2048, 3000, 4096
    emb = synth.random_matrix(rng, synth.Q4_K, V, K)
    w = synth.random_matrix(rng, synth.Q4_K, N, K)
    he = kern.register(720, "fused.embd", synth.Q4_K, K, V, emb.reshape(-1))
    hw = kern.register(720, "fused.in", synth.Q4_K, K, N, w.reshape(-1))
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    tok = 1234
    row = O.dequantize(synth.Q4_K, emb.reshape(-1), V * K).reshape(V, K)[tok]
    dx = torch.full((1, K), np.nan, dtype=torch.float32, device="cuda")
    dy = torch.full((1, N), np.nan, dtype=torch.float32, device="cuda")
    dg = torch.from_numpy(gamma).cuda()
    dt = torch.tensor([tok], dtype=torch.int32, device="cuda")
    _fused(kern, hw, 1, PRO_RMS, EPI_STORE, dx, None, dg, dy, N, emb=he, tok=dt)
    assert np.array_equal(dx.cpu().numpy()[0].view(np.uint32), row.view(np.uint32))
    _check(synth.Q4_K, dy.cpu().numpy(), O.matvec(synth.Q4_K, w.reshape(-1), N, K, O.rms_norm(row, gamma, 1e-6))[None])
    # greedy partials of an LM-head shaped projection (ties placed across workgroups)
    parts = int(L.lib().zg_gemv_greedy_parts(he.h))
    assert parts > 0
    gmax = torch.full((parts,), np.nan, dtype=torch.float32, device="cuda")
    gidx = torch.full((parts,), -1, dtype=torch.int32, device="cuda")
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).cuda()
    lg = torch.full((1, V), np.nan, dtype=torch.float32, device="cuda")
    _fused(kern, he, 1, PRO_RMS, EPI_STORE, x, None, dg, lg, V, gmax=gmax, gidx=gidx)
    logits = lg.cpu().numpy()[0]
    m, i = gmax.cpu().numpy(), gidx.cpu().numpy()
    best = np.max(m)
    assert best == np.max(logits)
    assert int(np.min(i[m == best])) == O.greedy(logits)


def test_fused_refusals(kern):
    import torch
    rng = np.random.default_rng(3)
    K, N = 2048, 256
    w = synth.random_matrix(rng, synth.Q4_K, N, K)
    h = kern.register(730, "fused.refuse", synth.Q4_K, K, N, w.reshape(-1))
    x = torch.zeros((8, K), dtype=torch.float32, device="cuda")
    y = torch.zeros((8, N), dtype=torch.float32, device="cuda")
    g = torch.ones(K, dtype=torch.float32, device="cuda")
    lib = L.lib()
    # five rows (the batched kernels are not one launch), a missing gamma,
    # a bad prologue code
    for M, pro, gam in ((5, PRO_RMS, g), (1, PRO_RMS, None), (1, 9, g)):
        rc = lib.zg_gemv_device_fused(kern.ctx.h, h.h, M, pro, EPI_STORE, x.data_ptr(), K, None, 0,
                                      None if gam is None else gam.data_ptr(), 1e-6, 128, y.data_ptr(), N, None,
                                      None, None, None, None)
        assert rc == L.E_MALFORMED, (M, pro)
