"""The allocation-free GEMV entry (zg_gemv_device_noalloc): the same
results as zg_gemv_device, bit for bit, on two calls in a row (the second
with a smaller input, so the static scratch holds the first call's larger
contents), for every codec path: bf16 input through the prepared
activation, f32 input through the in-kernel prologue (up to 4 rows),
through the f16 MFMA kernels (Q4_K beyond 4 rows) and through the
coded-once activation of the Q8_0 rows kernel (beyond 4 rows).  No counterpart in the
reference: the entry exists for callers that cannot allocate."""
import ctypes

import numpy as np
import pytest

from zerogravity_amd import _lib as L
from zerogravity_amd import regions as R
from zerogravity_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def kern():
    k = R.HipMatVecKernel(0)
    yield k
    k.ctx.close()


def _run(kern, fn, h, x, x_dtype, M, g, y):
    import torch
    kern.ctx.check(getattr(L.lib(), fn)(kern.ctx.h, h.h, x.data_ptr(), x_dtype, M, g.data_ptr(), 1e-6, y.data_ptr(),
                                        None))
    torch.cuda.synchronize()
    return y.cpu().numpy().copy()


@pytest.mark.parametrize("kind,N,K", [(synth.Q8_0, 3584, 1024), (synth.Q4_K, 2048, 6144), (synth.Q4_K, 6144, 2048),
                                      (synth.Q6_K, 1024, 2048), (synth.Q4_1, 640, 1024), (synth.F32, 300, 2048)])
@pytest.mark.parametrize("x_dtype", [L.F32, L.BF16])
def test_noalloc_matches_gemv_device(kern, kind, N, K, x_dtype):
    import torch
    rng = np.random.default_rng(N + K + x_dtype)
    w = synth.random_matrix(rng, kind, N, K)
    h = kern.register(900 + kind, f"noalloc.{kind}.{N}.{K}", kind, K, N, w.reshape(-1))
    g = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)).cuda()
    # first call with 32 rows, second with 3 (in-kernel prologue for f32) or 9
    for M in (32, 9, 3) if x_dtype == L.F32 else (32, 9):
        xf = rng.standard_normal((M, K)).astype(np.float32)
        if x_dtype == L.BF16:
            _, xb = synth.bf16_round(xf)
            x = torch.from_numpy(xb.view(np.int16)).cuda()
        else:
            x = torch.from_numpy(xf).cuda()
        y0 = torch.full((M, N), np.nan, dtype=torch.float32, device="cuda")
        y1 = torch.full((M, N), np.nan, dtype=torch.float32, device="cuda")
        rc = L.lib().zg_gemv_device(kern.ctx.h, h.h, x.data_ptr(), x_dtype, M, g.data_ptr(), 1e-6, y0.data_ptr(), None)
        if rc == L.UNSUPPORTED:
            pytest.skip("geometry not offered by the GEMV")
        kern.ctx.check(rc)
        torch.cuda.synchronize()  # the call ran on the context's stream
        want = y0.cpu().numpy()
        got = _run(kern, "zg_gemv_device_noalloc", h, x, x_dtype, M, g, y1)
        assert np.isfinite(want).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (M, x_dtype)


def test_noalloc_limits(kern):
    import torch
    rng = np.random.default_rng(5)
    K, N = 2048, 256
    w = synth.random_matrix(rng, synth.Q4_K, N, K)
    h = kern.register(950, "noalloc.limits", synth.Q4_K, K, N, w.reshape(-1))
    x = torch.zeros((65, K), dtype=torch.float32, device="cuda")
    y = torch.empty((65, N), dtype=torch.float32, device="cuda")
    g = torch.ones(K, dtype=torch.float32, device="cuda")
    rc = L.lib().zg_gemv_device_noalloc(kern.ctx.h, h.h, x.data_ptr(), L.F32, 65, g.data_ptr(), 1e-6, y.data_ptr(), None)
    assert rc == L.E_LIMIT
    # Q4_K beyond 4 rows on the 32-row kernel (K = 1536) before any
    # zg_gemv_device call built the weight's 32-row tiles
    K2 = 1536
    w2 = synth.random_matrix(rng, synth.Q4_K, N, K2)
    h2 = kern.register(951, "noalloc.limits.k1536", synth.Q4_K, K2, N, w2.reshape(-1))
    x2 = torch.zeros((8, K2), dtype=torch.float32, device="cuda")
    g2 = torch.ones(K2, dtype=torch.float32, device="cuda")
    rc = L.lib().zg_gemv_device_noalloc(kern.ctx.h, h2.h, x2.data_ptr(), L.F32, 8, g2.data_ptr(), 1e-6, y.data_ptr(),
                                        None)
    assert rc == L.E_STATE
    assert "tile layout" in kern.ctx.error()
    # the 16-row kernel (K = 2048) reads the weight's own layout: no tiles needed
    xr = torch.from_numpy(rng.standard_normal((8, K)).astype(np.float32)).cuda()
    got = _run(kern, "zg_gemv_device_noalloc", h, xr, L.F32, 8, g, torch.empty((8, N), device="cuda"))
    want = torch.empty((8, N), device="cuda")
    kern.ctx.check(L.lib().zg_gemv_device(kern.ctx.h, h.h, xr.data_ptr(), L.F32, 8, g.data_ptr(), 1e-6, want.data_ptr(),
                                          None))
    torch.cuda.synchronize()
    assert np.array_equal(got.view(np.uint32), want.cpu().numpy().view(np.uint32))


def test_noalloc_calls_on_two_streams_are_ordered(kern):
    """Calls on two streams, submitted back to back without a host wait,
    share the one static array: each must wait for the previous call's
    kernels, so both results still equal zg_gemv_device's bit for bit."""
    import torch
    rng = np.random.default_rng(77)
    K, N = 2048, 6144
    w = synth.random_matrix(rng, synth.Q4_K, N, K)
    h = kern.register(960, "noalloc.streams", synth.Q4_K, K, N, w.reshape(-1))
    g = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)).cuda()
    xs, wants = [], []
    for M in (32, 16, 8, 24):
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
        y = torch.full((M, N), np.nan, dtype=torch.float32, device="cuda")
        kern.ctx.check(L.lib().zg_gemv_device(kern.ctx.h, h.h, x.data_ptr(), L.F32, M, g.data_ptr(), 1e-6,
                                              y.data_ptr(), None))
        torch.cuda.synchronize()
        xs.append(x)
        wants.append(y.cpu().numpy())
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full(tuple(v.shape), np.nan, dtype=torch.float32, device="cuda") for v in wants]
    torch.cuda.synchronize()
    for rep in range(3):
        for i, (x, y) in enumerate(zip(xs, outs)):
            st = streams[i % 2]
            kern.ctx.check(L.lib().zg_gemv_device_noalloc(kern.ctx.h, h.h, x.data_ptr(), L.F32, x.shape[0],
                                                          g.data_ptr(), 1e-6, y.data_ptr(),
                                                          ctypes.c_void_p(st.cuda_stream)))
        torch.cuda.synchronize()
        for i, (y, want) in enumerate(zip(outs, wants)):
            got = y.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rep, i)
