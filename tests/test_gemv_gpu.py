"""GPU parity of the GGUF dequant / GEMV path against the CPU oracle.

Tolerances: block dequantization bit-exact.  Q8_0 GEMV bit-exact: the
device codes the activation exactly as the CPU does and forms every row dot
in the CPU's order (integer block pairs, 8 FMA lanes, fixed lane tree).
Q4_K GEMV within 1e-3 relative error, measured as max|gpu-ref| / max|ref|
per activation row: the device carries the activation as 16-bit fixed point
per 32-element group and sums integer products, the CPU sums f32 products.
"""
import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import regions as R
from zerogravity_amd import synth

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]

SHAPES = [(3584, 1024), (1024, 3584), (6144, 2048), (2048, 6144), (151936, 2048)]
KINDS = [synth.Q8_0, synth.Q4_K]
REL_TOL = 1e-3


@pytest.fixture(scope="module")
def kern():
    k = R.HipMatVecKernel(0)
    yield k
    k.ctx.close()


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


_weights = {}
_streams = []


def _stream(torch):
    """A non-null torch stream (default priority) shared with the launches."""
    if not _streams:
        _streams.append(torch.cuda.Stream())
    s = _streams[0]
    torch.cuda.set_stream(s)
    return s.cuda_stream


def weight(kern, kind, N, K, seed=1):
    key = (kind, N, K, seed)
    if key not in _weights:
        rng = np.random.default_rng(seed * 1000 + N + K + kind)
        w = synth.random_matrix(rng, kind, N, K)
        h = kern.register(77, f"w.{kind}.{N}.{K}.{seed}", kind, K, N, w)
        _weights[key] = (w, h)
    return _weights[key]


def rel_err(got, ref):
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def row_subset(N):
    if N <= 8192:
        return [np.arange(N)]
    return [np.arange(2048), np.arange(N - 2048, N)]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", [(64, 1024), (3584, 1024), (256, 6144)])
def test_dequantize_bit_exact(kern, kind, N, K):
    w, h = weight(kern, kind, N, K)
    dev = h.dequantize()
    ref = O.dequantize(kind, w.reshape(-1), N * K).reshape(N, K)
    assert np.array_equal(dev.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", SHAPES)
def test_matvec_region_matches_oracle(kern, kind, N, K):
    w, _ = weight(kern, kind, N, K)
    x = np.random.default_rng(N + K).standard_normal(K).astype(np.float32)
    region = R.MatVecRegion(R.SourceIdentity(77), f"w.{kind}.{N}.{K}.1", kind, K, N, w.reshape(-1), x)
    res = kern.try_execute(region)
    assert isinstance(res, R.Completed)
    R.validate_completed(region, res.values)
    for rows in row_subset(N):
        ref = O.matvec(kind, w[rows].reshape(-1), rows.size, K, x)
        if kind == synth.Q8_0:
            assert np.array_equal(res.values[rows].view(np.uint32), ref.view(np.uint32))
        assert rel_err(res.values[rows], ref) <= REL_TOL


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 4, 16, 32])
def test_gemv_device_rms_prologue_bf16(kern, torch_cuda, kind, N, K, M):
    torch = torch_cuda
    w, h = weight(kern, kind, N, K)
    rng = np.random.default_rng(M * 7 + N)
    xf, xb = synth.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d = torch.from_numpy(xb.view(np.int16)).cuda()
    g_d = torch.from_numpy(gamma).cuda()
    y_d = torch.empty((M, N), dtype=torch.float32, device="cuda")
    stream = _stream(torch)
    rc = L.lib().zg_gemv_device(kern.ctx.h, h.h, x_d.data_ptr(), L.BF16, M, g_d.data_ptr(), 1e-6,
                                y_d.data_ptr(), stream)
    kern.ctx.check(rc)
    torch.cuda.synchronize()
    y = y_d.cpu().numpy()
    assert np.isfinite(y).all()
    worst = 0.0
    for m in range(M):
        xn = O.rms_norm(xf[m], gamma, 1e-6)
        for rows in row_subset(N):
            ref = O.matvec(kind, w[rows].reshape(-1), rows.size, K, xn)
            if kind == synth.Q8_0:
                assert np.array_equal(y[m, rows].view(np.uint32), ref.view(np.uint32)), m
            worst = max(worst, rel_err(y[m, rows], ref))
    assert worst <= REL_TOL, worst


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K,M", [(3584, 1024, m) for m in (1, 3, 16, 32, 1024, 1056)] +
                         [(2048, 6144, m) for m in (1, 3, 16, 32, 2048)] +
                         [(151936, 2048, m) for m in (1, 3, 16, 32)] + [(8224, 2048, 1088)] +
                         [(1000, 3072, m) for m in (1, 3)] + [(777, 5120, m) for m in (1, 4)] +
                         [(513, 8192, 1), (1030, 1536, 1), (70, 256, 2)])
def test_gemv_device_f32_decode_kernels(kern, torch_cuda, kind, N, K, M):
    """f32 activations take the decode-step kernels (in-kernel RMS prologue;
    Q4_K beyond 4 rows on the f16 MFMA path, the LDS-staged variant from
    1024 rows: 4, 1, 4 and 2 activation blocks per workgroup at M = 1024,
    1056, 2048 and 1088).  Up to 4 rows the Q4_K lanes per row and chunks
    per lane follow K: 16 x 3 at K = 3072, 32 x 3 at 5120 and 6144, 64 x 2 at
    8192, 32 x 1 at 1536 and 2048, 4 x 1 at 256; N not a multiple of the rows
    per wave exercises the clamped loads of rows past N."""
    torch = torch_cuda
    w, h = weight(kern, kind, N, K)
    rng = np.random.default_rng(M * 11 + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d = torch.from_numpy(x).cuda()
    g_d = torch.from_numpy(gamma).cuda()
    y_d = torch.empty((M, N), dtype=torch.float32, device="cuda")
    stream = _stream(torch)
    kern.ctx.check(L.lib().zg_gemv_device(kern.ctx.h, h.h, x_d.data_ptr(), L.F32, M, g_d.data_ptr(), 1e-6,
                                          y_d.data_ptr(), stream))
    torch.cuda.synchronize()
    y = y_d.cpu().numpy()
    worst = 0.0
    check = range(M) if M <= 32 else sorted({0, 1, 31, 32, 63, 64, M // 2, M - 33, M - 1})
    for m in check:
        xn = O.rms_norm(x[m], gamma, 1e-6)
        for rows in row_subset(N):
            ref = O.matvec(kind, w[rows].reshape(-1), rows.size, K, xn)
            if kind == synth.Q8_0:
                assert np.array_equal(y[m, rows].view(np.uint32), ref.view(np.uint32)), m
            worst = max(worst, rel_err(y[m, rows], ref))
    assert worst <= REL_TOL, worst


# Q8_0 beyond 4 rows on ragged shapes: K not a multiple of 128 (a last
# chunk of 1-3 blocks, checked per block), N not a multiple of 8 or 16 (a
# last row group or tile past N), both row kernels (the int8 matrix-core
# one takes 128+ tiles of 16 rows at 32+ rows, 256+ at 16+, 512+ at any
# count; the v_dot4 one the rest), and K = 8192 (four rows per workgroup,
# the LDS bound).  f32 input through the coded-once activation, bf16 through
# the prepared activation; bit-exact against the oracle either way.
@pytest.mark.parametrize("N,K,M", [(1001, 1056, 9), (777, 96, 33), (2050, 1056, 32), (8200, 96, 16),
                                   (4100, 4128, 17), (600, 8192, 20)])
@pytest.mark.parametrize("x_dtype", [L.F32, L.BF16])
def test_q8_rows_ragged_shapes_bit_exact(kern, torch_cuda, N, K, M, x_dtype):
    torch = torch_cuda
    if x_dtype == L.BF16 and M > 64:
        pytest.skip("bf16 activations take at most 64 rows")
    w, h = weight(kern, synth.Q8_0, N, K)
    rng = np.random.default_rng(N * 3 + K + M + x_dtype)
    xf = rng.standard_normal((M, K)).astype(np.float32)
    if x_dtype == L.BF16:
        xf, xb = synth.bf16_round(xf)
        x_d = torch.from_numpy(xb.view(np.int16)).cuda()
    else:
        x_d = torch.from_numpy(xf).cuda()
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    g_d = torch.from_numpy(gamma).cuda()
    y_d = torch.full((M, N), np.nan, dtype=torch.float32, device="cuda")
    stream = _stream(torch)
    kern.ctx.check(L.lib().zg_gemv_device(kern.ctx.h, h.h, x_d.data_ptr(), x_dtype, M, g_d.data_ptr(), 1e-6,
                                          y_d.data_ptr(), stream))
    torch.cuda.synchronize()
    y = y_d.cpu().numpy()
    for m in range(M):
        xn = O.rms_norm(xf[m], gamma, 1e-6)
        ref = O.matvec(synth.Q8_0, w.reshape(-1), N, K, xn)
        assert np.array_equal(y[m].view(np.uint32), ref.view(np.uint32)), (m, float(np.max(np.abs(y[m] - ref))))


def test_q8_activation_codes_bit_exact(kern, torch_cuda):
    # The prepared Q8_0 activation (RMSNorm + dynamic coding) must equal the
    # oracle's codes and f16-rounded scales bit for bit.
    torch = torch_cuda
    rng = np.random.default_rng(5)
    M, K = 4, 2048
    _, h = weight(kern, synth.Q8_0, 64, K)
    xf, xb = synth.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d = torch.from_numpy(xb.view(np.int16)).cuda()
    g_d = torch.from_numpy(gamma).cuda()
    nbytes = L.lib().zg_act_prepared_bytes(h.h, M)
    prep = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    stream = _stream(torch)
    kern.ctx.check(L.lib().zg_act_prepare_device(kern.ctx.h, h.h, x_d.data_ptr(), L.BF16, M, g_d.data_ptr(), 1e-6,
                                                 prep.data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    raw = prep.cpu().numpy()
    codes = raw[:M * K].view(np.int8).reshape(M, K)
    off = (M * K + 255) // 256 * 256
    scales = raw[off:off + M * (K // 32) * 4].view(np.float32).reshape(M, K // 32)
    for m in range(M):
        xn = O.rms_norm(xf[m], gamma, 1e-6)
        qs, d, _ = O.q8_activation(xn)
        assert np.array_equal(codes[m], qs)
        assert np.array_equal(scales[m].view(np.uint32), d.view(np.uint32))


def test_region_refusals(kern):
    x = np.ones(32, np.float32)
    w = np.zeros(34, np.uint8)
    # unsupported codec -> Unsupported (caller may use its CPU path)
    r = R.MatVecRegion(R.SourceIdentity(5), "t.q4_0", 2, 32, 1, np.zeros(18, np.uint8), np.ones(32, np.float32))
    assert kern.try_execute(r) is R.UNSUPPORTED
    # nonfinite activation -> error
    bad = R.MatVecRegion(R.SourceIdentity(5), "t.q8", synth.Q8_0, 32, 1, w, np.full(32, np.nan, np.float32))
    with pytest.raises(L.ZgError):
        kern.try_execute(bad)
    # nonfinite block scale -> error (codecs/q8.rs:6-15)
    w2 = w.copy()
    w2[0:2] = [0x00, 0x7C]
    with pytest.raises(L.ZgError):
        kern.try_execute(R.MatVecRegion(R.SourceIdentity(0), "t.q8inf", synth.Q8_0, 32, 1, w2, x))
    # byte length mismatch -> error
    with pytest.raises(L.ZgError):
        kern.try_execute(R.MatVecRegion(R.SourceIdentity(5), "t.q8short", synth.Q8_0, 32, 1, w[:33], x))
    # unbound identity cannot key a resident weight
    with pytest.raises(L.ZgError):
        kern.register(0, "t.unbound", synth.Q8_0, 32, 1, w)


@pytest.mark.parametrize("kind", KINDS)
def test_embedding_region_matches_codec(kern, kind):
    rng = np.random.default_rng(3)
    V, H = 1000, 1024 if kind == synth.Q8_0 else 2048
    w = synth.random_matrix(rng, kind, V, H)
    for sid in (0, 91):
        for token in (0, 17, V - 1):
            r = R.EmbeddingRegion(R.SourceIdentity(sid), "token_embd.weight", kind, w.reshape(-1), token, H, V)
            res = kern.try_embedding(r)
            ref = O.dequantize(kind, w[token], H)
            assert np.array_equal(res.values.view(np.uint32), ref.view(np.uint32))
    with pytest.raises(L.ZgError):
        kern.try_embedding(R.EmbeddingRegion(R.SourceIdentity(91), "token_embd.weight", kind, w.reshape(-1), V, H, V))


def test_pointwise_regions_match_oracle(kern):
    rng = np.random.default_rng(12)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    m = rng.standard_normal(2048).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    # RMS: bit-exact (same f32 rounding points; f64 sum of 2048 f32 squares)
    r = kern.try_rms_norm(R.RmsNormRegion(R.SourceIdentity(1), "n", x, np.ones(2048, np.float32), 1e-6))
    assert np.array_equal(r.values.view(np.uint32), O.rms_norm(x, np.ones(2048, np.float32), 1e-6).view(np.uint32))
    r = kern.try_grouped_rms_norm(R.GroupedRmsNormRegion(R.SourceIdentity(1), "g", x, g, 128, 16, 1e-6))
    assert np.array_equal(r.values.view(np.uint32), O.grouped_rms_norm(x, g, 16, 1e-6).view(np.uint32))
    # SiLU: polynomial exp with explicit FMAs -> bit-exact
    r = kern.try_silu(R.SiluRegion(R.SourceIdentity(1), "s", x, m))
    assert np.array_equal(r.values.view(np.uint32), O.silu(x, m).view(np.uint32))
    r = kern.try_silu(R.SiluRegion(R.SourceIdentity(1), "s", x))
    assert np.array_equal(r.values.view(np.uint32), O.silu(x).view(np.uint32))
    # Add bit-exact; SigmoidGate uses device expf (1e-6 relative)
    r = kern.try_binary(R.BinaryRegion(R.SourceIdentity(1), "a", 0, x, m))
    assert np.array_equal(r.values.view(np.uint32), O.binary(0, x, m).view(np.uint32))
    r = kern.try_binary(R.BinaryRegion(R.SourceIdentity(1), "b", 1, x, m))
    np.testing.assert_allclose(r.values, O.binary(1, x, m), rtol=2e-6, atol=1e-30)
