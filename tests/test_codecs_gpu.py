"""GPU parity of the other GGUF codecs of the published checkpoints --
Q4_1 x Q8_1, Q6_K x Q8_K and the F32 4x8-lane dot -- against the CPU
oracle, which restates cpu/src/source/quantization.rs:198-285 and
cpu/src/source.rs:325-366 and is pinned by the reference's fixtures in
test_oracle_kat.py.

All three are integer block dots (or an f32 FMA schedule) whose rounding
points the device reproduces: the activation is coded in-kernel exactly as
QuantizedActivation::prepare codes it (Q8_1: f16 d and s; Q8_K: first
signed maximum, d = 1/inv, 16-element code sums), each lane keeps the
reference's integer accumulator and FMA lane, and the lane tree is the
reference's.  Dequantization, GEMV (plain and with the RMS prologue, 1-32
rows), embedding rows and whole-model logits are therefore required
bit-identical to the oracle, for one row and for batched rows.  A model
mixing these codecs with Q4_K is checked for identical greedy tokens (see
that test for why its logits are not held to bits or to 2e-2).
"""
import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L
from zerogravity_amd import gguf, qwen35
from zerogravity_amd import regions as R
from zerogravity_amd import synth

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]
KINDS = [synth.Q4_1, synth.Q6_K, synth.F32]


@pytest.fixture(scope="module")
def kern():
    k = R.HipMatVecKernel(0)
    yield k
    k.ctx.close()


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    torch.cuda.set_stream(torch.cuda.Stream())
    return torch


_weights = {}


def weight(kern, kind, N, K):
    key = (kind, N, K)
    if key not in _weights:
        rng = np.random.default_rng(N * 7 + K + kind)
        w = synth.random_matrix(rng, kind, N, K)
        _weights[key] = (w, kern.register(88, f"c.{kind}.{N}.{K}", kind, K, N, w))
    return _weights[key]


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", [(16, 2048), (301, 1024), (2048, 6144)])
def test_dequantize_bit_exact(kern, kind, N, K):
    w, h = weight(kern, kind, N, K)
    ref = O.dequantize(kind, w.reshape(-1), N * K).reshape(N, K)
    assert same_bits(h.dequantize(), ref)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", [(16, 2048), (301, 1024), (2048, 6144), (1024, 4096)])
def test_matvec_region_bit_exact(kern, kind, N, K):
    w, _ = weight(kern, kind, N, K)
    x = np.random.default_rng(N + K).standard_normal(K).astype(np.float32)
    region = R.MatVecRegion(R.SourceIdentity(88), f"c.{kind}.{N}.{K}", kind, K, N, w.reshape(-1), x)
    res = kern.try_execute(region)
    assert isinstance(res, R.Completed)
    assert same_bits(res.values, O.matvec(kind, w.reshape(-1), N, K, x))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("N,K", [(32, 2048), (2048, 6144), (5000, 1024)])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 32])
def test_gemv_device_rms_prologue_bit_exact(kern, torch_cuda, kind, N, K, M):
    torch = torch_cuda
    w, h = weight(kern, kind, N, K)
    rng = np.random.default_rng(M * 13 + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, 5] = 0.0
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d, g_d = torch.from_numpy(x).cuda(), torch.from_numpy(gamma).cuda()
    y_d = torch.empty((M, N), dtype=torch.float32, device="cuda")
    kern.ctx.check(L.lib().zg_gemv_device(kern.ctx.h, h.h, x_d.data_ptr(), L.F32, M, g_d.data_ptr(), 1e-6,
                                          y_d.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    y = y_d.cpu().numpy()
    for m in range(M):
        ref = O.matvec(kind, w.reshape(-1), N, K, O.rms_norm(x[m], gamma, 1e-6))
        assert same_bits(y[m], ref), (m, float(np.max(np.abs(y[m] - ref))))


@pytest.mark.parametrize("N,K,M", [(777, 512, 17), (3001, 1536, 33), (64, 8192, 6)])
def test_q6k_staged_rows_bit_exact(kern, torch_cuda, N, K, M):
    """Q6_K beyond 4 rows: each activation row coded once, then up to 16
    staged rows per workgroup; N not a multiple of 8 (a last row group past
    N), a partial last group of activation rows, K = 8192 (four rows per
    workgroup, the LDS bound): bit-exact against the oracle."""
    torch = torch_cuda
    w, h = weight(kern, synth.Q6_K, N, K)
    rng = np.random.default_rng(M * 17 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d, g_d = torch.from_numpy(x).cuda(), torch.from_numpy(gamma).cuda()
    y_d = torch.full((M, N), np.nan, dtype=torch.float32, device="cuda")
    kern.ctx.check(L.lib().zg_gemv_device(kern.ctx.h, h.h, x_d.data_ptr(), L.F32, M, g_d.data_ptr(), 1e-6,
                                          y_d.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    y = y_d.cpu().numpy()
    for m in range(M):
        ref = O.matvec(synth.Q6_K, w.reshape(-1), N, K, O.rms_norm(x[m], gamma, 1e-6))
        assert same_bits(y[m], ref), (m, float(np.max(np.abs(y[m] - ref))))


def test_q8_k_coding_edge_blocks_bit_exact(kern):
    # an all-zero superblock (d = 0), a block whose largest magnitude appears
    # twice with opposite signs (the first wins), and ties at the rounding
    # midpoint, through the Q6_K region against the oracle
    K, N = 1024, 24
    w, _ = weight(kern, synth.Q6_K, N, K)
    x = np.random.default_rng(4).standard_normal(K).astype(np.float32)
    x[:256] = 0.0
    x[256 + 10], x[256 + 200] = -3.0, 3.0
    x[512:768] = np.linspace(-2.5, 2.5, 256).astype(np.float32)
    res = kern.try_execute(R.MatVecRegion(R.SourceIdentity(88), f"c.{synth.Q6_K}.{N}.{K}", synth.Q6_K, K, N,
                                          w.reshape(-1), x))
    assert same_bits(res.values, O.matvec(synth.Q6_K, w.reshape(-1), N, K, x))


@pytest.mark.parametrize("kind", [synth.Q4_1, synth.Q6_K])
def test_embedding_rows_bit_exact(kern, kind):
    rng = np.random.default_rng(9)
    V, H = 1000, 2048
    w = synth.random_matrix(rng, kind, V, H)
    for token in (0, 17, V - 1):
        res = kern.try_embedding(R.EmbeddingRegion(R.SourceIdentity(93), "token_embd.weight", kind, w.reshape(-1),
                                                   token, H, V))
        assert same_bits(res.values, O.dequantize(kind, w[token], H))


TINY = dict(hidden=256, layers=4, ffn=512, vocab=1000, gdn_heads=2, gdn_dim=128, q_heads=2, kv_heads=1,
            head_dim=256, full_attention_interval=4, max_context=4096, eps=1e-6)


@pytest.mark.parametrize("kv", [L.F32, L.BF16])
def test_mixed_integer_codec_model_bit_exact(kern, kv):
    """Q8_0 projections with the Q6_K embedding / value / down projections,
    Q4_1 output gate and F32 alpha/beta (each stack split into runs of one
    codec): every projection is an integer block dot or the F32 schedule, so
    the logits equal the oracle's bit for bit over 16 greedy steps."""
    t = qwen35.synthetic_tensors(TINY, gguf.Q8_0, seed=31, kinds=qwen35.MIXED)
    m = qwen35.QwenModelHip(TINY, t, kernel=kern)
    s = m.session(max_batch=1, max_context=64, kv_dtype=kv)
    o = O.Model(TINY, t).session(kv_bf16=kv == L.BF16)
    tok = 3
    for step in range(16):
        lg = s.forward(tok)
        ref = o.forward(tok)
        assert same_bits(lg, ref), (step, float(np.max(np.abs(lg - ref))))
        tok = int(np.argmax(ref))
    m.close()


def test_mixed_integer_codec_batched_rows_bit_exact(kern):
    """The same mixed-codec model at B = 6 (every projection on the fused
    kernels, stacks split by codec): each row equals its own oracle session
    bit for bit."""
    t = qwen35.synthetic_tensors(TINY, gguf.Q8_0, seed=33, kinds=qwen35.MIXED)
    m = qwen35.QwenModelHip(TINY, t, kernel=kern)
    B, steps = 6, 4
    s = m.session(max_batch=B, max_context=64, kv_dtype=L.BF16)
    toks = np.random.default_rng(6).integers(0, TINY["vocab"], (steps, B)).astype(np.uint32)
    got = [s.step(toks[i])[0] for i in range(steps)]
    for b in (0, 3, 5):
        o = O.Model(TINY, t).session(kv_bf16=True)
        for i in range(steps):
            assert same_bits(got[i][b], o.forward(int(toks[i, b]))), (b, i)
    m.close()


def test_q8_model_wide_batch_bit_exact(kern):
    """An all-Q8_0 model at B = 33: every projection takes the coded-once
    activation and the Q8_0 rows kernels (the 4096-row LM head the int8
    matrix-core one, 256 tiles at 32+ rows; the narrower projections the
    v_dot4 one), in the step's own prologue forms (RMS, gated RMS, SiLU
    product) and epilogues; rows at either end and in the middle equal their
    own oracle sessions bit for bit."""
    g = dict(TINY, vocab=4096)
    t = qwen35.synthetic_tensors(g, gguf.Q8_0, seed=34)
    m = qwen35.QwenModelHip(g, t, kernel=kern)
    B, steps = 33, 3
    s = m.session(max_batch=B, max_context=64, kv_dtype=L.BF16)
    toks = np.random.default_rng(8).integers(0, g["vocab"], (steps, B)).astype(np.uint32)
    got = [s.step(toks[i])[0] for i in range(steps)]
    for b in (0, 16, 32):
        o = O.Model(g, t).session(kv_bf16=True)
        for i in range(steps):
            ref = o.forward(int(toks[i, b]))
            assert same_bits(got[i][b], ref), (b, i, float(np.max(np.abs(got[i][b] - ref))))
    m.close()


@pytest.mark.parametrize("B", [3, 6])
def test_mixed_q4k_model_greedy_matches_oracle(kern, B):
    """Q4_K projections beside the integer codecs, at B = 1 and B = 3 or 6
    (from two rows the Q4_K runs of each stack take the batched MFMA path,
    the integer codecs the fused kernels at up to 4 rows).  Q4_K is held to
    1e-3 per op, and its small differences move some downstream Q8_1/Q8_K
    activation codes across a rounding boundary, so the logits are not held
    to bits here; the greedy tokens must agree.  The reference's pinned
    checkpoints hold no Q4_K (cpu/src/source/quantization.rs:296)."""
    g = dict(TINY, hidden=512, ffn=512)
    t = qwen35.synthetic_tensors(g, gguf.Q4_K, seed=32, kinds=qwen35.MIXED)
    m = qwen35.QwenModelHip(g, t, kernel=kern)
    steps = 5
    s = m.session(max_batch=B, max_context=64, kv_dtype=L.BF16)
    one = m.session(max_batch=1, max_context=64, kv_dtype=L.BF16)
    toks = np.random.default_rng(5).integers(0, g["vocab"], (steps, B)).astype(np.uint32)
    got = [s.step(toks[i])[0] for i in range(steps)]
    worst = 0.0
    for b in (0, B - 1):
        o = O.Model(g, t).session(kv_bf16=True)
        for i in range(steps):
            ref = o.forward(int(toks[i, b]))
            assert int(np.argmax(got[i][b])) == int(np.argmax(ref)), (b, i)
            worst = max(worst, float(np.max(np.abs(got[i][b] - ref))))
            if b == 0:
                assert int(np.argmax(one.forward(int(toks[i, 0])))) == int(np.argmax(ref)), i
    print(f"mixed-codec Q4_K model B={B}: greedy identical, worst logit max-abs {worst:.3e}")
    with pytest.raises(L.ZgError) as e:
        one.prefill_batched(np.zeros(4, np.uint32))
    assert e.value.code == L.E_UNSUPPORTED
    m.close()


def test_mixed_codec_gguf_file_round_trip_decodes_bit_exact(kern, tmp_path):
    """The mixed-codec model written as a GGUF v3 file (artifact.rs:539-672
    layout) and read back through the reader loads on the device and decodes
    bit-identically to the oracle built from the file's own tensor table."""
    t = qwen35.synthetic_tensors(TINY, gguf.Q8_0, seed=34, kinds=qwen35.MIXED)
    path = str(tmp_path / "mixed.gguf")
    qwen35.write_gguf(path, TINY, t)
    g, tf, f = qwen35.read_gguf(path)
    assert {n: v[0] for n, v in tf.items()} == {n: v[0] for n, v in t.items()}
    m = qwen35.QwenModelHip(g, tf, kernel=kern)
    s = m.session(max_batch=1, max_context=64, kv_dtype=L.BF16)
    o = O.Model(g, tf).session(kv_bf16=True)
    prompt = np.random.default_rng(8).integers(0, g["vocab"], 6)
    lg = s.prefill_transaction(prompt)
    for tok in prompt[:-1]:
        o.forward(int(tok), need_logits=False)
    ref = o.forward(int(prompt[-1]))
    for step in range(6):
        assert same_bits(lg, ref), step
        tok = int(np.argmax(ref))
        lg, ref = s.forward(tok), o.forward(tok)
    m.close()
    del f
