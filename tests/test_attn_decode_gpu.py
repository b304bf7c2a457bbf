"""GPU parity of the resident attention decode step (zg_attn_decode_device)
against the CPU oracle's attention_layer (oracle/zg_oracle.c, the schedule of
model-qwen35/src/forward.rs:634-755): head RMSNorm, RoPE at each row's
position, K/V append (rounded to the cache type), 32-accumulator scores,
8-lane softmax with f64 partials, padded 4x8-lane value chains and the
sigmoid gate.  The device restates each step's order of operations, so the
outputs and the appended K/V are required bit-identical, for a bf16 and an
f32 cache, caches of 2048 to 8192 rows (the reference qualifies contexts
through 8192 tokens, scripts/cpu-qualification-gate.py:5-6) and 3 or 32
rows at positions up to 8191."""
import math

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import _lib as L

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("exact_libm")]
D = 256


def bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def to_bf16_bits(x):
    return (bf16(x).view(np.uint32) >> 16).astype(np.uint16)


@pytest.fixture(scope="module")
def ctx():
    c = L.Context(0)
    yield c
    c.close()


LONG32 = [0, 2303, 3100, 4100, 8191] + [int(p) for p in np.linspace(17, 8180, 27)]


def _run_case(ctx, kv, max_ctx, positions, split):
    """Device attention decode of one case and the oracle's reference per row:
    returns (device output, reference outputs, appended-K/V checks done)."""
    import torch
    nq, nkv, eps = 8, 2, 1e-6
    theta = math.pow(1e7, -2.0 / 64.0)
    pos = np.array(positions, np.int32)
    B = pos.size
    rng = np.random.default_rng(41 + kv + max_ctx + B)
    stride = (2 * nq + 2 * nkv) * D + 8
    proj = rng.standard_normal((B, stride)).astype(np.float32)
    qn_w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn_w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kw = nkv * D
    hist_k = bf16(rng.standard_normal((B, max_ctx, kw), dtype=np.float32))
    hist_v = bf16(rng.standard_normal((B, max_ctx, kw), dtype=np.float32))
    if kv == L.BF16:
        kc = torch.from_numpy(to_bf16_bits(hist_k).view(np.int16)).cuda()
        vc = torch.from_numpy(to_bf16_bits(hist_v).view(np.int16)).cuda()
    else:
        kc, vc = torch.from_numpy(hist_k.copy()).cuda(), torch.from_numpy(hist_v.copy()).cuda()
    d_proj, d_pos = torch.from_numpy(proj).cuda(), torch.from_numpy(pos).cuda()
    d_qn, d_kn = torch.from_numpy(qn_w).cuda(), torch.from_numpy(kn_w).cuda()
    if split:
        nbytes = L.lib().zg_attn_decode_split_workspace_bytes(B, nq, nkv, max_ctx)
        assert nbytes > 0
        entry = L.lib().zg_attn_decode_split_device
    else:
        nbytes = L.lib().zg_attn_decode_workspace_bytes(B, nq, max_ctx)
        entry = L.lib().zg_attn_decode_device
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty((B, nq * D), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.check(entry(ctx.h, B, nq, nkv, d_proj.data_ptr(), stride, d_qn.data_ptr(), d_kn.data_ptr(), eps, theta,
                    d_pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), max_ctx, kv, ws.data_ptr(), out.data_ptr(), None))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if kv == L.BF16:
        kd = (kc.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        vd = (vc.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        kd, vd = kc.cpu().numpy(), vc.cpu().numpy()
    refs = []
    for b in range(B):
        p = int(pos[b])
        row = proj[b]
        rq = np.concatenate([row[h * 2 * D:h * 2 * D + D] for h in range(nq)])
        gates = np.concatenate([row[h * 2 * D + D:h * 2 * D + 2 * D] for h in range(nq)])
        k = row[2 * nq * D:2 * nq * D + kw]
        v = row[2 * nq * D + kw:2 * nq * D + 2 * kw]
        qn = O.grouped_rms_norm(rq, qn_w, nq, eps)
        kn = O.grouped_rms_norm(k, kn_w, nkv, eps)
        qr, kr = O.rope_kv(qn, kn, D, nq, nkv, 64, p, np.float32(theta))
        if kv == L.BF16:
            kr, v = bf16(kr), bf16(v)
        keys = np.concatenate([hist_k[b, :p], kr[None, :]])
        vals = np.concatenate([hist_v[b, :p], v[None, :]])
        _, scores = O.attention_qk(qr, keys, D, nq, nkv, 1.0 / 16.0)
        probs, _, _ = O.attention_softmax(scores, nq, p + 1)
        refs.append(O.binary(1, O.attention_value(probs, vals, D, nq, nkv), gates))
        # K/V appended exactly in both forms, the history untouched
        assert np.array_equal(kd[b, p].view(np.uint32), kr.view(np.uint32)), b
        assert np.array_equal(vd[b, p].view(np.uint32), v.view(np.uint32)), b
        assert np.array_equal(kd[b, :p].view(np.uint32), hist_k[b, :p].view(np.uint32))
        assert np.array_equal(vd[b, :p].view(np.uint32), hist_v[b, :p].view(np.uint32))
    return got, refs


# Each case reaches one branch of the device kernels: a cache of <= 2304
# rows (one 72 x 32 value tile), of <= 3072 (one 96 x 32 tile), beyond
# (tiled values with the softmax statistics computed ahead), beyond 4096
# (statistics over several score spans), and 8 rows or more (a statistics
# launch, then 4 query heads x 16 channels per workgroup).
@pytest.mark.parametrize("kv,max_ctx,positions", [
    (L.BF16, 2048, [0, 299, 2047]),
    (L.F32, 2048, [0, 299, 2047]),
    (L.BF16, 3072, [0, 2303, 3071]),
    (L.BF16, 4096, [0, 2303, 3100]),
    (L.BF16, 8192, [4100, 8191, 2303]),
    (L.F32, 8192, [8191, 4100, 0]),
    (L.BF16, 8192, LONG32),
    (L.BF16, 2048, [int(p) for p in np.linspace(0, 2047, 32)]),
])
def test_attn_decode_device_matches_oracle(ctx, kv, max_ctx, positions):
    got, refs = _run_case(ctx, kv, max_ctx, positions, split=False)
    for b, ref in enumerate(refs):
        assert np.array_equal(got[b].view(np.uint32), ref.view(np.uint32)), (b, float(np.abs(got[b] - ref).max()))


# The split-T form (1..64 rows): spans of a fixed token count per launch
# (32 at one row and a 2k cache, up to 1024), the owner of the position
# among them; spans of one token block and of many, the position at a span's
# first and last token, spans past a row's tokens (rows at different
# positions), caches up to 8192 rows.  The output is held to the per-op
# bar, 1e-3 relative to the row's largest magnitude.
SPLIT_REL = 1e-3


@pytest.mark.parametrize("kv,max_ctx,positions", [
    (L.BF16, 2048, [0]),
    (L.BF16, 2048, [2047]),
    (L.BF16, 2048, [2047, 700]),  # two rows over 64 spans each: the quarter-channel combine
    (L.F32, 2048, [31, 32, 63, 64]),
    (L.BF16, 4096, [2047, 2048, 5, 4095]),
    (L.BF16, 8192, [8191, 4100, 1023]),
    (L.F32, 8192, [6000]),
    (L.BF16, 300, [299, 150]),
    (L.BF16, 4096, [int(p) for p in np.linspace(0, 4095, 8)]),
    (L.BF16, 2304, [int(p) for p in np.linspace(17, 2303, 32)]),
    (L.F32, 8192, LONG32),
])
def test_attn_decode_split_matches_oracle(ctx, kv, max_ctx, positions):
    got, refs = _run_case(ctx, kv, max_ctx, positions, split=True)
    for b, ref in enumerate(refs):
        err = float(np.max(np.abs(got[b].astype(np.float64) - ref)) / np.max(np.abs(ref)))
        assert err <= SPLIT_REL, (b, positions[b], err)
    print(f"split attention kv={kv} max_ctx={max_ctx}: worst rel {max(float(np.max(np.abs(got[b] - r)) / np.max(np.abs(r))) for b, r in enumerate(refs)):.2e}")


def _refusal_buffers(rows, q_heads, kv_heads, max_ctx):
    """Device buffers as large as a launch with these arguments would touch
    (f32 caches cover bf16 too), so a refusal test whose host check
    regressed reads and writes in bounds and fails instead of faulting."""
    import torch
    stride = 2 * q_heads * 256 + 2 * kv_heads * 256
    bufs = dict(proj=torch.zeros(rows * stride, dtype=torch.float32, device="cuda"),
                qn=torch.zeros(256, dtype=torch.float32, device="cuda"),
                kn=torch.zeros(256, dtype=torch.float32, device="cuda"),
                pos=torch.zeros(rows, dtype=torch.int32, device="cuda"),
                kc=torch.zeros(rows * max(max_ctx, 1) * kv_heads * 256, dtype=torch.float32, device="cuda"),
                vc=torch.zeros(rows * max(max_ctx, 1) * kv_heads * 256, dtype=torch.float32, device="cuda"),
                ws=torch.zeros(64 << 20, dtype=torch.uint8, device="cuda"),
                out=torch.zeros(rows * q_heads * 256, dtype=torch.float32, device="cuda"))
    torch.cuda.synchronize()
    return stride, bufs


def test_attn_decode_split_refuses_more_than_64_rows(ctx):
    assert L.lib().zg_attn_decode_split_workspace_bytes(65, 8, 2, 2048) == 0
    stride, b = _refusal_buffers(65, 8, 2, 64)
    rc = L.lib().zg_attn_decode_split_device(ctx.h, 65, 8, 2, b["proj"].data_ptr(), stride, b["qn"].data_ptr(),
                                             b["kn"].data_ptr(), 1e-6, 0.6, b["pos"].data_ptr(), b["kc"].data_ptr(),
                                             b["vc"].data_ptr(), 64, L.BF16, b["ws"].data_ptr(),
                                             b["out"].data_ptr(), None)
    assert rc == L.E_LIMIT


def test_attn_decode_device_refusals(ctx):
    for bad in (dict(q_heads=6, kv_heads=4), dict(q_heads=10, kv_heads=2), dict(max_ctx=0), dict(kv_dtype=8)):
        args = dict(q_heads=8, kv_heads=2, max_ctx=64, kv_dtype=L.BF16)
        args.update(bad)
        stride, b = _refusal_buffers(1, args["q_heads"], args["kv_heads"], args["max_ctx"])
        rc = L.lib().zg_attn_decode_device(ctx.h, 1, args["q_heads"], args["kv_heads"], b["proj"].data_ptr(), stride,
                                           b["qn"].data_ptr(), b["kn"].data_ptr(), 1e-6, 0.6, b["pos"].data_ptr(),
                                           b["kc"].data_ptr(), b["vc"].data_ptr(), args["max_ctx"],
                                           args["kv_dtype"], b["ws"].data_ptr(), b["out"].data_ptr(), None)
        assert rc == L.E_MALFORMED, bad
