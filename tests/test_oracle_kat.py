"""Pins the CPU oracle (oracle/zg_oracle.c) to the reference's own known-answer
tests and to closed forms the mathematics fixes.  Each test cites the
reference test it restates (zerogravity repository file:line).  CPU only.
"""
import math
import struct

import numpy as np
import pytest

import zg_oracle as O


def bits(x):
    return struct.unpack("<I", struct.pack("<f", np.float32(x)))[0]


def fbits(w):
    return struct.unpack("<f", struct.pack("<I", w))[0]


def le16(v):
    return [v & 0xFF, v >> 8]


# ----------------------------------------------------------------- codecs

def test_f16_specials_subnormal_and_normal():
    # artifacts/src/codecs/mod.rs:95-103
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0xBC00) == -1.0
    assert O.f16_to_f32(0x0001) == 2.0 ** -24
    assert O.f16_to_f32(0x7BFF) == 65504.0
    assert math.isinf(O.f16_to_f32(0x7C00))
    assert math.isnan(O.f16_to_f32(0x7E00))
    assert bits(O.f16_to_f32(0x8000)) == 0x80000000


def test_f16_decoder_matches_numpy_half_for_every_finite_code():
    # closed form: IEEE binary16 decode is fixed by the standard; numpy's
    # half is an independent implementation.  Covers all 63488 finite codes.
    codes = np.arange(1 << 16, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    ours = np.array([O.f16_to_f32(int(c)) for c in codes[finite]], np.float32)
    assert np.array_equal(ours.view(np.uint32), ref[finite].view(np.uint32))


def test_f16_rne_table():
    # codecs/mod.rs:243-261
    cases = [(0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-1.0, 0xBC00), (65504.0, 0x7BFF),
             (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000), (1.0 + 2.0 ** -11, 0x3C00),
             (1.0 + 3.0 * 2.0 ** -11, 0x3C02), (float("inf"), 0x7C00)]
    for x, raw in cases:
        assert O.f32_to_f16(x) == raw, x
    assert O.f32_to_f16(-(2.0 ** -24)) == 0x8001
    assert math.isnan(O.f16_to_f32(O.f32_to_f16(float("nan"))))


def test_f16_rne_matches_numpy_on_random_floats():
    # closed form: numpy's float32->float16 cast is IEEE round-to-nearest-even
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10 ** rng.uniform(-8, 5, 4000).astype(np.float32),
                        np.float32([6.1e-5, 6.0e-8, 3.0e-8, 65519.0, 65520.0])]).astype(np.float32)
    ours = np.array([O.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))


def test_dequantize_floats_and_blocks():
    # codecs/mod.rs:106-166
    q8 = bytes([0x00, 0x3C, 0x80, 0x7F] + [0] * 30)
    assert list(O.dequantize(O.Q8_0, q8, 32)[:2]) == [-128.0, 127.0]
    q4 = bytes([0x00, 0x3C] + [0x80] * 16)
    v = O.dequantize(O.Q4_0, q4, 32)
    assert list(v[:16]) == [-8.0] * 16 and list(v[16:]) == [0.0] * 16
    q4k = bytearray(144)
    q4k[0:2] = bytes(le16(0x3C00))
    q4k[2:4] = bytes(le16(0x3800))
    q4k[4] = 2
    q4k[8] = 4
    q4k[16:48] = bytes([0x53] * 32)
    d = O.dequantize(O.Q4_K, bytes(q4k), 256)
    assert list(d[:32]) == [4.0] * 32
    assert list(d[32:64]) == [0.0] * 32
    q4k[4] = 0b0100_0000
    q4k[8] = 0b1000_0000
    q4k[12] = 0b0010_0110
    q4k[80:112] = bytes([0x33] * 32)
    d = O.dequantize(O.Q4_K, bytes(q4k), 256)
    assert list(d[128:160]) == [49.0] * 32


def test_q4_k_groups_scale_two_min_three():
    # cpu/src/source.rs:605-619
    p = bytearray(144)
    p[0:2] = bytes(le16(0x3C00))
    p[2:4] = bytes(le16(0x3800))
    p[4:8] = bytes([2] * 4)
    p[8:12] = bytes([3] * 4)
    p[12:16] = bytes([0x32] * 4)
    p[16:] = bytes([0x51] * 128)
    d = O.dequantize(O.Q4_K, bytes(p), 256)
    for g in range(8):
        want = 0.5 if g % 2 == 0 else 8.5
        assert all(bits(v) == bits(want) for v in d[g * 32:(g + 1) * 32])


def test_exact_special_value_bits():
    # codecs/exact_tests.rs:5-62
    words = [0, 0x80000000, 1, 0x7F800000, 0xFF800000, 0x7FC12345]
    raw = b"".join(struct.pack("<I", w) for w in words)
    assert list(O.dequantize(O.F32, raw, len(words)).view(np.uint32)) == words
    b16 = [0, 0x8000, 1, 0x7F80, 0xFF80, 0x7FC1, 0xFF81]
    raw = b"".join(struct.pack("<H", w) for w in b16)
    assert list(O.dequantize(O.BF16, raw, len(b16)).view(np.uint32)) == [w << 16 for w in b16]
    h16 = [0, 0x8000, 1, 0x7C00, 0xFC00, 0x7E01, 0xFC01]
    raw = b"".join(struct.pack("<H", w) for w in h16)
    assert list(O.dequantize(O.F16, raw, len(h16)).view(np.uint32)) == [
        0, 0x80000000, 0x33800000, 0x7F800000, 0xFF800000, 0x7FC02000, 0xFF802000]


def test_q4_1_offset_and_q6_k_signed_scales():
    # codecs/exact_tests.rs:64-87
    q4 = bytearray([0xF2] * 20)
    q4[0:2] = bytes(le16(0x3800))
    q4[2:4] = bytes(le16(0xBC00))
    d = O.dequantize(O.Q4_1, bytes(q4), 32)
    assert list(d[:16]) == [0.0] * 16 and list(d[16:]) == [6.5] * 16
    q6 = bytearray(210)
    q6[:128] = bytes([0x21] * 128)
    q6[128:192] = bytes([0xE4] * 64)
    for half in range(2):
        q6[192 + half * 8:200 + half * 8] = bytes([1, 255, 2, 254, 3, 253, 4, 252])
    q6[208:] = bytes(le16(0x3C00))
    d = O.dequantize(O.Q6_K, bytes(q6), 256)
    expected = [-31.0, 31.0, -30.0, 30.0, 6.0, -6.0, 72.0, -72.0]
    for half in range(2):
        for lane in range(8):
            assert list(d[half * 128 + lane * 16: half * 128 + lane * 16 + 16]) == [expected[lane]] * 16


@pytest.mark.parametrize("t", [O.F32, O.F16, O.BF16, O.Q4_0, O.Q4_1, O.Q4_K, O.Q6_K, O.Q8_0])
def test_every_codec_rejects_truncated_and_excess_bytes(t):
    # codecs/exact_tests.rs:89-116
    elements, nbytes = O.BLOCK[t]
    for length in [0, nbytes - 1, nbytes + 1]:
        with pytest.raises(O.OracleError):
            O.dequantize(t, np.zeros(length, np.uint8), elements)
    assert O.dequantize(t, np.zeros(nbytes, np.uint8), elements).size == elements


@pytest.mark.parametrize("t,offsets", [(O.Q4_0, [0]), (O.Q4_1, [0, 2]), (O.Q4_K, [0, 2]),
                                       (O.Q6_K, [208]), (O.Q8_0, [0])])
def test_every_quantized_scale_rejects_nonfinite(t, offsets):
    # codecs/exact_tests.rs:118-140
    elements, nbytes = O.BLOCK[t]
    for off in offsets:
        for b in [0x7C00, 0xFC00, 0x7E01]:
            data = np.zeros(nbytes, np.uint8)
            data[off:off + 2] = le16(b)
            with pytest.raises(O.OracleError):
                O.dequantize(t, data, elements)


def test_q4_k_decode_matches_independent_numpy_restatement():
    # closed form of the GGML Q4_K layout on random blocks (scales, mins and
    # nibbles all exercised) against an independent vectorised decoder.
    rng = np.random.default_rng(3)
    nb = 64
    blocks = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    blocks[:, 0:2] = np.frombuffer(np.float16(rng.standard_normal(nb) * 0.01).tobytes(), np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = np.frombuffer(np.float16(np.abs(rng.standard_normal(nb)) * 0.01).tobytes(), np.uint8).reshape(nb, 2)
    ours = O.dequantize(O.Q4_K, blocks.reshape(-1), nb * 256).reshape(nb, 256)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nb)
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(nb)
    s = blocks[:, 4:16].astype(np.int32)
    sc = np.zeros((nb, 8), np.int32)
    mn = np.zeros((nb, 8), np.int32)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = blocks[:, 16:].reshape(nb, 4, 32)
    q = np.zeros((nb, 8, 32), np.int32)
    q[:, 0::2] = qs & 15
    q[:, 1::2] = qs >> 4
    scale = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    mins = (dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
    ref = (scale[:, :, None] * q.astype(np.float32)).astype(np.float32) - mins[:, :, None]
    assert np.array_equal(ours.view(np.uint32), ref.reshape(nb, 256).astype(np.float32).view(np.uint32))


# --------------------------------------------------------- activation coding

def test_small_activation_keeps_ties_even_half_scales_and_zero():
    # cpu/src/source/quantization.rs:318-365
    x = np.zeros(32, np.float32)
    x[:7] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    qs, d, s = O.q8_activation(x)
    assert bits(d[0]) == bits(1.0) and bits(s[0]) == bits(127.0)
    assert list(qs[:7]) == [127, 0, 2, 2, 0, -2, -2] and not qs[7:].any()
    qs, d, s = O.q8_activation(np.ones(32, np.float32))
    assert bits(d[0]) == 0x3C010000 and bits(s[0]) == bits(32.0) and (qs == 127).all()
    for zero in (0.0, -0.0):
        qs, d, s = O.q8_activation(np.full(32, zero, np.float32))
        assert bits(d[0]) == 0 and bits(s[0]) == 0 and not qs.any()


def test_activation_rejects_misaligned_or_nonfinite_inputs():
    # quantization.rs:402-433
    with pytest.raises(O.OracleError):
        O.q8_activation(np.zeros(31, np.float32))
    for v in (np.nan, np.inf, -np.inf):
        with pytest.raises(O.OracleError):
            O.q8_activation(np.full(32, v, np.float32))


def test_q8_0_block_dot_hand_computed_fixture():
    # quantization.rs:436-494: d=0.5, codes (-3, 2), x = 127 -> -1016.0 exactly
    row = np.zeros(34, np.uint8)
    row[0:2] = le16(0x3800)
    row[2::2] = np.uint8(256 - 3)
    row[3::2] = 2
    assert bits(O.dot_q8_0_row(row, np.full(32, 127.0, np.float32))) == bits(-1016.0)


def test_q8_0_row_dot_matches_exact_integer_closed_form():
    # closed form: sum_b f16(w_d) * d_act * sum_i w_i q_i in f64.  A dropped
    # block, wrong code index or wrong scale breaks the 1e-6 bound.
    rng = np.random.default_rng(11)
    K, rows = 1024, 40
    w = rng.integers(0, 256, size=(rows, K // 32, 34), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(rng.uniform(0.001, 0.01, rows * K // 32)).tobytes(), np.uint8).reshape(rows, K // 32, 2)
    x = rng.standard_normal(K).astype(np.float32)
    qs, d, _ = O.q8_activation(x)
    y = O.matvec(O.Q8_0, w.reshape(-1), rows, K, x)
    wd = w[:, :, 0:2].copy().view(np.float16).astype(np.float64).reshape(rows, K // 32)
    wq = w[:, :, 2:].view(np.int8).astype(np.int64)
    isum = (wq * qs.reshape(K // 32, 32).astype(np.int64)).sum(-1)
    scale = (wd.astype(np.float32) * d[None, :]).astype(np.float64)
    ref = (isum * scale).sum(-1)
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6 * np.abs(ref).max())


def test_q4_k_row_dot_within_reference_bound_and_f64_closed_form():
    # cpu/src/source.rs:641-679 (|dot - dequant.x| < 0.05) plus an f64 closed
    # form over the (bit-exact) decoded weights on random rows.
    row = np.zeros(144, np.uint8)
    x = np.array([(i % 17) - 8.0 for i in range(256)], np.float32)
    dec = O.dequantize(O.Q4_K, row, 256)
    assert abs(O.dot_q4k_row(row, x) - float((dec * x).sum())) < 0.05
    rng = np.random.default_rng(5)
    rows, K = 24, 2048
    w = rng.integers(0, 256, size=(rows, K // 256, 144), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(rng.uniform(1e-3, 4e-3, rows * K // 256)).tobytes(), np.uint8).reshape(rows, -1, 2)
    w[:, :, 2:4] = np.frombuffer(np.float16(rng.uniform(1e-3, 4e-3, rows * K // 256)).tobytes(), np.uint8).reshape(rows, -1, 2)
    x = rng.standard_normal(K).astype(np.float32)
    y = O.matvec(O.Q4_K, w.reshape(-1), rows, K, x)
    dec = O.dequantize(O.Q4_K, w.reshape(-1), rows * K).reshape(rows, K).astype(np.float64)
    ref = dec @ x.astype(np.float64)
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-5 * np.abs(ref).max())


def test_q8_k_keeps_first_signed_maximum_and_zero():
    # quantization.rs:367-400: the first element of largest magnitude sets
    # the signed scale; an all-zero block gives d = 0 and zero codes
    for first, scale, code in ((127.0, -1.0, -2), (-127.0, 1.0, 2)):
        x = np.zeros(256, np.float32)
        x[:4] = [first, -first, 0.5, 1.5]
        qs, d, bs = O.q8k_activation(x)
        assert bits(d[0]) == bits(scale)
        assert list(qs[:4]) == [-127, 127, 0, code] and not qs[4:].any()
        assert bs[0] == code and not bs[1:].any()
    for zero in (0.0, -0.0):
        qs, d, _ = O.q8k_activation(np.full(256, zero, np.float32))
        assert bits(d[0]) == 0 and not qs.any()
    with pytest.raises(O.OracleError):
        O.q8k_activation(np.zeros(255, np.float32))
    for v in (np.nan, np.inf):
        with pytest.raises(O.OracleError):
            O.q8k_activation(np.full(256, v, np.float32))


def test_source_exact_blocks_match_hand_computed_integer_fixtures():
    # quantization.rs:436-494: x = 127 everywhere, one block per codec
    x32 = np.full(32, 127.0, np.float32)
    q4_0 = np.array(le16(0x3C00) + [0xA9] * 16, np.uint8)  # 16 ones + 16 twos
    assert bits(O.dot_q4_0_row(q4_0, x32)) == bits(6096.0)
    assert bits(O.dot_q4_0_row(q4_0, x32, repacked=True)) == bits(6096.0)
    q4_1 = np.array(le16(0x3800) + le16(0xBC00) + [0x32] * 16, np.uint8)  # d=1/2, m=-1
    assert bits(O.dot_q4_1_row(q4_1, x32)) == bits(1016.0)
    q6 = np.zeros(210, np.uint8)
    q6[:128] = 0x21
    q6[128:192] = 0xAA  # codes 33/34 before the -32 shift
    q6[192:208] = 255  # local scales -1
    q6[208:] = le16(0x3800)
    assert bits(O.dot_q6k_row(q6, np.full(256, 127.0, np.float32))) == bits(-24384.0)


def test_q4_0_repacked_block_order_stays_distinct_from_eight_lane_reduction():
    # quantization.rs:497-531: block sums 2^24, 1, -2^24; the repacked
    # schedule loses the 1, the eight-lane one keeps it
    x = np.zeros(96, np.float32)
    x[31::32] = 127.0
    x[0], x[36], x[64] = -64.0, 1.0, 64.0
    row = np.full(54, 0x88, np.uint8)
    for b in range(3):
        row[18 * b:18 * b + 2] = le16(0x7800)
        row[18 * b + 2] = 0x80
    row[18:20] = le16(0x3C00)
    row[20] = 0x88
    row[24] = 0x89
    assert bits(O.dot_q4_0_row(row, x, repacked=True)) == 0
    assert bits(O.dot_q4_0_row(row, x)) == bits(1.0)


def test_q6_k_lane_of_an_element_is_its_position_mod_32_over_4():
    # Three superblocks whose lane-0 sums are 2^25, -32 (offset) and -2^25,
    # with a +1 that the reference puts in lane 1 (element 4: (4 % 32) / 4).
    # Lane 0 at 2^25 has spacing 2, so a layout that put element 4 in lane 0
    # (contiguous 32-groups) would lose it: -31 against -32.
    x = np.zeros(768, np.float32)
    row = np.zeros(3 * 210, np.uint8)
    for b, (probe_at, probe_x, dw, s0) in enumerate(((1, -1.0, 0xF000, 0x80), (4, -1.0, 0xBC00, 1),
                                                     (1, 1.0, 0xF000, 0x80))):
        blk = row[210 * b:210 * (b + 1)]
        x[256 * b] = 127.0  # the block maximum: d_a = -1, code 32, no net term
        x[256 * b + probe_at] = probe_x
        blk[:128] = 0x00
        blk[128:192] = 0xAA  # high bits 2 for every group: code 32 where the nibble is 0
        blk[192:208] = 1
        blk[192] = s0
        blk[208:210] = le16(dw)
        # element `probe_at` (< 32: half 0, group 0, low nibble of ql[probe_at], high bits qh[probe_at] & 3)
        code = 0 if b != 1 else 1
        blk[probe_at] = code & 15
        blk[128 + probe_at] = (0xAA & ~3) | (code >> 4)
    got = O.dot_q6k_row(row, x)
    assert bits(got) == bits(-31.0), got
    # the same rows through the matrix-vector entry
    assert bits(O.matvec(O.Q6_K, row, 1, 768, x)[0]) == bits(-31.0)


def test_q4_1_zero_points_accumulate_apart_from_the_lanes():
    # Lane 0 carries 2^24 then -2^24 while the zero points add m*s = 1 in
    # between: the reference adds the separate sum after the tree (result 1);
    # folding it into lane 0 would lose it at 2^24.
    x = np.zeros(96, np.float32)
    x[0:3] = [127.0, 127.0, 26.0]
    x[32:34] = [127.0, -126.0]
    x[64:67] = [-127.0, -127.0, -26.0]
    row = np.zeros(60, np.uint8)
    for b, (dw, m) in enumerate(((0x6C00, 0), (0x3C00, 0x3C00), (0x6C00, 0))):
        blk = row[20 * b:20 * (b + 1)]
        blk[0:2] = le16(dw)
        blk[2:4] = le16(m)
        if b != 1:
            blk[4:8] = [15, 15, 11, 0]
    assert bits(O.dot_q4_1_row(row, x)) == bits(1.0)


def test_f32_dot_four_by_eight_accumulators_and_tree():
    # source.rs:325-366: element 8 lands in accumulator (1, 0) and meets
    # elements 0 and 16 (accumulators (0, 0), (2, 0)) only in the tree:
    # (2^24 + -2^24) + 1 = 1, where a serial sum gives 0
    x = np.zeros(40, np.float32)
    x[0], x[8], x[16] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    x[33] = 3.0  # tail element past the last full 32-step, added serially
    w = np.ones(40, np.float32)
    w[33] = 0.5
    row = np.frombuffer(w.tobytes(), np.uint8)
    assert bits(O.dot_f32_row(row, x)) == bits(2.5)
    assert bits(O.matvec(O.F32, row, 1, 40, x)[0]) == bits(2.5)


@pytest.mark.parametrize("kind,K", [("Q4_0", 512), ("Q4_1", 512), ("Q6_K", 1024)])
def test_integer_block_dots_match_exact_integer_closed_form(kind, K):
    # f64 closed form over the decoded weights and the coded activation:
    # sum_b scale_b * sum_i w_i q_i (+ zero points).  A wrong nibble, high
    # bit, local scale or offset breaks the 1e-6 bound.
    rng = np.random.default_rng(hash(kind) % 1000)
    rows = 16
    t = getattr(O, kind)
    bb = {"Q4_0": 18, "Q4_1": 20, "Q6_K": 210}[kind]
    be = 256 if kind == "Q6_K" else 32
    w = rng.integers(0, 256, size=(rows, K // be, bb), dtype=np.uint8)
    hdr = {"Q4_0": [0], "Q4_1": [0, 2], "Q6_K": [208]}[kind]
    for o in hdr:
        w[:, :, o:o + 2] = np.frombuffer(np.float16(rng.uniform(-0.01, 0.01, rows * K // be)).tobytes(),
                                         np.uint8).reshape(rows, -1, 2)
    x = rng.standard_normal(K).astype(np.float32)
    y = O.matvec(t, w.reshape(-1), rows, K, x)
    dec = O.dequantize(t, w.reshape(-1), rows * K).reshape(rows, K).astype(np.float64)
    if kind == "Q6_K":
        qs, d, _ = O.q8k_activation(x)
        xa = (qs.reshape(-1, 256).astype(np.float64) * d[:, None]).reshape(-1)
    else:
        qs, d, s = O.q8_activation(x)
        xa = (qs.reshape(-1, 32).astype(np.float64) * d[:, None]).reshape(-1)
    ref = dec @ xa
    if kind == "Q4_1":
        # the zero point pairs with the f16-rounded s, not with sum(q) * f16(d)
        m = w[:, :, 2:4].copy().view(np.float16).astype(np.float64).reshape(rows, -1)
        qsum = qs.reshape(-1, 32).astype(np.float64).sum(-1)
        ref = ref - (m * (qsum * d)[None, :]).sum(-1) + (m * s[None, :]).sum(-1)
    np.testing.assert_allclose(y, ref, rtol=0, atol=1e-5 * np.abs(ref).max())


def test_q8_0_row_dot_within_reference_bound():
    # cpu/src/source.rs:641-679 for the Q8_0 codec (scale 1.0, zero codes)
    row = np.zeros(34, np.uint8)
    row[0:2] = le16(0x3C00)
    x = np.array([(i % 17) - 8.0 for i in range(32)], np.float32)
    assert abs(O.dot_q8_0_row(row, x)) < 0.05


# ------------------------------------------------------------------- norms

def test_rms_norm_closed_form():
    # cpu/src/ops.rs:157-159
    y = O.rms_norm([3.0, 4.0], [1.0, 1.0], 1e-6)
    assert abs(y[0] - 0.848528) < 1e-5 and abs(y[1] - 1.13137) < 1e-5


def _l2_reference(x, eps):
    # lib.rs:1509-1520 restated with numpy float32 arithmetic (test-only
    # two-stage L2 of the reference): f32 squares summed serially in f64.
    x = np.float32(x)
    n = np.float32(x.size)
    sq = (x * x).astype(np.float64)
    s = np.cumsum(sq)[-1] if x.size else 0.0
    mean = np.float32(s / x.size)
    inv = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(eps) / n))
    scale = np.float32(1.0) / np.sqrt(n)
    return (x * inv) * scale


@pytest.mark.parametrize("width", [2, 8, 64, 128, 256])
@pytest.mark.parametrize("eps", [1e-6, 1e-4])
def test_grouped_l2_two_stage_source_bits(width, eps):
    # lib.rs:1944-1969
    i = np.arange(width * 3)
    x = np.where(i % 11 == 0, -0.0, np.where(i % 11 == 1, 0.0, ((i * 71 % 201) - 100.0) / 37.0)).astype(np.float32)
    scales = np.full(width, np.float32(1.0) / np.sqrt(np.float32(width)), np.float32)
    grouped = O.grouped_rms_norm(x, scales, 3, np.float32(eps) / np.float32(width))
    ref = np.concatenate([_l2_reference(x[h * width:(h + 1) * width], eps) for h in range(3)])
    assert np.array_equal(grouped.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_l2_closed_form_three_four():
    # lib.rs:1972-1976
    y = O.grouped_rms_norm([3.0, 4.0], [1 / math.sqrt(2.0)] * 2, 1, 1e-6 / 2)
    assert abs(y[0] - 0.6) < 1e-5 and abs(y[1] - 0.8) < 1e-5


def test_grouped_rms_heads_match_independent_heads():
    # lib.rs:1911-1941
    coef = np.array([0.25 + i / 341.0 for i in range(128)], np.float32)
    act = np.array([((i * 37 % 499) - 245.0) / 193.0 for i in range(128 * 17)], np.float32)
    g = O.grouped_rms_norm(act, coef, 17, 1e-6)
    for h in range(17):
        one = O.rms_norm(act[h * 128:(h + 1) * 128], coef, 1e-6)
        assert np.array_equal(g[h * 128:(h + 1) * 128].view(np.uint32), one.view(np.uint32))
    with pytest.raises(O.OracleError):
        O.rms_norm(np.array([1.0, np.inf], np.float32), np.ones(2, np.float32), 1e-6)


# ---------------------------------------------------------- exp / SiLU / misc

def test_ggml_silu_bounded_against_exact_silu():
    # cpu/src/ops.rs:358-377
    for integer in range(-100, 101):
        x = integer / 10.0
        y = O.lib().zgo_ggml_silu(x)
        assert math.isfinite(y)
        assert abs(y - x / (1.0 + math.exp(-x))) <= 1e-5
    assert O.lib().zgo_ggml_silu(0.0) == 0.0


def test_ggml_exp_relative_error_closed_form():
    # closed form: exp polynomial within 2 ulp-ish of exp on the model range;
    # a wrong constant in the polynomial or range reduction breaks this.
    xs = np.linspace(-87.0, 20.0, 4001, dtype=np.float32)
    ours = np.array([O.lib().zgo_ggml_exp(float(x)) for x in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(ours - ref) / ref) < 4e-7


def test_binary_signed_zero_table():
    # lib.rs:1701-1736
    den = fbits(1)
    for a, b, want in [(-0.0, -0.0, 0x80000000), (0.0, -0.0, 0), (den, -den, 0)]:
        assert bits(O.binary(0, [a], [b])[0]) == want
    out = O.binary(1, [-den, -0.0, 1.0], [-128.0, 0.0, 128.0])
    assert bits(out[0]) == 0x80000000 and bits(out[1]) == 0x80000000 and out[2] == 1.0


def test_softplus_and_sigmoid_closed_forms():
    # lib.rs:2058-2068 (sigmoid(0)=0.5, softplus(0)=ln 2)
    L = O.lib()
    assert abs(L.zgo_sigmoid(0.0) - 0.5) < 1e-6
    assert abs(L.zgo_softplus(0.0) - math.log(2.0)) < 1e-6
    assert L.zgo_softplus(25.0) == 25.0
    assert abs(L.zgo_softplus(-25.0) - math.exp(-25.0)) < 1e-16


def test_greedy_first_maximum_and_refusals():
    # core/src/numerics.rs:146-162
    for v in ([-0.0, 0.0], [0.0, -0.0], [3.0, 3.0]):
        assert O.greedy(v) == 0
    assert O.greedy([-2.0, 4.0, 4.0]) == 1
    for bad in ([np.nan, 1.0], [1.0, np.inf], [-np.inf]):
        with pytest.raises(O.OracleError):
            O.greedy(bad)


# -------------------------------------------------------------- GDN ops

def test_gdn_conv_exact_bits_and_history():
    # cpu/src/ops/gdn.rs:51-84
    ch = 32
    qkv = np.array([((i * 13) - 199.0) / 117.0 for i in range(ch)], np.float32)
    w = np.array([((i * 37 % 71) - 35.0) / 509.0 for i in range(ch * 4)], np.float32)
    hist = np.array([((i * 19 % 83) - 41.0) / 239.0 for i in range(ch * 3)], np.float32)
    raw, new = O.gdn_conv_step(qkv, w, hist)
    for c in range(ch):
        o = hist[c * 3:c * 3 + 3]
        ww = w[c * 4:c * 4 + 4]
        e = np.float32(np.float32(np.float32(o[0] * ww[0]) + np.float32(o[1] * ww[1])) + np.float32(o[2] * ww[2]))
        e = np.float32(e + np.float32(qkv[c] * ww[3]))
        assert bits(raw[c]) == bits(e)
        assert list(new[c * 3:c * 3 + 3]) == [o[1], o[2], qkv[c]]
    bad = qkv.copy()
    bad[0] = np.nan
    with pytest.raises(O.OracleError):
        O.gdn_conv_step(bad, w, hist)


def test_gdn_coefficients_closed_form():
    # lib.rs:339-362 against f64 closed forms of softplus / sigmoid / exp
    rng = np.random.default_rng(2)
    alpha = rng.standard_normal(16).astype(np.float32)
    beta = rng.standard_normal(16).astype(np.float32)
    dt = rng.standard_normal(16).astype(np.float32)
    a = -np.exp(rng.standard_normal(16)).astype(np.float32)
    gain, b, sp, gr = O.gdn_coefficients(alpha, beta, dt, a, 1 / math.sqrt(128))
    z = (alpha + dt).astype(np.float64)
    sp_ref = np.log1p(np.exp(z))
    np.testing.assert_allclose(sp, sp_ref, rtol=2e-6)
    np.testing.assert_allclose(gain, np.exp(sp_ref * a), rtol=4e-6)
    np.testing.assert_allclose(b, 1 / (1 + np.exp(-beta.astype(np.float64))), rtol=2e-6)


def test_source_dot_f32_closed_form_and_tail():
    rng = np.random.default_rng(9)
    for n in (1, 31, 32, 33, 128, 200):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        ref = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(O.source_dot_f32(a, b) - ref) <= 1e-5 * max(1.0, np.abs(a * b).sum())


def test_recurrence_32768_tokens_against_independent_f64_oracle():
    # lib.rs:1998-2055
    DIM, TOKENS = 8, 32768
    gain, beta, scale = 0.965, 0.125, 0.35355338
    st = np.zeros(DIM * DIM, np.float32)
    ref = np.zeros((DIM, DIM))
    i = np.arange(DIM)
    L = O.lib()
    out = np.empty(DIM, np.float32)
    worst = 0.0
    for t in range(TOKENS):
        key = ((((t * 13 + i * 29) % 73) - 36.0) / 650.0).astype(np.float32)
        query = ((((t * 17 + i * 5) % 31) - 15.0) / 19.0).astype(np.float32)
        value = ((((t * 19 + i * 11) % 43) - 21.0) / 97.0).astype(np.float32)
        assert L.zgo_gdn_recurrent_step(O.ptr(st), O.ptr(query), O.ptr(key), O.ptr(value), gain, beta,
                                        scale, O.ptr(out), DIM) == 0
        g, k64 = float(np.float32(gain)), key.astype(np.float64)
        prev = ref @ k64
        delta = (value.astype(np.float64) - g * prev) * float(np.float32(beta))
        ref = g * ref + np.outer(delta, k64)
        expected = (ref @ query.astype(np.float64)) * float(np.float32(scale))
        worst = max(worst, float(np.max(np.abs(out - expected))))
    assert worst < 1e-5


# ----------------------------------------------------------- attention ops

def test_rope_rotates_pair_i_and_i_plus_half():
    # lib.rs:2078-2089 (pair (0, 2) rotates for rotate 4; (0, 1) must not)
    q, k = O.rope_kv(np.array([1.0, 0.0, 0.0, 0.0], np.float32), np.zeros(4, np.float32), 4, 1, 1, 4, 1, 0.5)
    assert abs(q[0] - math.cos(1.0)) < 1e-6 and abs(q[2] - math.sin(1.0)) < 1e-6
    assert q[1] == 0.0 and q[3] == 0.0


@pytest.mark.parametrize("width", [64, 128, 256])
@pytest.mark.parametrize("pos", [0, 1, 119, 120, 128, 8192, 16384, 32768])
def test_rope_iterative_f32_schedule_and_tail(width, pos):
    # lib.rs:1864-1908: the source schedule (f32 angle multiplied by
    # theta_scale per pair, FMA form) with the value slab and the unrotated
    # tail untouched; compared with the same schedule evaluated in f64 from
    # the f32 angles (closed form of each rotation).
    q = np.array([((i * 17 % 107) - 53.0) / 31.0 for i in range(width * 2)], np.float32)
    k = q[:width].copy()
    ts = np.float32(np.float32(10_000_000.0) ** np.float32(-2.0 / 64.0))
    rq, rk = O.rope_kv(q, k, width, 2, 1, 64, pos, float(ts))
    for head_in, head_out in [(q[:width], rq[:width]), (q[width:], rq[width:]), (k, rk)]:
        angle = np.float32(pos)
        for i in range(32):
            a, b = float(head_in[i]), float(head_in[i + 32])
            s, c = math.sin(float(angle)), math.cos(float(angle))
            assert abs(head_out[i] - (a * c - b * s)) < 2e-6 * max(1, abs(a) + abs(b))
            assert abs(head_out[i + 32] - (a * s + b * c)) < 2e-6 * max(1, abs(a) + abs(b))
            angle = np.float32(angle * ts)
        assert np.array_equal(head_out[64:].view(np.uint32), head_in[64:].view(np.uint32))


@pytest.mark.parametrize("width", [1, 7, 8, 9, 31, 32, 33, 255, 256, 257, 4096])
def test_softmax_padded_eight_lane_schedule(width):
    # lib.rs:1803-1862 and accelerator.rs:411-453 (p == e * f32(1/sum) bits,
    # sum >= 1), with an f64 softmax closed form.
    i = np.arange(width * 3)
    m7 = i % 7
    scores = np.where(m7 == 0, -0.0, np.where(m7 == 1, -fbits(1), np.where(m7 == 2, -3.4028235e38,
                      ((i * 37 % 140) - 104.0)))).astype(np.float32)
    probs, exps, sums = O.attention_softmax(scores, 3, width)
    L = O.lib()
    for h in range(3):
        row = scores[h * width:(h + 1) * width]
        mx = np.float32(row.max())
        e = np.array([L.zgo_ggml_exp(float(np.float32(v - mx))) for v in row], np.float32)
        assert np.array_equal(e.view(np.uint32), exps[h * width:(h + 1) * width].view(np.uint32))
        ep = np.zeros((width + 7) // 8 * 8, np.float32)
        ep[:width] = e
        s = 0.0
        for b in range(0, ep.size, 8):
            x = ep[b:b + 8]
            s += float(np.float32(np.float32(np.float32(x[0] + x[4]) + np.float32(x[2] + x[6]))
                                  + np.float32(np.float32(x[1] + x[5]) + np.float32(x[3] + x[7]))))
        assert s == sums[h] and s >= 1.0
        inv = np.float32(1.0 / s)
        assert np.array_equal((e * inv).view(np.uint32), probs[h * width:(h + 1) * width].view(np.uint32))
        ref = np.exp(row.astype(np.float64) - float(mx))
        np.testing.assert_allclose(probs[h * width:(h + 1) * width], ref / ref.sum(), atol=2e-7)


@pytest.mark.parametrize("tokens,expected", [(1, 0x80000001), (31, 0), (32, 0), (33, 0),
                                             (255, 0), (256, 0x80000000), (257, 0)])
def test_attention_value_padding_signed_zero(tokens, expected):
    # lib.rs:1738-1799
    values = np.full((tokens, 1), -fbits(1), np.float32)
    probs = np.full(tokens, np.float32(1.0) / np.float32(tokens), np.float32)
    out = O.attention_value(probs, values, 1, 1, 1)
    assert bits(out[0]) == expected


def test_attention_qk_score_is_rounded_dot_times_scale():
    # core/src/accelerator.rs:1012-1054 plus an f64 dot closed form (GQA map)
    rng = np.random.default_rng(4)
    hw, qh, kvh, T = 256, 8, 2, 37
    q = rng.standard_normal(qh * hw).astype(np.float32)
    keys = rng.standard_normal((T, kvh * hw)).astype(np.float32)
    dots, scores = O.attention_qk(q, keys, hw, qh, kvh, 0.0625)
    assert np.array_equal((dots * np.float32(0.0625)).view(np.uint32), scores.view(np.uint32))
    for h in range(qh):
        kv = h // (qh // kvh)
        ref = keys[:, kv * hw:(kv + 1) * hw].astype(np.float64) @ q[h * hw:(h + 1) * hw].astype(np.float64)
        np.testing.assert_allclose(dots[h * T:(h + 1) * T], ref, atol=1e-4)


def test_attention_value_closed_form_gqa():
    rng = np.random.default_rng(8)
    hw, qh, kvh, T = 256, 8, 2, 300
    probs = rng.uniform(0, 1, (qh, T)).astype(np.float32)
    probs /= probs.sum(1, keepdims=True)
    values = rng.standard_normal((T, kvh * hw)).astype(np.float32)
    out = O.attention_value(probs.reshape(-1), values, hw, qh, kvh).reshape(qh, hw)
    for h in range(qh):
        kv = h // (qh // kvh)
        ref = probs[h].astype(np.float64) @ values[:, kv * hw:(kv + 1) * hw].astype(np.float64)
        np.testing.assert_allclose(out[h], ref, atol=1e-5)


# ------------------------------------------------------ chunked prefill

def _tokenwise(q, k, v, beta, logd, H, d):
    T = beta.size // H
    scale = 1.0 / math.sqrt(d)
    sc = np.full(d, np.float32(1.0) / np.sqrt(np.float32(d)), np.float32)
    st = np.zeros(H * d * d, np.float32)
    outs = np.zeros((T, H, d), np.float32)
    for t in range(T):
        for h in range(H):
            sl = slice((t * H + h) * d, (t * H + h + 1) * d)
            qn = O.grouped_rms_norm(q[sl], sc, 1, 1e-6 / d)
            kn = O.grouped_rms_norm(k[sl], sc, 1, 1e-6 / d)
            o, s2 = O.gdn_recurrent_step(st[h * d * d:(h + 1) * d * d], qn, kn, v[sl],
                                         float(np.exp(np.float32(logd[t * H + h]))), float(beta[t * H + h]), scale)
            st[h * d * d:(h + 1) * d * d] = s2
            outs[t, h] = o
    return outs.reshape(-1), st


@pytest.mark.parametrize("T,chunk", [(5, 4), (70, 64), (130, 64)])
def test_chunked_prefill_matches_tokenwise_recurrence(T, chunk):
    # The chunk (WY/UT) algorithm of numerics/torch_cpu/gdn/chunk/core.rs:152-363
    # must reproduce the token-by-token recurrence (lib.rs:1446-1499) on the
    # final state and every output; this is the pin for the chunk restatement.
    rng = np.random.default_rng(T)
    H, d = 2, 32
    q = rng.standard_normal(T * H * d).astype(np.float32)
    k = rng.standard_normal(T * H * d).astype(np.float32)
    v = rng.standard_normal(T * H * d).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32)
    logd = (-np.log1p(np.exp(rng.standard_normal(T * H))) * np.exp(0.5 * rng.standard_normal(T * H))).astype(np.float32)
    out_c, st_c = O.gdn_chunk_prefill(q, k, v, beta, logd, H, d, chunk)
    out_t, st_t = _tokenwise(q, k, v, beta, logd, H, d)
    np.testing.assert_allclose(st_c, st_t, atol=2e-5 * max(1.0, np.abs(st_t).max()))
    np.testing.assert_allclose(out_c, out_t, atol=2e-5 * max(1.0, np.abs(out_t).max()))
