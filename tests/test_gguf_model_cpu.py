"""CPU checks of the on-disk format and of the oracle model driver:
GGUF v3 writer/reader against the reference parser's rules
(artifacts/src/artifact.rs:539-672), config.json geometry
(model-qwen35/src/config.rs:51-182), and the oracle session's state
domains / reset / import semantics (model-qwen35/src/lib.rs:95-191)."""
import json
import struct

import numpy as np
import pytest

import zg_oracle as O
from zerogravity_amd import gguf, qwen35

TINY = dict(hidden=256, layers=4, ffn=512, vocab=1000, gdn_heads=2, gdn_dim=128, q_heads=2, kv_heads=1,
            head_dim=256, full_attention_interval=4, max_context=256, eps=1e-6)


def oracle_model(g, t, threads=0):
    return O.Model(g, {k: (ty, s0, s1, d) for k, (ty, s0, s1, d) in t.items()}, threads)


@pytest.fixture(scope="module")
def tiny():
    return qwen35.synthetic_tensors(TINY, gguf.Q8_0, seed=3)


def test_gguf_round_trip(tmp_path, tiny):
    path = str(tmp_path / "m.gguf")
    qwen35.write_gguf(path, TINY, tiny)
    g, t, f = qwen35.read_gguf(path)
    assert g == TINY
    assert set(t) == set(tiny)
    for name, (ty, s0, s1, data) in tiny.items():
        assert t[name][:3] == (ty, s0, s1)
        assert np.array_equal(t[name][3], data)
    f.close()


def _header(n_tensors, kvs=b"", n_kv=0):
    return b"GGUF" + struct.pack("<IQQ", 3, n_tensors, n_kv) + kvs


def test_gguf_reader_refusals(tmp_path):
    def parse(b):
        return gguf.parse(memoryview(b), len(b))
    with pytest.raises(gguf.GgufError):
        parse(b"GGUX" + b"\0" * 20)
    with pytest.raises(gguf.GgufError):
        parse(b"GGUF" + struct.pack("<IQQ", 2, 0, 0))
    name = b"t"
    def tensor(ty, shape, off):
        return (struct.pack("<Q", len(name)) + name + struct.pack("<I", len(shape))
                + b"".join(struct.pack("<Q", d) for d in shape) + struct.pack("<IQ", ty, off))
    # unaligned offset
    with pytest.raises(gguf.GgufError):
        parse(_header(1) + tensor(gguf.F32, (4,), 4) + b"\0" * 64)
    # row not aligned to blocks
    with pytest.raises(gguf.GgufError):
        parse(_header(1) + tensor(gguf.Q8_0, (31,), 0) + b"\0" * 64)
    # unknown type
    with pytest.raises(gguf.GgufError):
        parse(_header(1) + tensor(40, (4,), 0) + b"\0" * 64)
    # past EOF
    with pytest.raises(gguf.GgufError):
        parse(_header(1) + tensor(gguf.F32, (1024,), 0) + b"\0" * 64)
    # bad alignment metadata
    key = b"general.alignment"
    kv = struct.pack("<Q", len(key)) + key + struct.pack("<II", 4, 12)
    with pytest.raises(gguf.GgufError):
        parse(_header(0, kv, 1))


def test_config_geometry_round_trip_and_refusals():
    cfg = qwen35.config_json(qwen35.QWEN35_2B)
    assert qwen35.geometry_from_config(json.loads(json.dumps(cfg))) == qwen35.QWEN35_2B
    kinds = cfg["text_config"]["layer_types"]
    assert kinds.count("full_attention") == 6 and kinds[3] == "full_attention" and kinds[0] == "linear_attention"
    bad = json.loads(json.dumps(cfg))
    bad["text_config"]["layer_types"][0] = "full_attention"
    with pytest.raises(ValueError):
        qwen35.geometry_from_config(bad)


def test_oracle_session_state_domains_reset_and_import(tiny):
    m = oracle_model(TINY, tiny)
    s = m.session()
    toks = [5, 17, 999, 0, 42]
    first = [s.forward(t) for t in toks]
    assert s.position == len(toks)
    st = s.state()
    # domains: 3 GDN layers x (conv 3*768*... ) + 1 attention layer x 2 * T * kv
    W = TINY["gdn_heads"] * TINY["gdn_dim"]
    n_gdn = 3
    expect = n_gdn * (3 * W * 3 + TINY["gdn_heads"] * 128 * 128) + 2 * len(toks) * TINY["kv_heads"] * 256
    assert st.size == expect
    nxt = s.forward(7)
    s2 = m.session()
    s2.load_state(st, len(toks))
    assert np.array_equal(s2.forward(7), nxt)
    # a fresh session reproduces the same logits bit for bit
    s3 = m.session()
    again = [s3.forward(t) for t in toks]
    for a, b in zip(first, again):
        assert np.array_equal(a, b)
    with pytest.raises(O.OracleError):
        s3.forward(TINY["vocab"])
    assert all(np.isfinite(x).all() for x in first)
