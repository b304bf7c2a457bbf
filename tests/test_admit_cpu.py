"""Boundary B plan admission on the CPU (zg_model_admit: host only, no device).

A provider prepares whatever plan it is given (core/src/provider.rs:38-42),
while LoadedQwenModel runs only plans of the GGUF source profile
(require_execution_profile, model-qwen35/src/source/binding.rs:363-371;
the profiles are ProgramNumericalProfile, core/src/numerics.rs:30-40).  The
backend therefore refuses, before any device work, a plan of another
profile and a tensor table whose codecs or shapes are not the schedule its
decode step runs.
"""
import numpy as np
import pytest

from zerogravity_amd import _lib as L
from zerogravity_amd import gguf, qwen35

G = dict(hidden=256, layers=4, ffn=512, vocab=300, gdn_heads=2, gdn_dim=128, q_heads=2, kv_heads=1,
         head_dim=256, full_attention_interval=4, max_context=64, eps=1e-6)


@pytest.fixture(scope="module")
def table():
    return qwen35.synthetic_tensors(G, gguf.Q4_K, seed=7)


def _code(t, profile="GgufSourceV1", g=G):
    try:
        qwen35.admit(g, t, profile)
        return L.COMPLETED, ""
    except L.ZgError as e:
        return e.code, str(e)


def test_gguf_profile_and_schedule_tensors_are_admitted(table):
    assert _code(table) == (L.COMPLETED, "")
    t8 = qwen35.synthetic_tensors(G, gguf.Q8_0, seed=8)
    assert _code(t8)[0] == L.COMPLETED


@pytest.mark.parametrize("profile", [p for p in qwen35.PROFILES if p != "GgufSourceV1"])
def test_other_numerical_profiles_are_unsupported(table, profile):
    code, msg = _code(table, profile)
    assert code == L.E_UNSUPPORTED, msg
    assert "profile" in msg


def test_codec_the_schedule_does_not_run_is_unsupported(table):
    t = dict(table)
    ty, k, n, data = t["blk.0.ffn_down.weight"]
    t["blk.0.ffn_down.weight"] = (L.BF16, k, n, np.zeros(k * n * 2, np.uint8))
    code, msg = _code(t)
    assert code == L.E_UNSUPPORTED and "blk.0.ffn_down.weight" in msg, msg


def test_missing_or_misshaped_tensors_are_malformed(table):
    t = dict(table)
    del t["blk.3.attn_k.weight"]
    code, msg = _code(t)
    assert code == L.E_MALFORMED and "missing tensor blk.3.attn_k.weight" in msg, msg
    # a matrix handed over with its axes swapped
    t = dict(table)
    ty, k, n, data = t["blk.1.attn_qkv.weight"]
    t["blk.1.attn_qkv.weight"] = (ty, n, k, data)
    assert _code(t)[0] == L.E_MALFORMED
    # a packed length that is not rows x row bytes
    t = dict(table)
    ty, k, n, data = t["blk.2.ssm_out.weight"]
    t["blk.2.ssm_out.weight"] = (ty, k, n, data[:-144])
    assert _code(t)[0] == L.E_MALFORMED
    # a norm vector that is not F32
    t = dict(table)
    ty, k, n, data = t["output_norm.weight"]
    t["output_norm.weight"] = (L.F16, k, n, np.zeros(k * n * 2, np.uint8))
    assert _code(t)[0] == L.E_MALFORMED


def test_geometry_outside_the_schedule_is_unsupported(table):
    assert _code(table, g=dict(G, head_dim=128))[0] == L.E_UNSUPPORTED
    assert _code(table, g=dict(G, q_heads=8))[0] == L.E_UNSUPPORTED  # 8 query heads per KV head
