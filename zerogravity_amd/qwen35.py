"""Qwen3.5 hybrid (Gated DeltaNet + GQA) model on the MI355X backend.

`QwenDenseHip` mirrors the reference's `QwenDenseCpu` session API
(crates/zerogravity-model-qwen35/src/lib.rs:1058-1254): `forward(token)`,
`prefill_transaction(tokens)`, `prefill_chunk_without_logits(tokens)`,
`reset()`, `position`, state domain export/import (lib.rs:112-150), plus
the batched decode of a continuous batch.  Weights come from a GGUF file
(`LoadedQwenModel::open`, lib.rs:371-375) or from an in-memory tensor table.
"""
import ctypes as C
import itertools
import json
import os

import numpy as np

from . import _lib as L
from . import gguf
from . import synth

_SOURCE_IDS = itertools.count(1 << 32)

# BASELINE shapes: 0.8B-shaped (Q8_0) and 2B-shaped (Q4_K)
QWEN35_0_8B = dict(hidden=1024, layers=24, ffn=3584, vocab=151936, gdn_heads=16, gdn_dim=128, q_heads=8,
                   kv_heads=2, head_dim=256, full_attention_interval=4, max_context=262144, eps=1e-6)
QWEN35_2B = dict(QWEN35_0_8B, hidden=2048, ffn=6144)


class TensorDesc(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_int), ("shape0", C.c_uint64), ("shape1", C.c_uint64),
                ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class Geometry(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("layers", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32),
                ("gdn_heads", C.c_uint32), ("gdn_dim", C.c_uint32), ("q_heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("full_attention_interval", C.c_uint32),
                ("max_context", C.c_uint32), ("eps", C.c_float)]


def layer_kinds(g):
    """config.rs:146-167: layer i is full attention iff (i+1) % interval == 0."""
    return ["full_attention" if (i + 1) % g["full_attention_interval"] == 0 else "linear_attention"
            for i in range(g["layers"])]


def config_json(g):
    """A config.json that ModelGeometry::from_json (config.rs:51-182) accepts."""
    return {
        "model_type": "qwen3_5",
        "architectures": ["Qwen3_5ForConditionalGeneration"],
        "text_config": {
            "model_type": "qwen3_5_text",
            "layer_types": layer_kinds(g),
            "num_hidden_layers": g["layers"],
            "hidden_size": g["hidden"],
            "intermediate_size": g["ffn"],
            "head_dim": g["head_dim"],
            "num_attention_heads": g["q_heads"],
            "num_key_value_heads": g["kv_heads"],
            "vocab_size": g["vocab"],
            "max_position_embeddings": g["max_context"],
            "full_attention_interval": g["full_attention_interval"],
            "linear_conv_kernel_dim": 4,
            "linear_num_key_heads": g["gdn_heads"],
            "linear_num_value_heads": g["gdn_heads"],
            "linear_key_head_dim": g["gdn_dim"],
            "linear_value_head_dim": g["gdn_dim"],
            "rms_norm_eps": g["eps"],
        },
    }


def geometry_from_config(cfg, gdn_dim=128):
    t = cfg["text_config"]
    if cfg.get("model_type") != "qwen3_5" or t.get("model_type") != "qwen3_5_text":
        raise ValueError("no registered reference geometry for this model_type")
    g = dict(hidden=t["hidden_size"], layers=t["num_hidden_layers"], ffn=t["intermediate_size"],
             vocab=t["vocab_size"], gdn_heads=t["linear_num_value_heads"],
             gdn_dim=t.get("linear_value_head_dim", gdn_dim), q_heads=t["num_attention_heads"],
             kv_heads=t["num_key_value_heads"], head_dim=t["head_dim"],
             full_attention_interval=t["full_attention_interval"],
             max_context=t["max_position_embeddings"], eps=1e-6)
    if layer_kinds(g) != t["layer_types"]:
        raise ValueError("Qwen hybrid layer schedule disagrees with interval")
    return g


# A mixed-codec table in the manner of the published mixed-quant
# checkpoints: Q6_K for the embedding, value and down projections, F32 for
# the small GDN alpha/beta projections (the F32 ssm_alpha projection named
# at cpu/src/source.rs:316-323), Q4_1 for the output gate.  Suffix -> codec;
# everything else keeps `kind`.
MIXED = {"token_embd.weight": gguf.Q6_K, "attn_v.weight": gguf.Q6_K, "ffn_down.weight": gguf.Q6_K,
         "ssm_alpha.weight": gguf.F32, "ssm_beta.weight": gguf.F32, "attn_gate.weight": gguf.Q4_1}


def synthetic_tensors(g, kind, seed, kinds=None):
    """Seeded random-init tensor table {name: (ggml_type, shape0, shape1, uint8 bytes)}.

    Matrices use `kind` (or kinds[suffix] when given, e.g. MIXED) with row norms ~1 so activations stay
    O(1) through the 24 layers; norms gamma ~ N(1, 0.1); ssm_a = -exp(N(0,0.5));
    ssm_dt ~ N(0, 1); conv taps ~ N(0, 0.5).  Shapes per
    model-qwen35/src/source/binding.rs:43-91 (GGML order [K, N]).
    """
    rng = np.random.default_rng(seed)
    H, F, V = g["hidden"], g["ffn"], g["vocab"]
    W = g["gdn_heads"] * g["gdn_dim"]
    QD, KD = g["q_heads"] * g["head_dim"], g["kv_heads"] * g["head_dim"]
    t = {}

    def mat(name, K, N):
        k = kind
        if kinds:
            k = kinds.get(name.split(".", 2)[-1] if name.startswith("blk.") else name, kind)
        t[name] = (k, K, N, synth.random_matrix(rng, k, N, K).reshape(-1))

    def vec(name, values):
        a = np.ascontiguousarray(values, np.float32)
        t[name] = (gguf.F32, a.size, 1, a.view(np.uint8))

    mat("token_embd.weight", H, V)
    vec("output_norm.weight", 1 + 0.1 * rng.standard_normal(H))
    for i, kindname in enumerate(layer_kinds(g)):
        p = f"blk.{i}."
        vec(p + "attn_norm.weight", 1 + 0.1 * rng.standard_normal(H))
        vec(p + "post_attention_norm.weight", 1 + 0.1 * rng.standard_normal(H))
        mat(p + "ffn_gate.weight", H, F)
        mat(p + "ffn_up.weight", H, F)
        mat(p + "ffn_down.weight", F, H)
        if kindname == "full_attention":
            mat(p + "attn_q.weight", H, 2 * QD)
            mat(p + "attn_k.weight", H, KD)
            mat(p + "attn_v.weight", H, KD)
            mat(p + "attn_output.weight", QD, H)
            vec(p + "attn_q_norm.weight", 1 + 0.1 * rng.standard_normal(g["head_dim"]))
            vec(p + "attn_k_norm.weight", 1 + 0.1 * rng.standard_normal(g["head_dim"]))
        else:
            mat(p + "attn_qkv.weight", H, 3 * W)
            mat(p + "attn_gate.weight", H, W)
            mat(p + "ssm_alpha.weight", H, g["gdn_heads"])
            mat(p + "ssm_beta.weight", H, g["gdn_heads"])
            mat(p + "ssm_out.weight", W, H)
            conv = (0.5 * rng.standard_normal((3 * W, 4))).astype(np.float32)
            t[p + "ssm_conv1d.weight"] = (gguf.F32, 4, 3 * W, conv.reshape(-1).view(np.uint8))
            vec(p + "ssm_norm.weight", 1 + 0.1 * rng.standard_normal(g["gdn_dim"]))
            vec(p + "ssm_a", -np.exp(0.5 * rng.standard_normal(g["gdn_heads"])))
            vec(p + "ssm_dt.bias", rng.standard_normal(g["gdn_heads"]))
    return t


def write_gguf(path, g, tensors):
    """Write a qwen35 GGUF + config.json beside it."""
    items = [(name, ty, (s0, s1) if s1 != 1 or ty != gguf.F32 else (s0,), data)
             for name, (ty, s0, s1, data) in tensors.items()]
    gguf.write(path, items, {"general.architecture": "qwen35", "general.name": "qwen35-synthetic"})
    with open(os.path.splitext(path)[0] + ".config.json", "w") as f:
        json.dump(config_json(g), f, indent=1)


def read_gguf(path, config_path=None):
    """(geometry, tensor table) from a GGUF + config.json; architecture must be
    qwen35 (lib.rs:387-391)."""
    f = gguf.GgufFile(path)
    if f.architecture != "qwen35":
        raise ValueError("Qwen runner needs qwen35 GGUF tensors")
    cfg_path = config_path or os.path.splitext(path)[0] + ".config.json"
    with open(cfg_path) as fh:
        g = geometry_from_config(json.load(fh))
    t = {}
    for name, info in f.tensors.items():
        s0 = info.shape[0]
        s1 = int(np.prod(info.shape[1:])) if len(info.shape) > 1 else 1
        t[name] = (info.ggml_type, s0, s1, f.data(name))
    return g, t, f


# ProgramNumericalProfile (core/src/numerics.rs:30-40), in its order
PROFILES = {"GgufSourceV1": 0, "TorchCpuBf16Avx2MixedSourceV1": 1, "SourceCudaSm86Bf16V1": 2,
            "AnalyticF32TextV1": 3, "DirectGammaBf16TextCandidateV1": 4}


def _tensor_table(tensors):
    """zg_tensor_desc[] over the host arrays of {name: (type, ne0, ne1, bytes)};
    the second value keeps the arrays alive while the table is used."""
    descs = (TensorDesc * len(tensors))()
    keep = []
    for i, (name, (ty, s0, s1, data)) in enumerate(tensors.items()):
        data = np.ascontiguousarray(data)
        nb = name.encode()
        keep += [data, nb]
        descs[i] = TensorDesc(nb, ty, s0, s1, data.ctypes.data, data.nbytes)
    return descs, keep


def admit(geometry: dict, tensors: dict, profile="GgufSourceV1"):
    """Plan admission before any device work (zg_model_admit): raises ZgError
    E_UNSUPPORTED unless the plan's numerical profile is GgufSourceV1 and its
    tensors carry codecs the schedule's kernels take (LoadedQwenModel::
    require_execution_profile, model-qwen35/src/source/binding.rs:363-371),
    E_MALFORMED for a missing tensor or a shape that differs from the
    geometry.  Host only: runs without a GPU."""
    code = PROFILES[profile] if isinstance(profile, str) else int(profile)
    descs, keep = _tensor_table(tensors)
    msg = C.create_string_buffer(512)
    rc = L.lib().zg_model_admit(code, C.byref(Geometry(**geometry)), descs, len(tensors), msg, len(msg))
    if rc != L.COMPLETED:
        raise L.ZgError(rc, msg.value.decode(errors="replace"))


class QwenModelHip:
    """LoadedQwenModel on the device: weights resident once, sessions share them."""

    def __init__(self, geometry: dict, tensors: dict, kernel=None, device=0, source_id=None, profile="GgufSourceV1"):
        from .regions import HipMatVecKernel
        # a plan of another numerical profile is refused before any device work
        admit(geometry, tensors, profile)
        self.kernel = kernel or HipMatVecKernel(device)
        self.ctx = self.kernel.ctx
        self.g = dict(geometry)
        # SourceIdentity of the tensor source (core/src/accelerator.rs:22-59):
        # models loaded from the same source share its resident weights
        self.source_id = next(_SOURCE_IDS) if source_id is None else int(source_id)
        descs, keep = _tensor_table(tensors)
        geo = Geometry(**self.g)
        h = C.c_void_p()
        self.ctx.check(L.lib().zg_model_load(self.ctx.h, self.source_id, C.byref(geo), descs, len(tensors),
                                             C.byref(h)))
        self.h = h
        self.ctx.adopt(self)

    def session(self, max_batch=1, max_context=4096, kv_dtype=L.BF16):
        return QwenDenseHip(self, max_batch, max_context, kv_dtype)

    def close(self):
        if getattr(self, "h", None) and getattr(self.ctx, "h", None):
            L.lib().zg_model_destroy(self.h)
        self.h = None

    def __del__(self):
        self.close()


class Snapshot:
    """A zg_snapshot: device memory holding one row's state and position."""

    def __init__(self, session, row):
        h = C.c_void_p()
        session.model.ctx.check(L.lib().zg_session_snapshot(session.h, row, C.byref(h)))
        self.h = h
        self.position = L.lib().zg_snapshot_position(h)
        self.nbytes = L.lib().zg_snapshot_bytes(h)
        session.model.ctx.adopt(self)

    def close(self):
        if getattr(self, "h", None):
            L.lib().zg_snapshot_destroy(self.h)
        self.h = None

    def __del__(self):
        self.close()


class QwenDenseHip:
    """QwenDenseCpu's session API over a device session of `max_batch` rows."""

    def __init__(self, model, max_batch, max_context, kv_dtype):
        self.model = model
        self.rows = max_batch
        self.vocab = model.g["vocab"]
        h = C.c_void_p()
        model.ctx.check(L.lib().zg_session_create(model.h, max_batch, max_context, kv_dtype, C.byref(h)))
        self.h = h
        model.ctx.adopt(self)

    @property
    def position(self):
        return L.lib().zg_session_position(self.h, 0)

    def positions(self):
        return [L.lib().zg_session_position(self.h, r) for r in range(self.rows)]

    def step(self, tokens, logits=True, greedy=False):
        """One forward_token for rows [0, len(tokens))."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        n = toks.size
        lg = np.empty((n, self.vocab), np.float32) if logits else None
        gr = np.empty(n, np.uint32) if greedy else None
        self.model.ctx.check(L.lib().zg_decode_step(self.h, n, toks.ctypes.data, None if lg is None else lg.ctypes.data,
                                                    None if gr is None else gr.ctypes.data))
        return lg, gr

    def forward(self, token):
        """QwenDenseCpu::forward (lib.rs:1227-1232): logits of one token on row 0."""
        return self.step([token])[0][0]

    def next_logits(self, tokens, greedy=False):
        """QwenDenseCpu::next_logits (lib.rs:1057-1070): logits of one token per
        row [0, len(tokens)) on a draft; publish with commit()."""
        toks = np.ascontiguousarray(np.atleast_1d(tokens), np.uint32)
        n = toks.size
        lg = np.empty((n, self.vocab), np.float32)
        gr = np.empty(n, np.uint32) if greedy else None
        self.model.ctx.check(L.lib().zg_session_propose(self.h, n, toks.ctypes.data, lg.ctypes.data,
                                                        None if gr is None else gr.ctypes.data))
        return (lg, gr) if greedy else lg

    def commit(self):
        """QwenDenseCpu::commit (lib.rs:1211-1225): publish the pending proposal."""
        self.model.ctx.check(L.lib().zg_session_commit(self.h))

    def snapshot(self, row=0):
        """Device-side copy of one row's published state (ResidentSession::snapshot)."""
        return Snapshot(self, row)

    def restore(self, snap, row=0):
        """Install a snapshot of this model into `row` (ResidentSession::restore)."""
        self.model.ctx.check(L.lib().zg_session_restore(self.h, row, snap.h))

    def prefill_transaction(self, tokens):
        """Per-token prefill on row 0, logits of the last token (lib.rs:1119-1187)."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        if toks.size == 0:
            raise L.ZgError(L.E_MALFORMED, "prefill must contain at least one token")
        lg = np.empty(self.vocab, np.float32)
        self.model.ctx.check(L.lib().zg_prefill(self.h, 1, toks.size, toks.ctypes.data, lg.ctypes.data))
        return lg

    def prefill_batched(self, tokens, row=0, logits=True):
        """The whole prompt of one row layer by layer (batched projections,
        chunked GDN prefill, causal attention); logits of the last token."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        if toks.size == 0:
            raise L.ZgError(L.E_MALFORMED, "prefill must contain at least one token")
        lg = np.empty(self.vocab, np.float32) if logits else None
        self.model.ctx.check(L.lib().zg_prefill_batched(self.h, row, toks.size, toks.ctypes.data,
                                                          None if lg is None else lg.ctypes.data))
        return lg

    def prefill_chunk_without_logits(self, tokens):
        toks = np.ascontiguousarray(tokens, np.uint32)
        self.model.ctx.check(L.lib().zg_prefill(self.h, 1, toks.size, toks.ctypes.data, None))

    def reset(self):
        self.model.ctx.check(L.lib().zg_session_reset(self.h))

    def reset_row(self, row):
        """Retire one row: its state and KV cache zeroed, position 0."""
        self.model.ctx.check(L.lib().zg_session_reset_row(self.h, row))

    def copy_row(self, dst, src):
        """Row dst takes a copy of row src's state, KV prefix and position."""
        self.model.ctx.check(L.lib().zg_session_copy_row(self.h, dst, src))

    def retire(self, row, active):
        """Retire `row` of a batch whose active rows are [0, active): the last
        active row moves into its slot, so [0, active - 1) stays dense.
        Returns the new active count."""
        if not 0 <= row < active <= self.rows:
            raise L.ZgError(L.E_LIMIT, "row outside the active batch")
        last = active - 1
        if row != last:
            self.copy_row(row, last)
        self.reset_row(last)
        return last

    def state(self, row=0):
        n = L.lib().zg_state_floats(self.h, row)
        out = np.empty(n, np.float32)
        self.model.ctx.check(L.lib().zg_state_export(self.h, row, out.ctypes.data, n))
        return out

    def load_state(self, values, position, row=0):
        v = np.ascontiguousarray(values, np.float32)
        self.model.ctx.check(L.lib().zg_state_import(self.h, row, v.ctypes.data, v.size, position))

    def fill_random_prefix(self, rows, prefix, seed):
        self.model.ctx.check(L.lib().zg_session_fill_random(self.h, rows, prefix, seed))

    def close(self):
        if getattr(self, "h", None) and getattr(self.model, "h", None):
            L.lib().zg_session_destroy(self.h)
        self.h = None

    def __del__(self):
        self.close()
