"""ctypes binding of the CPU oracle (libzg_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product package never
imports this module.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzg_oracle.so")

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20),
         Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_int), ("shape0", C.c_uint64),
                ("shape1", C.c_uint64), ("data", P), ("nbytes", C.c_uint64)]


class Geometry(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("layers", C.c_uint32), ("ffn", C.c_uint32),
                ("vocab", C.c_uint32), ("gdn_heads", C.c_uint32), ("gdn_dim", C.c_uint32),
                ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("full_attention_interval", C.c_uint32), ("max_context", C.c_uint32),
                ("eps", C.c_float)]


def _declare(L):
    sig = {
        "zgo_set_libm_mode": (C.c_int, [C.c_int]),
        "zgo_libm_mode": (C.c_int, []),
        "zgo_f16_to_f32": (C.c_float, [C.c_uint16]),
        "zgo_f32_to_f16_rne": (C.c_uint16, [C.c_float]),
        "zgo_dequantize": (C.c_int, [C.c_int, P, SZ, SZ, P]),
        "zgo_q8_activation": (C.c_int, [P, SZ, P, P, P]),
        "zgo_dot_q8_0_row": (C.c_float, [P, P, P, SZ]),
        "zgo_dot_q4k_row": (C.c_float, [P, P, SZ]),
        "zgo_dot_f32_row": (C.c_float, [P, P, SZ]),
        "zgo_q8k_activation": (C.c_int, [P, SZ, P, P, P]),
        "zgo_dot_q4_0_row": (C.c_float, [P, P, P, SZ]),
        "zgo_dot_q4_0_repacked_row": (C.c_float, [P, P, P, SZ]),
        "zgo_dot_q4_1_row": (C.c_float, [P, P, P, P, SZ]),
        "zgo_dot_q6k_row": (C.c_float, [P, P, P, P, SZ]),
        "zgo_matvec": (C.c_int, [C.c_int, P, SZ, SZ, SZ, P, P, C.c_int]),
        "zgo_rms_norm": (C.c_int, [P, P, SZ, C.c_float, P]),
        "zgo_grouped_rms_norm": (C.c_int, [P, P, SZ, SZ, C.c_float, P]),
        "zgo_ggml_exp": (C.c_float, [C.c_float]),
        "zgo_ggml_silu": (C.c_float, [C.c_float]),
        "zgo_silu": (C.c_int, [P, P, SZ, P]),
        "zgo_sigmoid": (C.c_float, [C.c_float]),
        "zgo_softplus": (C.c_float, [C.c_float]),
        "zgo_binary": (C.c_int, [C.c_int, P, P, SZ, P]),
        "zgo_gdn_conv_step": (C.c_int, [P, P, P, P, SZ]),
        "zgo_gdn_coefficients": (C.c_int, [P, P, P, P, SZ, C.c_float, P, P, P, P]),
        "zgo_source_dot_f32": (C.c_float, [P, P, SZ]),
        "zgo_gdn_recurrent_step": (C.c_int, [P, P, P, P, C.c_float, C.c_float, C.c_float, P, SZ]),
        "zgo_rope_kv": (C.c_int, [P, P, SZ, SZ, SZ, SZ, SZ, C.c_float]),
        "zgo_attention_qk": (C.c_int, [P, P, SZ, SZ, SZ, SZ, C.c_float, P, P]),
        "zgo_attention_softmax": (C.c_int, [P, SZ, SZ, P, P, P]),
        "zgo_attention_value": (C.c_int, [P, P, SZ, SZ, SZ, SZ, SZ, P]),
        "zgo_greedy": (C.c_int, [P, SZ, P]),
        "zgo_gdn_chunk_prefill": (C.c_int, [P, P, P, P, P, SZ, SZ, SZ, SZ, P, P]),
        "zgo_model_create": (P, [P, P, SZ, C.c_int]),
        "zgo_model_destroy": (None, [P]),
        "zgo_model_error": (C.c_char_p, [P]),
        "zgo_session_create": (P, [P]),
        "zgo_session_set_kv_bf16": (None, [P, C.c_int]),
        "zgo_session_destroy": (None, [P]),
        "zgo_session_position": (C.c_int, [P]),
        "zgo_forward_token": (C.c_int, [P, C.c_uint32, P]),
        "zgo_state_floats": (SZ, [P]),
        "zgo_state_export": (C.c_int, [P, P, SZ]),
        "zgo_state_import": (C.c_int, [P, P, SZ, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


LIBM_GLIBC, LIBM_CORRECT = 0, 1


def set_libm_mode(mode):
    """Select glibc f32 transcendentals (LIBM_GLIBC, the default: what Rust's
    f32::{exp, ln, sin_cos} call) or correctly rounded ones (LIBM_CORRECT: what
    the HIP kernels compute).  Returns the previous mode."""
    return lib().zgo_set_libm_mode(mode)


class libm_mode:
    """Context manager: run a block with the oracle in the given libm mode."""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        self.old = set_libm_mode(self.mode)
        return self

    def __exit__(self, *exc):
        set_libm_mode(self.old)


def ptr(a):
    return None if a is None else a.ctypes.data_as(P)


class OracleError(RuntimeError):
    def __init__(self, rc, what):
        super().__init__(f"{what}: oracle status {rc}")
        self.rc = rc


def _chk(rc, what):
    if rc != 0:
        raise OracleError(rc, what)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- wrappers

def f16_to_f32(bits):
    return lib().zgo_f16_to_f32(bits)


def f32_to_f16(x):
    return lib().zgo_f32_to_f16_rne(x)


def dequantize(ggml_type, data, elements):
    data = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else data, dtype=np.uint8)
    out = np.empty(elements, np.float32)
    _chk(lib().zgo_dequantize(ggml_type, ptr(data), data.size, elements, ptr(out)), "dequantize")
    return out


def q8_activation(x):
    x = f32(x)
    qs = np.empty(x.size, np.int8)
    d = np.empty(x.size // 32, np.float32)
    s = np.empty(x.size // 32, np.float32)
    _chk(lib().zgo_q8_activation(ptr(x), x.size, ptr(qs), ptr(d), ptr(s)), "q8_activation")
    return qs, d, s


def dot_q8_0_row(row, x):
    qs, d, _ = q8_activation(x)
    row = np.ascontiguousarray(row, np.uint8)
    return lib().zgo_dot_q8_0_row(ptr(row), ptr(qs), ptr(d), x.size // 32)


def q8k_activation(x):
    x = f32(x)
    qs = np.empty(x.size, np.int8)
    d = np.empty(x.size // 256, np.float32)
    bs = np.empty(x.size // 16, np.int32)
    _chk(lib().zgo_q8k_activation(ptr(x), x.size, ptr(qs), ptr(d), ptr(bs)), "q8k_activation")
    return qs, d, bs


def dot_q4_0_row(row, x, repacked=False):
    qs, d, _ = q8_activation(x)
    row = np.ascontiguousarray(row, np.uint8)
    fn = lib().zgo_dot_q4_0_repacked_row if repacked else lib().zgo_dot_q4_0_row
    return fn(ptr(row), ptr(qs), ptr(d), x.size // 32)


def dot_q4_1_row(row, x):
    qs, d, s = q8_activation(x)
    row = np.ascontiguousarray(row, np.uint8)
    return lib().zgo_dot_q4_1_row(ptr(row), ptr(qs), ptr(d), ptr(s), x.size // 32)


def dot_q6k_row(row, x):
    qs, d, bs = q8k_activation(x)
    row = np.ascontiguousarray(row, np.uint8)
    return lib().zgo_dot_q6k_row(ptr(row), ptr(qs), ptr(d), ptr(bs), x.size // 256)


def dot_f32_row(row, x):
    row = np.ascontiguousarray(row, np.uint8)
    x = f32(x)
    return lib().zgo_dot_f32_row(ptr(row), ptr(x), x.size)


def dot_q4k_row(row, x):
    row = np.ascontiguousarray(row, np.uint8)
    x = f32(x)
    return lib().zgo_dot_q4k_row(ptr(row), ptr(x), x.size // 256)


def matvec(ggml_type, w, rows, cols, x, threads=0):
    w = np.ascontiguousarray(w, np.uint8)
    x = f32(x)
    y = np.empty(rows, np.float32)
    _chk(lib().zgo_matvec(ggml_type, ptr(w), w.size, rows, cols, ptr(x), ptr(y), threads), "matvec")
    return y


def rms_norm(x, w, eps):
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    _chk(lib().zgo_rms_norm(ptr(x), ptr(w), x.size, eps, ptr(out)), "rms_norm")
    return out


def grouped_rms_norm(x, w, groups, eps):
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    _chk(lib().zgo_grouped_rms_norm(ptr(x), ptr(w), w.size, groups, eps, ptr(out)), "grouped_rms")
    return out


def silu(x, mult=None):
    x = f32(x)
    m = None if mult is None else f32(mult)
    out = np.empty_like(x)
    _chk(lib().zgo_silu(ptr(x), ptr(m), x.size, ptr(out)), "silu")
    return out


def binary(kind, a, b):
    a, b = f32(a), f32(b)
    out = np.empty_like(a)
    _chk(lib().zgo_binary(kind, ptr(a), ptr(b), a.size, ptr(out)), "binary")
    return out


def gdn_conv_step(act, w, history):
    act, w = f32(act), f32(w)
    hist = f32(history).copy()
    raw = np.empty_like(act)
    _chk(lib().zgo_gdn_conv_step(ptr(act), ptr(w), ptr(hist), ptr(raw), act.size), "gdn_conv")
    return raw, hist


def gdn_coefficients(alpha, beta, dt, a, scale):
    alpha, beta, dt, a = f32(alpha), f32(beta), f32(dt), f32(a)
    n = alpha.size
    gain, bo, sp, gr = (np.empty(n, np.float32) for _ in range(4))
    _chk(lib().zgo_gdn_coefficients(ptr(alpha), ptr(beta), ptr(dt), ptr(a), n, scale, ptr(gain),
                                    ptr(bo), ptr(sp), ptr(gr)), "gdn_coefficients")
    return gain, bo, sp, gr


def source_dot_f32(a, b):
    a, b = f32(a), f32(b)
    return lib().zgo_source_dot_f32(ptr(a), ptr(b), a.size)


def gdn_recurrent_step(state, q, k, v, gain, beta, scale):
    state = f32(state).copy()
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty_like(q)
    _chk(lib().zgo_gdn_recurrent_step(ptr(state), ptr(q), ptr(k), ptr(v), gain, beta, scale,
                                      ptr(out), q.size), "gdn_recurrent")
    return out, state


def rope_kv(q, k, head_width, q_heads, kv_heads, rotate, position, theta_scale):
    q, k = f32(q).copy(), f32(k).copy()
    _chk(lib().zgo_rope_kv(ptr(q), ptr(k), head_width, q_heads, kv_heads, rotate, position,
                           theta_scale), "rope")
    return q, k


def attention_qk(q, keys, head_width, q_heads, kv_heads, scale):
    q, keys = f32(q), f32(keys)
    T = keys.shape[0]
    dots = np.empty(q_heads * T, np.float32)
    scores = np.empty(q_heads * T, np.float32)
    _chk(lib().zgo_attention_qk(ptr(q), ptr(keys), T, head_width, q_heads, kv_heads, scale,
                                ptr(dots), ptr(scores)), "attention_qk")
    return dots, scores


def attention_softmax(scores, heads, width):
    scores = f32(scores)
    exps = np.empty_like(scores)
    probs = np.empty_like(scores)
    sums = np.empty(heads, np.float64)
    _chk(lib().zgo_attention_softmax(ptr(scores), heads, width, ptr(exps), ptr(probs), ptr(sums)),
         "attention_softmax")
    return probs, exps, sums


def attention_value(probs, values, head_width, q_heads, kv_heads, padded=None):
    probs, values = f32(probs), f32(values)
    T = values.shape[0]
    if padded is None:
        padded = (T + 255) // 256 * 256
    out = np.empty(q_heads * head_width, np.float32)
    _chk(lib().zgo_attention_value(ptr(probs), ptr(values), T, head_width, q_heads, kv_heads,
                                   padded, ptr(out)), "attention_value")
    return out


def greedy(logits):
    logits = f32(logits)
    out = C.c_uint32()
    _chk(lib().zgo_greedy(ptr(logits), logits.size, C.byref(out)), "greedy")
    return out.value


def gdn_chunk_prefill(q, k, v, beta, log_decay, heads, d, chunk, state=None):
    q, k, v, beta, log_decay = f32(q), f32(k), f32(v), f32(beta), f32(log_decay)
    T = beta.size // heads
    st = np.zeros(heads * d * d, np.float32) if state is None else f32(state).copy()
    out = np.empty(T * heads * d, np.float32)
    _chk(lib().zgo_gdn_chunk_prefill(ptr(q), ptr(k), ptr(v), ptr(beta), ptr(log_decay), T, heads, d,
                                     chunk, ptr(st), ptr(out)), "gdn_chunk_prefill")
    return out, st


class Model:
    """Oracle model over a tensor table {name: (ggml_type, shape0, shape1, ndarray)}."""

    def __init__(self, geometry: dict, tensors: dict, threads=0):
        self._keep = []
        arr = (Tensor * len(tensors))()
        for i, (name, (t, s0, s1, data)) in enumerate(tensors.items()):
            data = np.ascontiguousarray(data)
            nb = name.encode()
            self._keep += [data, nb]
            arr[i] = Tensor(nb, t, s0, s1, data.ctypes.data_as(P), data.nbytes)
        self._arr = arr
        g = Geometry(**geometry)
        self._g = g
        self.vocab = g.vocab
        self.m = lib().zgo_model_create(C.byref(g), arr, len(tensors), threads)
        err = lib().zgo_model_error(self.m)
        if err:
            raise OracleError(-1, err.decode())

    def session(self, kv_bf16=False):
        return Session(self, kv_bf16)

    def __del__(self):
        if getattr(self, "m", None):
            lib().zgo_model_destroy(self.m)
            self.m = None


class Session:
    def __init__(self, model, kv_bf16=False):
        self.model = model
        self.s = lib().zgo_session_create(model.m)
        if kv_bf16:
            lib().zgo_session_set_kv_bf16(self.s, 1)

    @property
    def position(self):
        return lib().zgo_session_position(self.s)

    def forward(self, token, need_logits=True):
        logits = np.empty(self.model.vocab, np.float32) if need_logits else None
        _chk(lib().zgo_forward_token(self.s, token, ptr(logits)), "forward_token")
        return logits

    def state(self):
        n = lib().zgo_state_floats(self.s)
        out = np.empty(n, np.float32)
        _chk(lib().zgo_state_export(self.s, ptr(out), n), "state_export")
        return out

    def load_state(self, values, position):
        values = f32(values)
        _chk(lib().zgo_state_import(self.s, ptr(values), values.size, position), "state_import")

    def __del__(self):
        if getattr(self, "s", None):
            lib().zgo_session_destroy(self.s)
            self.s = None
