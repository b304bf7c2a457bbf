"""ctypes binding of libzg_hip.so (the gfx950 backend).

There is no CPU fallback anywhere in this package: if the HIP library is not
built, or no GPU is visible, these functions raise.
"""
import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzg_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "zg_hip.h")

COMPLETED, UNSUPPORTED = 0, 1
E_MALFORMED, E_UNSUPPORTED, E_RESOURCE, E_LIMIT, E_STATE, E_DEVICE = -1, -2, -3, -4, -5, -6
F32, F16, Q8_0, Q4_K, BF16 = 0, 1, 8, 12, 30

_lib = None
P = C.c_void_p
SZ = C.c_size_t
FP = C.POINTER(C.c_float)

_SIGS = {
    "zg_version": (C.c_char_p, []),
    "zg_ctx_create": (C.c_int, [C.c_int, C.POINTER(P)]),
    "zg_ctx_destroy": (None, [P]),
    "zg_last_error": (C.c_char_p, [P]),
    "zg_weight_register": (C.c_int, [P, C.c_uint64, C.c_char_p, C.c_int, SZ, SZ, P, SZ, C.POINTER(P)]),
    "zg_source_release": (C.c_int, [P, C.c_uint64]),
    "zg_weight_device_bytes": (SZ, [P]),
    "zg_weight_dequantize": (C.c_int, [P, P, P, SZ]),
    "zg_matvec": (C.c_int, [P, C.c_uint64, C.c_char_p, C.c_int, SZ, SZ, P, SZ, P, SZ, P, SZ]),
    "zg_embedding": (C.c_int, [P, C.c_uint64, C.c_char_p, C.c_int, P, SZ, C.c_uint32, SZ, SZ, P, SZ]),
    "zg_rms_norm": (C.c_int, [P, P, P, SZ, C.c_float, P]),
    "zg_grouped_rms_norm": (C.c_int, [P, P, P, SZ, SZ, C.c_float, P]),
    "zg_silu": (C.c_int, [P, P, P, SZ, P]),
    "zg_binary": (C.c_int, [P, C.c_int, P, P, SZ, P]),
    "zg_gemv_device": (C.c_int, [P, P, P, C.c_int, SZ, P, C.c_float, P, P]),
    "zg_gemv_device_fused": (C.c_int, [P, P, SZ, C.c_int, C.c_int, P, SZ, P, SZ, P, C.c_float, SZ, P, SZ, P, P, P,
                                       P, P]),
    "zg_gemv_greedy_parts": (SZ, [P]),
    "zg_gdn_conv": (C.c_int, [P, P, P, P, SZ, P, P]),
    "zg_gdn_coefficients": (C.c_int, [P, P, P, P, P, SZ, C.c_float, P, P, P, P]),
    "zg_gdn_recurrent": (C.c_int, [P, SZ, SZ, P, P, P, P, P, P, P]),
    "zg_gdn_chunk": (C.c_int, [P, SZ, SZ, P, P, P, P, P, P, P, P]),
    "zg_gdn_chunk_scratch_bytes": (SZ, [SZ, SZ]),
    "zg_gdn_chunk_prefill_device": (C.c_int, [P, SZ, SZ, P, P, P, P, P, P, P, P]),
    "zg_gdn_decode_device": (C.c_int, [P, SZ, SZ, P, SZ, P, P, P, P, P, C.c_float, P, P, P]),
    "zg_rope_kv": (C.c_int, [P, P, P, P, SZ, SZ, SZ, SZ, SZ, C.c_float, P, P, P]),
    "zg_attention_qk": (C.c_int, [P, P, P, SZ, SZ, SZ, SZ, C.c_float, P, P]),
    "zg_attention_softmax": (C.c_int, [P, P, SZ, SZ, P]),
    "zg_attention_value": (C.c_int, [P, P, P, SZ, SZ, SZ, SZ, P]),
    "zg_model_admit": (C.c_int, [C.c_int, P, P, SZ, C.c_char_p, SZ]),
    "zg_model_load": (C.c_int, [P, C.c_uint64, P, P, SZ, C.POINTER(P)]),
    "zg_model_destroy": (None, [P]),
    "zg_session_create": (C.c_int, [P, SZ, SZ, C.c_int, C.POINTER(P)]),
    "zg_session_destroy": (None, [P]),
    "zg_session_reset": (C.c_int, [P]),
    "zg_session_position": (C.c_int, [P, SZ]),
    "zg_decode_step": (C.c_int, [P, SZ, P, P, P]),
    "zg_prefill": (C.c_int, [P, SZ, SZ, P, P]),
    "zg_prefill_batched": (C.c_int, [P, SZ, SZ, P, P]),
    "zg_attn_decode_workspace_bytes": (SZ, [SZ, SZ, SZ]),
    "zg_attn_decode_split_workspace_bytes": (SZ, [SZ, SZ, SZ, SZ]),
    "zg_attn_decode_split_device": (C.c_int, [P, SZ, SZ, SZ, P, SZ, P, P, C.c_float, C.c_float, P, P, P, SZ, C.c_int,
                                              P, P, P]),
    "zg_attn_decode_device": (C.c_int, [P, SZ, SZ, SZ, P, SZ, P, P, C.c_float, C.c_float, P, P, P, SZ, C.c_int, P, P,
                                        P]),
    "zg_session_reset_row": (C.c_int, [P, SZ]),
    "zg_session_copy_row": (C.c_int, [P, SZ, SZ]),
    "zg_decode_step_device": (C.c_int, [P, SZ, P, P, P, P]),
    "zg_session_check": (C.c_int, [P, P]),
    "zg_state_floats": (SZ, [P, SZ]),
    "zg_state_export": (C.c_int, [P, SZ, P, SZ]),
    "zg_state_import": (C.c_int, [P, SZ, P, SZ, C.c_int]),
    "zg_session_fill_random": (C.c_int, [P, SZ, SZ, C.c_uint64]),
    "zg_act_prepared_bytes": (SZ, [P, SZ]),
    "zg_act_prepare_device": (C.c_int, [P, P, P, C.c_int, SZ, P, C.c_float, P, SZ, P]),
    "zg_gemv_prepared_device": (C.c_int, [P, P, SZ, P, P, P]),
    "zg_greedy": (C.c_int, [P, P, SZ, SZ, P]),
    "zg_gemv_device_noalloc": (C.c_int, [P, P, P, C.c_int, SZ, P, C.c_float, P, P]),
    "zg_gdn_decode_tiles_bytes": (SZ, [SZ, SZ]),
    "zg_gdn_decode_gated_device": (C.c_int, [P, SZ, SZ, P, SZ, P, P, P, P, P, P, C.c_float, P, P, P, P]),
    "zg_session_propose": (C.c_int, [P, SZ, P, P, P]),
    "zg_session_commit": (C.c_int, [P]),
    "zg_session_snapshot": (C.c_int, [P, SZ, C.POINTER(P)]),
    "zg_session_restore": (C.c_int, [P, SZ, P]),
    "zg_snapshot_bytes": (SZ, [P]),
    "zg_snapshot_position": (C.c_int, [P]),
    "zg_snapshot_destroy": (None, [P]),
}


def header_symbols():
    """Every function the public header declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zg_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        # One HIP runtime per process: when torch (which ships its own
        # libamdhip64) is importable, load it first so this library binds to
        # the same runtime instead of pulling in a second one.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP backend first (python -c 'import __graft_entry__ as g; g.build()')")
        _lib = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


class ZgError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"zg status {code}: {msg}")
        self.code = code


class Context:
    """One device context (zg_ctx) with its own stream and weight cache."""

    def __init__(self, device=0):
        h = P()
        rc = lib().zg_ctx_create(device, C.byref(h))
        if rc != COMPLETED:
            raise ZgError(rc, "zg_ctx_create failed (no usable HIP device?)")
        self.h = h
        self._dependents = []  # weakrefs to models/sessions living on this ctx

    def adopt(self, obj):
        """Register an object whose native handle lives on this context; it is
        closed before the context is destroyed, whatever the teardown order."""
        import weakref
        self._dependents.append(weakref.ref(obj))

    def error(self):
        return lib().zg_last_error(self.h).decode()

    def check(self, rc):
        if rc < 0:
            raise ZgError(rc, self.error())
        return rc

    def close(self):
        if getattr(self, "h", None):
            for ref in reversed(self._dependents):
                obj = ref()
                if obj is not None:
                    obj.close()
            self._dependents = []
            lib().zg_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter teardown: the library may be gone; the process releases the device
            pass
