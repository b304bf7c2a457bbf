"""Host-side mirror of the reference's per-region operator API.

`HipMatVecKernel` is the device implementation of the reference trait
    pub trait MatVecKernel: Send + Sync { fn try_execute(..); fn try_rms_norm(..); .. }
(core/src/accelerator.rs:682-731), with the same region structs
(accelerator.rs:61-655) as dataclasses and the same three outcomes
(accelerator.rs:671-681): `Completed(values)`, `Unsupported`, or an
exception (`Err`), after which a caller must abort, never fall back.
"""
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib as L


class Unsupported:
    """RegionExecution::Unsupported — the caller may run its CPU operator."""

    def __repr__(self):
        return "Unsupported"


UNSUPPORTED = Unsupported()


@dataclass
class Completed:
    """RegionExecution::Completed — device work finished and read back."""
    values: np.ndarray


@dataclass(frozen=True)
class SourceIdentity:
    """accelerator.rs:22-59; 0 is the reserved unbound identity."""
    value: int

    @staticmethod
    def unbound():
        return SourceIdentity(0)

    def is_bound(self):
        return self.value != 0


@dataclass
class MatVecRegion:
    """accelerator.rs:61-75"""
    source_identity: SourceIdentity
    tensor_name: str
    kind: int  # ggml type code
    columns: int
    rows: int
    packed_weights: np.ndarray  # uint8
    activation: np.ndarray  # f32[columns]


@dataclass
class RmsNormRegion:
    """accelerator.rs:77-88"""
    source_identity: SourceIdentity
    tensor_name: str
    input: np.ndarray
    weights: np.ndarray
    eps: float


@dataclass
class GroupedRmsNormRegion:
    """accelerator.rs:90-104"""
    source_identity: SourceIdentity
    tensor_name: str
    input: np.ndarray
    weights: np.ndarray
    group_width: int
    groups: int
    eps: float


@dataclass
class SiluRegion:
    """accelerator.rs:509-530"""
    source_identity: SourceIdentity
    operation: str
    input: np.ndarray
    multiplier: Optional[np.ndarray] = None


@dataclass
class BinaryRegion:
    """accelerator.rs:383-416; kind 0 = Add, 1 = SigmoidGate"""
    source_identity: SourceIdentity
    operation: str
    kind: int
    left: np.ndarray
    right: np.ndarray


@dataclass
class EmbeddingRegion:
    """accelerator.rs:417-453"""
    source_identity: SourceIdentity
    tensor_name: str
    kind: int
    packed_weights: np.ndarray
    token: int
    width: int
    vocabulary: int


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def _p(a):
    return None if a is None else a.ctypes.data


class HipMatVecKernel:
    """MatVecKernel implemented on one MI355X through libzg_hip.so."""

    def __init__(self, device=0):
        self.ctx = L.Context(device)
        self._lib = L.lib()

    def _result(self, rc, out):
        if rc == L.UNSUPPORTED:
            return UNSUPPORTED
        self.ctx.check(rc)
        return Completed(out)

    # accelerator.rs:683
    def try_execute(self, r: MatVecRegion):
        w = _u8(r.packed_weights)
        x = _f32(r.activation)
        out = np.empty(r.rows, np.float32)
        rc = self._lib.zg_matvec(self.ctx.h, r.source_identity.value, r.tensor_name.encode(), r.kind, r.columns,
                                 r.rows, _p(w), w.size, _p(x), x.size, _p(out), out.size)
        return self._result(rc, out)

    def try_rms_norm(self, r: RmsNormRegion):
        x, g = _f32(r.input), _f32(r.weights)
        if x.size != g.size:
            raise L.ZgError(L.E_MALFORMED, "invalid Qwen RMSNorm source geometry")
        out = np.empty_like(x)
        return self._result(self._lib.zg_rms_norm(self.ctx.h, _p(x), _p(g), x.size, r.eps, _p(out)), out)

    def try_grouped_rms_norm(self, r: GroupedRmsNormRegion):
        x, g = _f32(r.input), _f32(r.weights)
        if g.size != r.group_width or x.size != r.group_width * r.groups:
            raise L.ZgError(L.E_MALFORMED, "invalid grouped source RMS normalization dimensions")
        out = np.empty_like(x)
        rc = self._lib.zg_grouped_rms_norm(self.ctx.h, _p(x), _p(g), r.group_width, r.groups, r.eps, _p(out))
        return self._result(rc, out)

    def try_silu(self, r: SiluRegion):
        x = _f32(r.input)
        m = None if r.multiplier is None else _f32(r.multiplier)
        if m is not None and m.size != x.size:
            raise L.ZgError(L.E_MALFORMED, "invalid source SiLU inputs")
        out = np.empty_like(x)
        return self._result(self._lib.zg_silu(self.ctx.h, _p(x), _p(m), x.size, _p(out)), out)

    def try_binary(self, r: BinaryRegion):
        a, b = _f32(r.left), _f32(r.right)
        if a.size != b.size:
            raise L.ZgError(L.E_MALFORMED, "invalid source binary region")
        out = np.empty_like(a)
        return self._result(self._lib.zg_binary(self.ctx.h, r.kind, _p(a), _p(b), a.size, _p(out)), out)

    def try_embedding(self, r: EmbeddingRegion):
        w = _u8(r.packed_weights)
        out = np.empty(r.width, np.float32)
        rc = self._lib.zg_embedding(self.ctx.h, r.source_identity.value, r.tensor_name.encode(), r.kind, _p(w), w.size,
                                    r.token, r.width, r.vocabulary, _p(out), out.size)
        return self._result(rc, out)

    # ------------------------------------------------------------ weights

    def register(self, source_id, name, kind, columns, rows, packed):
        """Resident weight handle (zg_weight_register)."""
        import ctypes as C
        w = _u8(packed)
        h = C.c_void_p()
        self.ctx.check(self._lib.zg_weight_register(self.ctx.h, source_id, name.encode(), kind, columns, rows, _p(w),
                                                    w.size, C.byref(h)))
        return Weight(self, h, kind, columns, rows)

    def release_source(self, source_id):
        self.ctx.check(self._lib.zg_source_release(self.ctx.h, source_id))


class Weight:
    def __init__(self, kernel, handle, kind, columns, rows):
        self.kernel, self.h, self.kind, self.columns, self.rows = kernel, handle, kind, columns, rows

    @property
    def device_bytes(self):
        return self.kernel._lib.zg_weight_device_bytes(self.h)

    def dequantize(self):
        out = np.empty(self.rows * self.columns, np.float32)
        self.kernel.ctx.check(self.kernel._lib.zg_weight_dequantize(self.kernel.ctx.h, self.h, _p(out), out.size))
        return out.reshape(self.rows, self.columns)


def validate_completed(region: MatVecRegion, values: Sequence[float]):
    """core/src/accelerator.rs:734-744: a Completed GEMV must hold `rows`
    finite values, else the proposal is aborted (Error::State)."""
    v = np.asarray(values)
    if v.size != region.rows or not np.isfinite(v).all():
        raise L.ZgError(L.E_STATE, f"accelerator returned invalid or incomplete output for '{region.tensor_name}'")
