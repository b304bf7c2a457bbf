"""GGUF v3 reader/writer for the tensor table the resident model loads.

Reader rules follow the reference parser parse_gguf
(crates/zerogravity-artifacts/src/artifact.rs:539-672): little-endian v3
only; unique non-empty metadata keys and tensor names; general.alignment a
power of two in 8..4096 (default 32); rank 1..8; ne0 a multiple of the codec
block; tensor offsets aligned; data after the aligned table end; tensors
inside the file and non-overlapping.  Type codes: core/src/encoding.rs:77-91.
"""
import mmap
import struct
from dataclasses import dataclass

import numpy as np

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34),
         Q4_K: (256, 144), Q6_K: (256, 210)}

# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<?",
           _U64: "<Q", _I64: "<q", _F64: "<d"}


class GgufError(ValueError):
    pass


@dataclass
class TensorInfo:
    name: str
    shape: tuple  # GGML order: (ne0, ne1, ...)
    ggml_type: int
    offset: int  # absolute byte offset in the file
    nbytes: int


def byte_len(ggml_type, elements):
    if ggml_type not in BLOCK:
        raise GgufError(f"GGUF ggml tensor type {ggml_type}: no validated byte codec")
    be, bb = BLOCK[ggml_type]
    if elements % be:
        raise GgufError("element count not a whole number of blocks")
    return elements // be * bb


class _Reader:
    def __init__(self, buf):
        self.b = buf
        self.p = 0

    def take(self, n):
        if self.p + n > len(self.b):
            raise GgufError("GGUF truncated")
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def string(self, limit):
        n = self.u64()
        if n > limit:
            raise GgufError("GGUF string too long")
        return bytes(self.take(n)).decode("utf-8")

    def value(self, ty, depth=0):
        if ty in _SCALAR:
            fmt = _SCALAR[ty]
            return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
        if ty == _STR:
            return self.string(1 << 24)
        if ty == _ARR:
            if depth > 2:
                raise GgufError("GGUF nested array depth")
            ety = self.u32()
            n = self.u64()
            if n > (1 << 24):
                raise GgufError("GGUF array too long")
            return [self.value(ety, depth + 1) for _ in range(n)]
        raise GgufError(f"GGUF metadata type {ty}")


class GgufFile:
    """Parsed GGUF file; tensor data are zero-copy numpy views of an mmap."""

    def __init__(self, path):
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        self.metadata, self.tensors = parse(memoryview(self._mm), len(self._mm))

    @property
    def architecture(self):
        return self.metadata.get("general.architecture")

    def data(self, name):
        t = self.tensors[name]
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)

    def close(self):
        """Release the mapping; views handed out by data() keep it alive
        until they are dropped."""
        self.tensors = {}
        try:
            self._mm.close()
        except BufferError:
            pass
        self._f.close()


def parse(buf, file_len):
    r = _Reader(buf)
    if bytes(r.take(4)) != b"GGUF":
        raise GgufError("invalid GGUF magic")
    if r.u32() != 3:
        raise GgufError("only little-endian GGUF v3 is implemented")
    n, m = r.u64(), r.u64()
    if n > 1 << 20 or m > 1 << 20:
        raise GgufError("GGUF tensor/metadata count too large")
    meta = {}
    align = 32
    for _ in range(m):
        key = r.string(1 << 16)
        if not key or key in meta:
            raise GgufError("empty or duplicate GGUF metadata key")
        ty = r.u32()
        val = r.value(ty)
        if key == "general.architecture" and ty != _STR:
            raise GgufError("GGUF architecture is not string")
        if key == "general.alignment":
            if ty not in (_U32, _U64):
                raise GgufError("GGUF alignment is not unsigned integer")
            if not (8 <= val <= 4096) or val & (val - 1):
                raise GgufError("GGUF alignment must be power of two 8..4096")
            align = val
        meta[key] = val
    infos = []
    names = set()
    for _ in range(n):
        name = r.string(64)
        if not name or name in names:
            raise GgufError("GGUF duplicate/empty tensor name")
        names.add(name)
        rank = r.u32()
        if rank == 0 or rank > 8:
            raise GgufError("GGUF rank must be 1..8")
        shape = tuple(r.u64() for _ in range(rank))
        ty = r.u32()
        if ty not in BLOCK:
            raise GgufError(f"GGUF ggml tensor type {ty}: no validated byte codec")
        if shape[0] % BLOCK[ty][0]:
            raise GgufError("GGUF quantized row not aligned to full blocks")
        rel = r.u64()
        if rel % align:
            raise GgufError("unaligned GGUF tensor offset")
        elements = int(np.prod(shape, dtype=np.uint64))
        infos.append((name, shape, ty, rel, byte_len(ty, elements)))
    start = (r.p + align - 1) // align * align
    if start > file_len:
        raise GgufError("GGUF table extends past EOF")
    tensors = {}
    ranges = []
    for name, shape, ty, rel, nb in infos:
        off = start + rel
        if off + nb > file_len:
            raise GgufError(f"GGUF tensor '{name}' extends beyond EOF")
        ranges.append((off, off + nb))
        tensors[name] = TensorInfo(name, shape, ty, off, nb)
    ranges.sort()
    for a, b in zip(ranges, ranges[1:]):
        if b[0] < a[1]:
            raise GgufError("GGUF tensor regions overlap")
    return meta, tensors


def _kv(key, value):
    kb = key.encode()
    out = struct.pack("<Q", len(kb)) + kb
    if isinstance(value, str):
        vb = value.encode()
        return out + struct.pack("<IQ", _STR, len(vb)) + vb
    if isinstance(value, bool):
        return out + struct.pack("<I?", _BOOL, value)
    if isinstance(value, int):
        return out + struct.pack("<II", _U32, value)
    if isinstance(value, float):
        return out + struct.pack("<If", _F32, value)
    raise TypeError(value)


def write(path, tensors, metadata, alignment=32):
    """tensors: list of (name, ggml_type, shape (GGML order), uint8 ndarray)."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata) + 1)
    head += _kv("general.alignment", alignment)
    for k, v in metadata.items():
        head += _kv(k, v)
    off = 0
    table = b""
    offsets = []
    for name, ty, shape, data in tensors:
        nb = name.encode()
        assert data.nbytes == byte_len(ty, int(np.prod(shape))), name
        table += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(shape))
        table += b"".join(struct.pack("<Q", d) for d in shape)
        table += struct.pack("<IQ", ty, off)
        offsets.append(off)
        off += (data.nbytes + alignment - 1) // alignment * alignment
    body = head + table
    pad = (-len(body)) % alignment
    with open(path, "wb") as f:
        f.write(body + b"\0" * pad)
        for (name, ty, shape, data), o in zip(tensors, offsets):
            f.write(np.ascontiguousarray(data).view(np.uint8).data)
            f.write(b"\0" * ((-data.nbytes) % alignment))
