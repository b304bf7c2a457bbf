"""Chunked (WY/UT) Gated DeltaNet prefill on the GPU.

`core(ctx, ChunkInputs)` mirrors the reference's one-chunk entry
    pub fn core(input: ChunkInputs<'_>) -> Result<ChunkCompleted>
(cpu/src/numerics/torch_cpu/gdn/chunk/core.rs:8-23, 69-274): the same
fields, the same input checks (an `Err` becomes `ZgError(E_MALFORMED)`),
key-major state [heads][128 key][128 value] and bf16-rounded outputs.

`prefill_device` runs any number of 64-token chunks in order over device
buffers (torch tensors or raw pointers) with the value-major state the
decode recurrence uses; it is the entry the prefill benchmark times.
"""
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib as L

ORDER = 64   # chunk rows (gdn/chunk.rs:4)
WIDTH = 128  # head width (gdn/chunk.rs:5)


@dataclass
class ChunkInputs:
    """core.rs:8-18; q/k/v [rows][heads][128], beta/log_decay [rows][heads]."""
    rows: int
    heads: int
    query: np.ndarray
    key: np.ndarray
    value: np.ndarray
    beta: np.ndarray
    log_decay: np.ndarray
    previous_state: Optional[np.ndarray] = None


@dataclass
class ChunkCompleted:
    """core.rs:20-23"""
    output_bf16: np.ndarray
    state: np.ndarray


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def core(ctx: "L.Context", inp: ChunkInputs) -> ChunkCompleted:
    q, k, v = _f32(inp.query), _f32(inp.key), _f32(inp.value)
    b, g = _f32(inp.beta), _f32(inp.log_decay)
    n, nb = inp.rows * inp.heads * WIDTH, inp.rows * inp.heads
    if q.size != n or k.size != n or v.size != n or b.size != nb or g.size != nb:
        raise L.ZgError(L.E_MALFORMED, "source chunk grouped input/state geometry")
    prev = None if inp.previous_state is None else _f32(inp.previous_state)
    if prev is not None and prev.size != inp.heads * WIDTH * WIDTH:
        raise L.ZgError(L.E_MALFORMED, "source chunk grouped input/state geometry")
    out = np.empty(n, np.float32)
    st = np.empty(inp.heads * WIDTH * WIDTH, np.float32)
    p = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    ctx.check(L.lib().zg_gdn_chunk(ctx.h, inp.rows, inp.heads, p(q), p(k), p(v), p(b), p(g), p(prev), p(out),
                                   p(st)))
    return ChunkCompleted(out, st)


def scratch_bytes(tokens: int, heads: int) -> int:
    return int(L.lib().zg_gdn_chunk_scratch_bytes(tokens, heads))


def _ptr(t):
    return t if isinstance(t, int) else t.data_ptr()


def prefill_device(ctx: "L.Context", tokens, heads, query, key, value, beta, log_decay, state, output, stream=None):
    """zg_gdn_chunk_prefill_device on device buffers (f32, contiguous)."""
    for t in (query, key, value, beta, log_decay, state, output):
        if not isinstance(t, int) and (not t.is_cuda or not t.is_contiguous() or t.dtype.itemsize != 4):
            raise L.ZgError(L.E_MALFORMED, "chunk prefill wants contiguous f32 device tensors")
    ctx.check(L.lib().zg_gdn_chunk_prefill_device(ctx.h, tokens, heads, _ptr(query), _ptr(key), _ptr(value),
                                                  _ptr(beta), _ptr(log_decay), _ptr(state), _ptr(output),
                                                  stream))
