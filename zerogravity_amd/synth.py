"""Seeded synthetic GGUF tensors (no network: every weight is generated here).

Block layouts follow ggml: Q8_0 = [f16 d][32 x i8] (34 B, core/src/encoding.rs:59);
Q4_K = [f16 d][f16 dmin][12 B packed 6-bit scales/mins][128 B nibbles]
(144 B, encoding.rs:60; unpack rule artifacts/src/codecs/q4.rs:39-70);
Q4_1 = [f16 d][f16 m][16 B nibbles] (20 B); Q6_K = [128 B low nibbles][64 B
high 2-bit pairs][16 x i8 scales][f16 d] (210 B, codecs/q6.rs).
"""
import numpy as np

Q8_0, Q4_K, F32, Q4_1, Q6_K = 8, 12, 0, 3, 14


def _f16_bytes(values):
    return np.ascontiguousarray(np.asarray(values, np.float16)).view(np.uint8)


def random_q8_0(rng, rows, cols, scale=None):
    """[rows, cols/32*34] uint8.  Codes ~U[-127,127]; d = scale (f16) per block,
    default 1/(127*sqrt(cols)/sqrt(3)) so each output is O(|x|)."""
    assert cols % 32 == 0
    nb = rows * (cols // 32)
    if scale is None:
        scale = 1.7 / (127.0 * np.sqrt(cols))
    out = np.empty((nb, 34), np.uint8)
    out[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    d = np.full(nb, scale, np.float32) * rng.uniform(0.5, 1.5, nb).astype(np.float32)
    out[:, 0:2] = _f16_bytes(d).reshape(nb, 2)
    return out.reshape(rows, -1)


def random_q4_k(rng, rows, cols, d_scale=None):
    """[rows, cols/256*144] uint8 with random nibbles, random 6-bit scales and
    mins, f16 d and dmin sized so outputs are O(|x|)."""
    assert cols % 256 == 0
    nb = rows * (cols // 256)
    if d_scale is None:
        # std(sc*q - 7.5*mn) is ~258 for uniform 6-bit sc/mn and 4-bit q
        d_scale = 1.0 / (258.0 * np.sqrt(cols))
    out = np.empty((nb, 144), np.uint8)
    out[:, 16:] = rng.integers(0, 256, size=(nb, 128), dtype=np.uint8)
    out[:, 4:16] = rng.integers(0, 256, size=(nb, 12), dtype=np.uint8)
    d = (d_scale * rng.uniform(0.5, 1.5, nb)).astype(np.float32)
    # dmin chosen so the mean weight is near zero: E[sc*q] ~ 31.5*7.5, E[mn] ~ 31.5
    dmin = (d * 7.5 * rng.uniform(0.8, 1.2, nb)).astype(np.float32)
    out[:, 0:2] = _f16_bytes(d).reshape(nb, 2)
    out[:, 2:4] = _f16_bytes(dmin).reshape(nb, 2)
    return out.reshape(rows, -1)


def random_q4_1(rng, rows, cols):
    """[rows, cols/32*20] uint8: random nibbles, d sized so outputs are
    O(|x|), m = -7.5 d (zero-mean weights) with a little jitter."""
    assert cols % 32 == 0
    nb = rows * (cols // 32)
    d = (1.7 / (4.6 * np.sqrt(cols)) * rng.uniform(0.5, 1.5, nb)).astype(np.float32)
    m = (-7.5 * d * rng.uniform(0.9, 1.1, nb)).astype(np.float32)
    out = np.empty((nb, 20), np.uint8)
    out[:, 0:2] = _f16_bytes(d).reshape(nb, 2)
    out[:, 2:4] = _f16_bytes(m).reshape(nb, 2)
    out[:, 4:] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
    return out.reshape(rows, -1)


def random_q6_k(rng, rows, cols):
    """[rows, cols/256*210] uint8: random 6-bit codes, signed local scales in
    [-63, 63], d sized so outputs are O(|x|)."""
    assert cols % 256 == 0
    nb = rows * (cols // 256)
    out = np.empty((nb, 210), np.uint8)
    out[:, :192] = rng.integers(0, 256, size=(nb, 192), dtype=np.uint8)
    out[:, 192:208] = rng.integers(-63, 64, size=(nb, 16), dtype=np.int8).view(np.uint8)
    d = (1.0 / (18.5 * 36.0 * np.sqrt(cols)) * rng.uniform(0.5, 1.5, nb)).astype(np.float32)
    out[:, 208:210] = _f16_bytes(d).reshape(nb, 2)
    return out.reshape(rows, -1)


def random_matrix(rng, kind, rows, cols):
    if kind == Q8_0:
        return random_q8_0(rng, rows, cols)
    if kind == Q4_K:
        return random_q4_k(rng, rows, cols)
    if kind == Q4_1:
        return random_q4_1(rng, rows, cols)
    if kind == Q6_K:
        return random_q6_k(rng, rows, cols)
    if kind == F32:
        return (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32).view(np.uint8).reshape(rows, -1)
    raise ValueError(kind)


def bf16_round(x):
    """Round f32 to bf16 (RNE) and return the f32 values and the raw u16 bits."""
    x = np.ascontiguousarray(x, np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return (r.astype(np.uint32) << 16).view(np.float32), r
