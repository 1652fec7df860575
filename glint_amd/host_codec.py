"""Host (numpy) GLINT codec for the verify gates of the pin tools, nothing else.

`verify --cuda` compares the GPU expand with this expand, and `verify --parity`
compares a pin's bytes with this encode, the way the reference's verify gates use its
numpy codec (glint_verify.py:85-122, glint_np.py:16-95). The GPU paths never call
it: encode, expand and unpin run on the device or fail.

Encode rule (glint_encode.cu:41-102): absmax = max |w| per block (NaN skipped),
v = (s == 0) ? 0 : w / s (f32 division), hole = first index of the smallest
|v - PARENT[k]|, plug = first index of the smallest |v - CELLS[hole][j]| (strict '<',
so NaN and inf give 0), element 2e in the low nibble of byte e, pad nibble 0.
"""
from __future__ import annotations

import numpy as np

from . import codebook

CELLS = np.frombuffer(codebook.cells_f32_bytes(), dtype="<f4").reshape(16, 16).copy()
PARENT = np.frombuffer(codebook.parent_f32_bytes(), dtype="<f4").copy()


def dense_to_f32(dtype: str, raw, n: int) -> np.ndarray:
    if dtype == "BF16":
        return (np.frombuffer(raw, dtype="<u2", count=n).astype(np.uint32) << 16).view(np.float32)
    if dtype == "F16":
        return np.frombuffer(raw, dtype="<f2", count=n).astype(np.float32)
    if dtype == "F32":
        return np.frombuffer(raw, dtype="<f4", count=n).astype(np.float32)
    raise ValueError(f"dense unpack does not support dtype {dtype}")


def unpack_nibbles(packed, n: int) -> np.ndarray:
    b = np.frombuffer(packed, dtype=np.uint8)
    out = np.empty(2 * b.size, np.uint8)
    out[0::2] = b & 15
    out[1::2] = b >> 4
    return out[:n]


def pack_nibbles(idx: np.ndarray) -> bytes:
    if idx.size & 1:
        idx = np.concatenate([idx, np.zeros(1, np.uint8)])
    return (idx[0::2] | (idx[1::2] << 4)).astype(np.uint8).tobytes()


def expand(hole, plug, absmax: np.ndarray, n: int, blocksize: int, cells=None) -> np.ndarray:
    tab = CELLS if cells is None else np.asarray(cells, dtype=np.float32).reshape(16, 16)
    s = np.repeat(np.asarray(absmax, dtype=np.float32), blocksize)[:n]
    return tab[unpack_nibbles(hole, n), unpack_nibbles(plug, n)] * s


def _first_nearest(v: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """First index of the smallest |v - rows[:, k]| over k < 16, strict '<'."""
    best = np.zeros(v.shape, np.uint8)
    bd = np.abs(v - rows[:, 0])
    for k in range(1, 16):
        d = np.abs(v - rows[:, k])
        t = d < bd
        best[t] = k
        bd = np.where(t, d, bd)
    return best


def encode_f32(w: np.ndarray, blocksize: int, chunk_blocks: int = 1 << 16):
    """-> (hole bytes, plug bytes, absmax f32 array)."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = w.size
    nb = (n + blocksize - 1) // blocksize
    a = np.abs(w)
    a = np.where(np.isnan(a), np.float32(0), a)
    a = np.concatenate([a, np.zeros(nb * blocksize - n, np.float32)]).reshape(nb, blocksize)
    am = a.max(axis=1) if nb else np.zeros(0, np.float32)
    h = np.empty(n, np.uint8)
    p = np.empty(n, np.uint8)
    step = chunk_blocks * blocksize
    with np.errstate(invalid="ignore", divide="ignore"):
        for i0 in range(0, n, step):
            x = w[i0:i0 + step]
            s = np.repeat(am, blocksize)[i0:i0 + x.size]
            v = np.where(s == 0, np.float32(0), x / np.where(s == 0, np.float32(1), s)).astype(np.float32)
            hh = _first_nearest(v, np.broadcast_to(PARENT, (v.size, 16)))
            h[i0:i0 + x.size] = hh
            p[i0:i0 + x.size] = _first_nearest(v, CELLS[hh])
    return pack_nibbles(h), pack_nibbles(p), am.astype(np.float32)


def rmse(a: np.ndarray, b: np.ndarray) -> float:
    d = a.astype(np.float64) - b.astype(np.float64)
    return float(np.sqrt(np.mean(d * d))) if d.size else 0.0
