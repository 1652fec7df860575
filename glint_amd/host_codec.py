"""Host (numpy) GLINT codec, used only by the verify gates of the pin tools.

`verify --cuda` compares the device expand against `expand` here, and `verify --parity`
compares a pin's bytes against `encode_f32` here, as the reference's verify gates compare
against its numpy codec (glint_verify.py:85-122). Encode, expand and unpin of the pin
tools themselves run on the device or fail.

The arithmetic is the format's definition (glint_encode.cu:41-114, glint_np.py:16-92):
absmax = largest |w| of each block (NaN skipped); v = w / absmax in f32 (0 for a zero
block); hole = first index of the smallest |v - PARENT[k]|, plug = first index of the
smallest |v - CELLS[hole][j]| (strict '<': NaN and inf give index 0); code (hole, plug) is
stored as two nibble planes, element 2e in the low nibble of byte e, pad nibble 0;
expand = CELLS[hole][plug] * absmax (one f32 product).
"""
from __future__ import annotations

import numpy as np

from . import codebook

CELLS = np.frombuffer(codebook.cells_f32_bytes(), dtype="<f4").reshape(16, 16).copy()
PARENT = np.frombuffer(codebook.parent_f32_bytes(), dtype="<f4").copy()

# source dtype -> function of (raw bytes, element count) giving f32 values
_WIDEN = {
    "BF16": lambda raw, n: np.left_shift(np.frombuffer(raw, "<u2", n).astype(np.uint32), 16).view(np.float32),
    "F16": lambda raw, n: np.frombuffer(raw, "<f2", n).astype(np.float32),
    "F32": lambda raw, n: np.array(np.frombuffer(raw, "<f4", n), dtype=np.float32),
}


def to_f32(dtype: str, raw, n: int) -> np.ndarray:
    """The first n elements of a dense BF16 / F16 / F32 tensor as f32 (exact widening)."""
    try:
        widen = _WIDEN[dtype]
    except KeyError:
        raise ValueError(f"a dense GLINT source is BF16, F16 or F32, not {dtype}") from None
    return widen(raw, n)


def nibbles(packed, n: int) -> np.ndarray:
    """Nibble plane -> one index per element (low nibble first)."""
    b = np.frombuffer(packed, dtype=np.uint8)
    return np.stack([b & 15, b >> 4], axis=1).reshape(-1)[:n]


def pack_nibbles(idx: np.ndarray) -> bytes:
    """One index per element -> nibble plane; an odd count gets a zero pad nibble."""
    idx = np.asarray(idx, dtype=np.uint8)
    pairs = np.zeros(2 * ((idx.size + 1) // 2), np.uint8)
    pairs[:idx.size] = idx
    return (pairs[0::2] | (pairs[1::2] << 4)).tobytes()


def expand(hole, plug, absmax, n: int, blocksize: int, cells=None) -> np.ndarray:
    """f32 weights CELLS[hole][plug] * absmax[i // blocksize] of a pin (cells: a 256-entry
    table to use instead of the built-in one, e.g. a pin's own _glint_cells)."""
    flat = CELLS.reshape(-1) if cells is None else np.asarray(cells, dtype=np.float32).reshape(-1)
    code = (nibbles(hole, n).astype(np.int32) << 4) | nibbles(plug, n)
    scale = np.asarray(absmax, dtype=np.float32)[np.arange(n) // blocksize]
    return flat[code] * scale


def _first_min(v: np.ndarray, table: np.ndarray) -> np.ndarray:
    """Per element, the first k < 16 minimising |v - table[..., k]| (ties and NaN keep the
    earlier index, as a strict '<' scan does)."""
    dist = np.abs(v[:, None] - table)
    dist = np.where(np.isnan(dist), np.inf, dist)
    best = dist.argmin(axis=1)  # first index of the minimum
    best[~np.isfinite(dist.min(axis=1))] = 0  # NaN / inf inputs: no distance beats index 0
    return best.astype(np.uint8)


def encode_f32(w: np.ndarray, blocksize: int, block_chunk: int = 1 << 14):
    """f32 weights -> (hole bytes, plug bytes, absmax f32 array)."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = w.size
    nb = -(-n // blocksize)
    mag = np.zeros(nb * blocksize, np.float32)
    mag[:n] = np.nan_to_num(np.abs(w), nan=0.0, posinf=np.inf)
    absmax = mag.reshape(nb, blocksize).max(axis=1) if nb else np.zeros(0, np.float32)
    hole = np.empty(n, np.uint8)
    plug = np.empty(n, np.uint8)
    span = block_chunk * blocksize
    with np.errstate(invalid="ignore", divide="ignore"):
        for lo in range(0, n, span):
            x = w[lo:lo + span]
            s = absmax[(lo + np.arange(x.size)) // blocksize]
            v = np.where(s == 0, np.float32(0), x / np.where(s == 0, np.float32(1), s)).astype(np.float32)
            h = _first_min(v, PARENT[None, :])
            hole[lo:lo + x.size] = h
            plug[lo:lo + x.size] = _first_min(v, CELLS[h])
    return pack_nibbles(hole), pack_nibbles(plug), absmax.astype(np.float32)


def rms_error(a: np.ndarray, b: np.ndarray) -> float:
    """Root-mean-square of a - b, in f64."""
    if a.size == 0:
        return 0.0
    diff = np.subtract(a, b, dtype=np.float64)
    return float(np.linalg.norm(diff) / np.sqrt(diff.size))
