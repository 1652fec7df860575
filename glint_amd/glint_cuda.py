"""Drop-in for the reference's ``glint_cuda.py`` (same module name, functions,
argument meaning and errors), backed by the MI355X ``libglint_encode.so``.

Reference: glint_cuda.py:9-85. Callers such as ``glint_pin.py`` / ``glint_verify.py`` that
``import glint_cuda`` get the same API: ``lib_path``, ``load``, ``encode_bf16_cuda``,
``expand_cuda``, ``gpu_ok``. ``load()`` returns None when the library is absent (as the
reference does); the encode/expand functions then raise RuntimeError.
"""
from __future__ import annotations

from pathlib import Path
from typing import Optional, Tuple

from . import glint_hip

_ERR: Optional[str] = None


def lib_path() -> Optional[Path]:
    return glint_hip.encode_lib_path()


def load():
    global _ERR
    try:
        return glint_hip.encode_lib()
    except (RuntimeError, OSError) as e:
        _ERR = str(e)
        return None


def encode_bf16_cuda(raw_bf16: bytes, n: int, blocksize: int = 64) -> Tuple[bytes, bytes, bytes]:
    if load() is None:
        raise RuntimeError(_ERR)
    return glint_hip.encode_bf16_host(raw_bf16, n, blocksize)


def expand_cuda(hole: bytes, plug: bytes, absmax_f32: bytes, n: int, blocksize: int = 64) -> bytes:
    """GPU expand -> n little-endian f32."""
    if load() is None:
        raise RuntimeError(_ERR)
    return glint_hip.expand_host(hole, plug, absmax_f32, n, blocksize)


def gpu_ok() -> bool:
    """Library loads and a 2-weight encode runs. False on a box with no GPU."""
    try:
        encode_bf16_cuda(b"\x80\x3f\x00\x00", 2, 64)
        return True
    except (RuntimeError, OSError):
        return False
