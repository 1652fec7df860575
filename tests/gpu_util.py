"""Helpers for the GPU parity tests (device buffers via torch, checks via the oracle)."""
import numpy as np
import pytest


def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def dev(a: np.ndarray, pad_front: int = 0):
    """Copy a numpy array to the GPU (uint16 travels as int16 bits). With pad_front > 0
    the returned tensor is a view pad_front elements into a larger allocation, i.e. a
    pointer that is not 16-byte aligned."""
    torch = torch_cuda()
    a = np.ascontiguousarray(a).reshape(-1)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    t = torch.from_numpy(a.copy())
    if pad_front:
        big = torch.zeros(a.size + pad_front, dtype=t.dtype)
        big[pad_front:] = t
        return big.cuda()[pad_front:]
    return t.cuda()


def host(t, dtype=None) -> np.ndarray:
    torch = torch_cuda()
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def bf16_bits(a: np.ndarray) -> np.ndarray:
    from oracle.glint_oracle import f32_to_bf16_bits
    return f32_to_bf16_bits(np.asarray(a, np.float32))


def first_diff(a: np.ndarray, b: np.ndarray):
    a, b = np.asarray(a).reshape(-1), np.asarray(b).reshape(-1)
    if a.shape != b.shape:
        return f"shape {a.shape} != {b.shape}"
    d = np.flatnonzero(a != b)
    return None if d.size == 0 else f"{d.size} differ, first at {d[0]}: {a[d[0]]} vs {b[d[0]]}"
