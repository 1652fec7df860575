"""TEST INFRASTRUCTURE ONLY — the CPU oracle for GLINT's hot path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this,
and only as the checker; the product (glint_amd/) never does.

Two restatements of the reference's host path:

* numpy functions restating ``glint_np.py`` op for op (block absmax in f32, f32 divide,
  searchsorted nearest with a left/right compare, lo-then-hi nibbles, RNE to BF16);
* ``Oracle``: ctypes over ``oracle/liboracle.so`` (glint_oracle.c), the linear-scan C
  restatement of the reference kernels' arithmetic, used for larger sizes.

Plus ``codec_encode_f64``, a pure-Python restatement of the reference's f64
``glint_codec.encode`` (glint_codec.py:119-149), used only to pin the f32 path on the
reference's own seeded test data.
"""
from __future__ import annotations

import ctypes
import os
import struct
from pathlib import Path
from typing import List, Sequence, Tuple

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent


def _load_tables() -> Tuple[np.ndarray, np.ndarray]:
    """Parse the committed C header (the table the product compiles in)."""
    import re
    text = (ROOT / "include" / "glint_cells.h").read_text()
    nums = [float(x[:-1]) for x in re.findall(r"[-+0-9.]+e[-+][0-9]+f", text)]
    assert len(nums) == 256 + 16, len(nums)
    cells = np.asarray(nums[:256], dtype=np.float32).reshape(16, 16)
    parent = np.asarray(nums[256:], dtype=np.float32)
    return cells, parent


CELLS_F32, PARENT_F32 = _load_tables()
CELLS_FLAT = CELLS_F32.reshape(-1)  # strictly ascending across rows


# ---------------------------------------------------------------- numpy restatement
def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    """glint_np.py:16-20 (BF16 branch of dense_to_f32)."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(w: np.ndarray) -> np.ndarray:
    """glint_np.py:25-31: round to nearest even; NaN -> (u >> 16) | 0x40."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    u = w.view(np.uint32)
    rounded = (u + (np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1)))) >> 16
    return np.where(np.isnan(w), (u >> 16) | np.uint32(0x40), rounded).astype(np.uint16)


def block_absmax(w: np.ndarray, bs: int) -> np.ndarray:
    """glint_np.py:32-40: per-block max |w| with NaN treated as 0."""
    n = w.size
    nb = (n + bs - 1) // bs
    a = np.abs(w)
    a = np.where(np.isnan(a), np.float32(0), a)
    pad = nb * bs - n
    if pad:
        a = np.concatenate([a, np.zeros(pad, dtype=np.float32)])
    return a.reshape(nb, bs).max(axis=1) if nb else np.zeros(0, np.float32)


def nearest(v: np.ndarray, flat: np.ndarray, lo, width: int = 16) -> np.ndarray:
    """glint_np.py:41-52: index in [lo, lo+width) of the nearest entry, minus lo; a tie
    goes to the lower index; NaN/inf -> 0."""
    pos = np.searchsorted(flat, v, side="left").astype(np.int64)
    pos = np.clip(pos, np.asarray(lo) + 1, np.asarray(lo) + width - 1)
    left = flat[pos - 1]
    right = flat[pos]
    take_right = np.abs(v - right) < np.abs(v - left)
    idx = pos - 1 + take_right - lo
    return np.where(np.isfinite(v), idx, 0).astype(np.uint8)


def pack_nibbles(idx: np.ndarray) -> np.ndarray:
    """glint_np.py:53-56: element 2e low nibble, 2e+1 high nibble; pad 0."""
    if idx.size & 1:
        idx = np.concatenate([idx, np.zeros(1, dtype=np.uint8)])
    return ((idx[0::2] & 15) | ((idx[1::2] & 15) << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, n: int) -> np.ndarray:
    """glint_np.py:57-62."""
    b = np.frombuffer(packed, dtype=np.uint8) if isinstance(packed, (bytes, bytearray)) else np.asarray(packed, np.uint8)
    out = np.empty(b.size * 2, dtype=np.uint8)
    out[0::2] = b & 15
    out[1::2] = b >> 4
    return out[:n]


def encode_f32(w: np.ndarray, bs: int = 64, chunk: int = 1 << 22) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """glint_np.py:63-83: returns (hole u8[ceil(n/2)], plug u8[ceil(n/2)], absmax f32[ceil(n/bs)])."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = w.size
    absmax = block_absmax(w, bs)
    hole = np.empty((n + 1) // 2, dtype=np.uint8)
    plug = np.empty((n + 1) // 2, dtype=np.uint8)
    step = max(bs, (chunk // bs) * bs)
    if step & 1:
        step *= 2
    with np.errstate(divide="ignore", invalid="ignore"):
        for i0 in range(0, n, step):
            i1 = min(n, i0 + step)
            s = np.repeat(absmax[i0 // bs:(i1 + bs - 1) // bs], bs)[: i1 - i0]
            v = np.where(s == 0, np.float32(0), w[i0:i1] / s).astype(np.float32, copy=False)
            h = nearest(v, PARENT_F32, 0)
            p = nearest(v, CELLS_FLAT, h.astype(np.int64) * 16)
            hole[i0 // 2:(i1 + 1) // 2] = pack_nibbles(h)
            plug[i0 // 2:(i1 + 1) // 2] = pack_nibbles(p)
    return hole, plug, absmax


def encode_bf16(u16: np.ndarray, bs: int = 64):
    return encode_f32(bf16_bits_to_f32(np.asarray(u16).reshape(-1)), bs)


def expand(hole, plug, absmax, n: int, bs: int = 64) -> np.ndarray:
    """glint_np.py:84-92: f32 CELLS[h][p] * absmax[i // bs]."""
    h = unpack_nibbles(hole, n)
    p = unpack_nibbles(plug, n)
    s = np.repeat(np.asarray(absmax, dtype=np.float32), bs)[:n]
    return CELLS_F32[h, p] * s


def expand_bf16(hole, plug, absmax, n: int, bs: int = 64) -> np.ndarray:
    """glint_unpin.py:25-32: BF16 bits of the f32 expand."""
    return f32_to_bf16_bits(expand(hole, plug, absmax, n, bs))


def htile_ref_f64(hole, plug, absmax, x_u16: np.ndarray, M: int, N: int, K: int, bs: int) -> np.ndarray:
    """y[m, n] = sum_k CELLS[h][p] * absmax[(nK+k)/bs] * x[m, k] in float64 (the
    reference device test's oracle, test_htile_k_bounds_device.cu:90-98)."""
    w = expand(hole, plug, absmax, N * K, bs).astype(np.float64).reshape(N, K)
    x = bf16_bits_to_f32(np.asarray(x_u16).reshape(-1)).astype(np.float64).reshape(M, K)
    return x @ w.T


# ----------------------------------------------------------------- f64 codec restatement
def codec_encode_f64(weights: Sequence[float], bs: int = 64) -> Tuple[List[int], List[int], List[float]]:
    """glint_codec.py:119-149: Python-float absmax, divide and linear scans."""
    par = [float(x) for x in PARENT_F32]
    cel = [[float(x) for x in row] for row in CELLS_F32]
    n = len(weights)
    nb = (n + bs - 1) // bs
    absmax = [0.0] * nb
    for i, w in enumerate(weights):
        a = abs(float(w))
        if a > absmax[i // bs]:
            absmax[i // bs] = a
    hole, plug = [0] * n, [0] * n
    for i, w in enumerate(weights):
        s = absmax[i // bs] or 1.0
        v = float(w) / s
        best, bd = 0, abs(v - par[0])
        for k in range(1, 16):
            d = abs(v - par[k])
            if d < bd:
                best, bd = k, d
        hole[i] = best
        row = cel[best]
        bj, bd = 0, abs(v - row[0])
        for j in range(1, 16):
            d = abs(v - row[j])
            if d < bd:
                bj, bd = j, d
        plug[i] = bj
    return hole, plug, absmax


def pack_indices(idx: Sequence[int]) -> bytes:
    """glint_codec.py:36-43."""
    n = len(idx)
    out = bytearray((n + 1) // 2)
    for i in range(0, n, 2):
        out[i // 2] = (idx[i] & 15) | (((idx[i + 1] & 15) if i + 1 < n else 0) << 4)
    return bytes(out)


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


# ------------------------------------------------------------------ C oracle (ctypes)
def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


class Oracle:
    """ctypes over oracle/liboracle.so (linear-scan C restatement, OpenMP)."""

    def __init__(self, path: str | os.PathLike | None = None):
        p = Path(path) if path else HERE / "liboracle.so"
        if not p.is_file():
            raise RuntimeError(f"{p} missing: run `make -C oracle`")
        self.lib = ctypes.CDLL(str(p))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        sig = {
            "oracle_encode_f32": ([vp, i64, i32, vp, vp, vp], i32),
            "oracle_encode_bf16": ([vp, i64, i32, vp, vp, vp, vp], i32),
            "oracle_expand_f32": ([vp, vp, vp, i64, i32, vp], None),
            "oracle_expand_bf16": ([vp, vp, vp, i64, i32, vp], None),
            "oracle_f32_to_bf16": ([vp, i64, vp], None),
            "oracle_htile_f32": ([vp, vp, vp, vp, vp, i32, i32, i32, i32], None),
            "oracle_htile_f64": ([vp, vp, vp, vp, vp, vp, i32, i32, i32, i32], None),
            "oracle_quant_act": ([vp, i32, i32, vp, vp], None),
            "oracle_int8_mma_emu": ([vp, vp, vp, vp, i32, i32, i32, vp], None),
            "oracle_int8_mma_emu_sep": ([vp, vp, vp, vp, i32, i32, i32, vp], None),
            "oracle_fmaf_n": ([vp, vp, vp, i64, vp], None),
            "oracle_int8_gemm_i32": ([vp, vp, i32, i32, i32, i32, i32, vp], None),
            "oracle_int8_scale_bf16": ([vp, vp, vp, i32, i32, vp], None),
            "oracle_unpack_res4": ([vp, i64, vp], None),
            "oracle_int8_mma_plug_fused": ([vp, vp, vp, vp, vp, vp, i32, i32, i32, vp], None),
            "oracle_quant_act_resid": ([vp, vp, vp, i32, i32, vp, vp], None),
            "oracle_int8_pin_dequant_bf16": ([vp, vp, i64, vp], None),
            "oracle_int8_tile_f64": ([vp, vp, vp, i32, i32, i32, vp, vp], None),
            "oracle_kmajor_pack": ([vp, vp, vp, i32, i32, vp, vp, vp], None),
            "oracle_gemv_km_fold": ([vp, vp, vp, i32, i32, i32, vp], None),
            "oracle_select_topk": ([vp, i32, i32, vp], i32),
            "oracle_select_ex": ([vp, i32, i32, i32, i32, vp], i32),
            "oracle_select_threshold": ([vp, i32, i32, i32, i32], i32),
            "oracle_select_price_key": ([vp, i32, i32], i32),
            "oracle_apply_corr_km": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, vp], None),
            "oracle_threads": ([], i32),
        }
        for name, (args, res) in sig.items():
            f = getattr(self.lib, name)
            f.argtypes = args
            f.restype = res

    def threads(self) -> int:
        return int(self.lib.oracle_threads())

    def encode_bf16(self, u16: np.ndarray, bs: int = 64):
        u16 = np.ascontiguousarray(u16, dtype=np.uint16).reshape(-1)
        n = u16.size
        hole = np.zeros((n + 1) // 2, np.uint8)
        plug = np.zeros((n + 1) // 2, np.uint8)
        am = np.zeros((n + bs - 1) // bs if bs > 0 else 0, np.float32)
        scratch = np.empty(n, np.float32)
        rc = self.lib.oracle_encode_bf16(_ptr(u16), n, bs, _ptr(hole), _ptr(plug), _ptr(am), _ptr(scratch))
        if rc:
            raise ValueError(f"oracle_encode_bf16 rc={rc}")
        return hole, plug, am

    def encode_f32(self, w: np.ndarray, bs: int = 64):
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        n = w.size
        hole = np.zeros((n + 1) // 2, np.uint8)
        plug = np.zeros((n + 1) // 2, np.uint8)
        am = np.zeros((n + bs - 1) // bs if bs > 0 else 0, np.float32)
        rc = self.lib.oracle_encode_f32(_ptr(w), n, bs, _ptr(hole), _ptr(plug), _ptr(am))
        if rc:
            raise ValueError(f"oracle_encode_f32 rc={rc}")
        return hole, plug, am

    def expand_f32(self, hole, plug, am, n: int, bs: int = 64) -> np.ndarray:
        out = np.empty(n, np.float32)
        hole, plug, am = (np.ascontiguousarray(a) for a in (hole, plug, am))
        self.lib.oracle_expand_f32(_ptr(hole), _ptr(plug), _ptr(am), n, bs, _ptr(out))
        return out

    def expand_bf16(self, hole, plug, am, n: int, bs: int = 64) -> np.ndarray:
        out = np.empty(n, np.uint16)
        hole, plug, am = (np.ascontiguousarray(a) for a in (hole, plug, am))
        self.lib.oracle_expand_bf16(_ptr(hole), _ptr(plug), _ptr(am), n, bs, _ptr(out))
        return out

    def htile_f32(self, hole, plug, am, x_u16, M, N, K, bs) -> np.ndarray:
        y = np.empty(M * N, np.float32)
        hole, plug, am, x_u16 = (np.ascontiguousarray(a) for a in (hole, plug, am, x_u16))
        self.lib.oracle_htile_f32(_ptr(hole), _ptr(plug), _ptr(am), _ptr(x_u16), _ptr(y), M, N, K, bs)
        return y.reshape(M, N)

    def htile_f64(self, hole, plug, am, x_u16, M, N, K, bs):
        y = np.empty(M * N, np.float64)
        a = np.empty(M * N, np.float64)
        hole, plug, am, x_u16 = (np.ascontiguousarray(t) for t in (hole, plug, am, x_u16))
        self.lib.oracle_htile_f64(_ptr(hole), _ptr(plug), _ptr(am), _ptr(x_u16), _ptr(y), _ptr(a), M, N, K, bs)
        return y.reshape(M, N), a.reshape(M, N)

    def quant_act(self, x_u16: np.ndarray, m: int, k: int):
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        xq = np.empty(m * k, np.int8)
        sx = np.empty(m * (k // 64), np.float32)
        self.lib.oracle_quant_act(_ptr(x_u16), m, k, _ptr(xq), _ptr(sx))
        return xq, sx

    def int8_mma_emu(self, xq, sx, wq, sw, m, n, k) -> np.ndarray:
        """The reference kernel's W8A8 arithmetic as its nvcc build compiles it (fused
        multiply-add for the last step)."""
        y = np.empty(m * n, np.float32)
        xq, sx, wq, sw = (np.ascontiguousarray(t) for t in (xq, sx, wq, sw))
        self.lib.oracle_int8_mma_emu(_ptr(xq), _ptr(sx), _ptr(wq), _ptr(sw), m, n, k, _ptr(y))
        return y.reshape(m, n)

    def int8_mma_emu_sep(self, xq, sx, wq, sw, m, n, k) -> np.ndarray:
        """The reference test's host emulation: the last multiply and add separate."""
        y = np.empty(m * n, np.float32)
        xq, sx, wq, sw = (np.ascontiguousarray(t) for t in (xq, sx, wq, sw))
        self.lib.oracle_int8_mma_emu_sep(_ptr(xq), _ptr(sx), _ptr(wq), _ptr(sw), m, n, k, _ptr(y))
        return y.reshape(m, n)

    def fmaf(self, a, b, c) -> np.ndarray:
        a, b, c = (np.ascontiguousarray(t, np.float32) for t in (a, b, c))
        out = np.empty(a.size, np.float32)
        self.lib.oracle_fmaf_n(_ptr(a), _ptr(b), _ptr(c), a.size, _ptr(out))
        return out

    def unpack_res4(self, q4, n: int) -> np.ndarray:
        q4 = np.ascontiguousarray(q4, np.uint8)
        out = np.empty(n, np.int8)
        self.lib.oracle_unpack_res4(_ptr(q4), n, _ptr(out))
        return out

    def int8_mma_plug_fused(self, xq, sx, wq, sw, pq, sp, m, n, k) -> np.ndarray:
        arrs = [np.ascontiguousarray(a, t) for a, t in ((xq, np.int8), (sx, np.float32), (wq, np.int8),
                                                          (sw, np.float32), (pq, np.int8), (sp, np.float32))]
        y = np.empty(m * n, np.float32)
        self.lib.oracle_int8_mma_plug_fused(*[_ptr(a) for a in arrs], m, n, k, _ptr(y))
        return y.reshape(m, n)

    def quant_act_resid(self, x_u16, xq, sx, m: int, k: int):
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        xq = np.ascontiguousarray(xq, np.int8)
        sx = np.ascontiguousarray(sx, np.float32)
        rq = np.empty(m * k, np.int8)
        sr = np.empty(m * (k // 64), np.float32)
        self.lib.oracle_quant_act_resid(_ptr(x_u16), _ptr(xq), _ptr(sx), m, k, _ptr(rq), _ptr(sr))
        return rq, sr

    def int8_gemm_i32(self, A, B, M, N, K, row0=0, row1=None) -> np.ndarray:
        row1 = M if row1 is None else row1
        C = np.zeros(M * N, np.int32)
        A, B = np.ascontiguousarray(A, np.int8), np.ascontiguousarray(B, np.int8)
        self.lib.oracle_int8_gemm_i32(_ptr(A), _ptr(B), M, N, K, row0, row1, _ptr(C))
        return C.reshape(M, N)

    def int8_scale_bf16(self, C, sa, sb, M, N) -> np.ndarray:
        out = np.empty(M * N, np.uint16)
        C, sa, sb = (np.ascontiguousarray(t) for t in (C, sa, sb))
        self.lib.oracle_int8_scale_bf16(_ptr(C), _ptr(sa), _ptr(sb), M, N, _ptr(out))
        return out.reshape(M, N)

    def int8_pin_dequant_bf16(self, q, scale) -> np.ndarray:
        q = np.ascontiguousarray(q, np.int8).reshape(-1)
        scale = np.ascontiguousarray(scale, np.float32)
        assert scale.size >= (q.size + 63) // 64
        out = np.empty(q.size, np.uint16)
        self.lib.oracle_int8_pin_dequant_bf16(_ptr(q), _ptr(scale), q.size, _ptr(out))
        return out

    def int8_tile_f64(self, x_u16, q, scale, M, N, K):
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        q = np.ascontiguousarray(q, np.int8)
        scale = np.ascontiguousarray(scale, np.float32)
        assert x_u16.size >= M * K and q.size >= N * K and scale.size >= (N * K + 63) // 64
        y = np.empty(M * N, np.float64)
        a = np.empty(M * N, np.float64)
        self.lib.oracle_int8_tile_f64(_ptr(x_u16), _ptr(q), _ptr(scale), M, N, K, _ptr(y), _ptr(a))
        return y.reshape(M, N), a.reshape(M, N)

    def kmajor_pack(self, hole, plug, am, N: int, K: int):
        hole, plug = np.ascontiguousarray(hole, np.uint8), np.ascontiguousarray(plug, np.uint8)
        am = np.ascontiguousarray(am, np.float32)
        assert N % 2 == 0 and K % 64 == 0 and hole.size >= N * K // 2 and am.size >= N * K // 64
        hk = np.empty(K * N // 2, np.uint8)
        pk = np.empty(K * N // 2, np.uint8)
        sk = np.empty(N * K // 64, np.float32)
        self.lib.oracle_kmajor_pack(_ptr(hole), _ptr(plug), _ptr(am), N, K, _ptr(hk), _ptr(pk), _ptr(sk))
        return hk, pk, sk

    def gemv_km_fold(self, hole_k, scales_k, x_u16, N: int, K: int, ksg: int = 1) -> np.ndarray:
        hole_k = np.ascontiguousarray(hole_k, np.uint8)
        scales_k = np.ascontiguousarray(scales_k, np.float32)
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        assert K % (64 * ksg) == 0 and hole_k.size >= K * N // 2 and x_u16.size >= K
        y = np.empty(N, np.float32)
        self.lib.oracle_gemv_km_fold(_ptr(hole_k), _ptr(scales_k), _ptr(x_u16), N, K, ksg, _ptr(y))
        return y

    def select_topk(self, x_u16, K: int, nsel: int) -> np.ndarray:
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        idx = np.empty(max(K, 1), np.int32)
        n = self.lib.oracle_select_topk(_ptr(x_u16), K, nsel, _ptr(idx))
        return idx[:n].copy()

    def select_ex(self, x_u16, K: int, nsel: int, tkey: int = 0, nfloor: int = 0) -> np.ndarray:
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        idx = np.empty(max(K, 1), np.int32)
        n = self.lib.oracle_select_ex(_ptr(x_u16), K, nsel, tkey, nfloor, _ptr(idx))
        return idx[:n].copy()

    def select_threshold(self, x_u16, K: int, nsel: int, tkey: int = 0, nfloor: int = 0) -> int:
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        return int(self.lib.oracle_select_threshold(_ptr(x_u16), K, nsel, tkey, nfloor))

    def select_price_key(self, x_u16, K: int, tkey: int) -> int:
        x_u16 = np.ascontiguousarray(x_u16, np.uint16)
        return int(self.lib.oracle_select_price_key(_ptr(x_u16), K, tkey))

    def apply_corr_km(self, hole_k, plug_k, scales_k, x_u16, idx, N: int, K: int, y, ks: int = 1) -> np.ndarray:
        arrs = [np.ascontiguousarray(a, t) for a, t in ((hole_k, np.uint8), (plug_k, np.uint8),
                                                          (scales_k, np.float32), (x_u16, np.uint16))]
        idx = np.ascontiguousarray(idx, np.int32)
        out = np.array(y, dtype=np.float32, copy=True)
        self.lib.oracle_apply_corr_km(*[_ptr(a) for a in arrs], _ptr(idx), idx.size, N, K, ks, _ptr(out))
        return out
