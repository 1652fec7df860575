"""ctypes bindings to the GLINT C ABI (libglint_encode.so, libp7_kernels.so).

Two layers:

* ``EncodeLib`` / ``P7Lib``: the raw C entry points with their argtypes, as a caller of
  the reference's ``glint_cuda.py`` would bind them (the host-pointer ABI takes bytes);
* tensor helpers (``encode_bf16`` ... ``int8_gemm_i32``) that pass torch device tensors
  and torch's current stream straight to the device entry points. torch is only the
  allocator and stream here; every result is computed by the HIP kernels.

A missing library raises RuntimeError: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Tuple

PKG = Path(__file__).resolve().parent
LIB_DIR = PKG / "lib"

_c = ctypes
VP, I64, I32 = _c.c_void_p, _c.c_int64, _c.c_int


def encode_lib_path() -> Optional[Path]:
    """$GLINT_ENCODE_SO, else glint_amd/lib/libglint_encode.so (reference glint_cuda.py:9-18)."""
    env = os.environ.get("GLINT_ENCODE_SO")
    if env:
        p = Path(env)
        return p if p.is_file() else None
    p = LIB_DIR / "libglint_encode.so"
    return p if p.is_file() else None


def p7_lib_path() -> Optional[Path]:
    env = os.environ.get("GLINT_P7_SO")
    if env:
        p = Path(env)
        return p if p.is_file() else None
    p = LIB_DIR / "libp7_kernels.so"
    return p if p.is_file() else None


_ENCODE_SIGS = {
    "glint_encode_n_absmax": ([I64, I32], I32),
    "glint_encode_n_packed": ([I64], I32),
    "glint_encode_bf16_host": ([VP, I64, I32, VP, VP, VP], I32),
    "glint_encode_f32_host": ([VP, I64, I32, VP, VP, VP], I32),
    "glint_expand_packed_to_f32_host": ([VP, VP, VP, I64, I32, VP], I32),
    "glint_expand_packed_to_bf16_host": ([VP, VP, VP, I64, I32, VP], I32),
    "glint_expand_packed_to_f32_device": ([VP, VP, VP, I64, I32, VP, VP], I32),
    "glint_expand_packed_to_bf16_device": ([VP, VP, VP, I64, I32, VP, VP], I32),
    "glint_encode_bf16_device": ([VP, I64, I32, VP, VP, VP, VP], I32),
    "glint_encode_f32_device": ([VP, I64, I32, VP, VP, VP, VP], I32),
    "launch_glint_htile_s3_f32_stream": ([VP, VP, VP, VP, VP, I32, I32, I32, I32, VP], I32),
    "launch_glint_htile_s3_f32": ([VP, VP, VP, VP, VP, I32, I32, I32, I32], I32),
    "launch_glint_htile_bf16_stream": ([VP, VP, VP, VP, VP, I32, I32, I32, I32, VP], I32),
    "glint_htile_workspace_reserve": ([VP], I32),
    "glint_htile_workspace_release": ([VP], I32),
    "launch_glint_htile_bf16_stream_noalloc": ([VP, VP, VP, VP, VP, I32, I32, I32, I32, VP], I32),
    "glint_kmajor_pack": ([VP, VP, VP, I32, I32, VP, VP, VP, VP], I32),
    "glint_gemv_km_fold": ([VP, VP, VP, VP, I32, I32, I32, VP, VP], I32),
    "glint_select_topk": ([VP, I32, I32, VP, VP, VP], I32),
    "glint_select_topk_ex": ([VP, I32, I32, I32, I32, VP, VP, VP, I32, VP], I32),
    "glint_apply_corr_km": ([VP, VP, VP, VP, VP, VP, VP, I32, I32, I32, VP, VP], I32),
}


class Int8MmaLinear(_c.Structure):
    """include/int8_mma_gemm.h Int8MmaLinear, passed by value."""
    _fields_ = [("q", VP), ("scale", VP), ("n_out", I32), ("k_in", I32)]


class Int8PinLinear(_c.Structure):
    """include/int8_tile_gemm.h Int8PinLinear, passed by value (same layout as Int8MmaLinear)."""
    _fields_ = [("q", VP), ("scale", VP), ("n_out", I32), ("k_in", I32)]


class GlintStreamerStats(ctypes.Structure):
    """include/glint_plug_streamer.h GlintStreamerStats."""
    _fields_ = [("total_h2d_bytes", ctypes.c_uint64), ("total_stall_ms", ctypes.c_double),
                ("per_layer_stall_ms", ctypes.c_double * 64), ("n_layers", ctypes.c_int)]


_P7_SIGS = {
    "p7_abi_version": ([], _c.c_char_p),
    "p7_abi_selftest": ([_c.c_char_p, _c.c_size_t], I32),
    "int8_mma_gemm": ([VP, Int8MmaLinear, VP, I32, VP, VP, VP], I32),
    "int8_mma_gemm_plug": ([VP, Int8MmaLinear, VP, VP, VP, I32, VP, VP, VP, VP], I32),
    "int8_mma_gemm_plug_fused": ([VP, Int8MmaLinear, VP, VP, VP, I32, VP, VP, VP], I32),
    "int8_mma_gemm_resolve": ([VP, Int8MmaLinear, VP, VP, VP, I32, VP, VP, VP, VP, VP, VP], I32),
    "p7_int8_gemm_flat": ([VP, VP, VP, I32, I32, VP, I32, VP, VP, VP], I32),
    "p7_int8_gemm_plug_flat": ([VP, VP, VP, VP, VP, I32, I32, VP, I32, VP, VP, VP], I32),
    "int8_tile_gemm_bf16": ([VP, Int8PinLinear, VP, I32, VP], I32),
    "int8_tile_gemm_workspace_release": ([VP], I32),
    "glint_int8_gemm_i32": ([VP, VP, VP, I32, I32, I32, VP], I32),
    "glint_int8_gemm_scaled_bf16": ([VP, VP, VP, VP, VP, I32, I32, I32, VP], I32),
    "glint_plug_streamer_create": ([_c.POINTER(VP), I32, _c.POINTER(_c.c_uint64), VP, VP], I32),
    "glint_plug_streamer_destroy": ([VP], None),
    "glint_plug_streamer_set_host_data": ([VP, I32, VP, _c.c_uint64], I32),
    "glint_plug_streamer_start": ([VP], I32),
    "glint_plug_streamer_acquire": ([VP, I32, _c.POINTER(VP)], I32),
    "glint_plug_streamer_release": ([VP, I32], I32),
    "glint_plug_streamer_get_stats": ([VP, _c.POINTER(GlintStreamerStats)], I32),
    "glint_plug_streamer_reset_stats": ([VP], None),
}

ENCODE_SYMBOLS = tuple(_ENCODE_SIGS)
P7_SYMBOLS = tuple(_P7_SIGS)


def _bind(path: Path, sigs: dict) -> ctypes.CDLL:
    # One HIP runtime per process: torch's wheel ships its own libamdhip64.so.7. If torch
    # is importable, load it first so our library binds to that already-loaded runtime
    # (same SONAME) instead of pulling in a second copy from /opt/rocm.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(path))
    for name, (args, res) in sigs.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    return lib


_ENC: Optional[ctypes.CDLL] = None
_P7: Optional[ctypes.CDLL] = None


def encode_lib() -> ctypes.CDLL:
    global _ENC
    if _ENC is None:
        p = encode_lib_path()
        if p is None:
            raise RuntimeError("libglint_encode.so not built: run `python -m glint_amd.build`")
        _ENC = _bind(p, _ENCODE_SIGS)
    return _ENC


_PROBE: Optional[ctypes.CDLL] = None


def probe_lib() -> ctypes.CDLL:
    """glint_amd/lib/libglint_probe.so: bench.py's HBM read ceiling (not part of the ABI)."""
    global _PROBE
    if _PROBE is None:
        p = LIB_DIR / "libglint_probe.so"
        if not p.is_file():
            raise RuntimeError("libglint_probe.so not built: run `python -m glint_amd.build`")
        _PROBE = _bind(p, {"glint_probe_read": ([VP, I64, VP, I32, VP], I32)})
    return _PROBE


def p7_lib() -> ctypes.CDLL:
    global _P7
    if _P7 is None:
        p = p7_lib_path()
        if p is None:
            raise RuntimeError("libp7_kernels.so not built: run `python -m glint_amd.build`")
        _P7 = _bind(p, _P7_SIGS)
    return _P7


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} rc={rc}")


# ------------------------------------------------------------ tensor helpers (device)
def _torch():
    import torch
    return torch


def _stream(stream=None) -> ctypes.c_void_p:
    torch = _torch()
    s = torch.cuda.current_stream() if stream is None else stream
    return VP(s.cuda_stream)


def _p(t) -> ctypes.c_void_p:
    return VP(t.data_ptr())


def _as_u16(t):
    torch = _torch()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16)
    if t.dtype in (torch.int16, torch.uint16):
        return t
    raise TypeError(f"expected bf16 bits, got {t.dtype}")


def encode_bf16(w, blocksize: int = 64, out=None, stream=None):
    """GPU encode of a BF16 device tensor -> (hole u8, plug u8, absmax f32) device tensors."""
    torch = _torch()
    w = _as_u16(w).contiguous()
    n = w.numel()
    if out is None:
        npk, nam = (n + 1) // 2, (n + blocksize - 1) // blocksize
        out = (torch.empty(npk, dtype=torch.uint8, device=w.device), torch.empty(npk, dtype=torch.uint8, device=w.device),
               torch.empty(nam, dtype=torch.float32, device=w.device))
    hole, plug, am = out
    _check(encode_lib().glint_encode_bf16_device(_p(w), n, blocksize, _p(hole), _p(plug), _p(am), _stream(stream)),
           "glint_encode_bf16_device")
    return hole, plug, am


def encode_f32(w, blocksize: int = 64, stream=None):
    torch = _torch()
    w = w.contiguous()
    assert w.dtype == torch.float32
    n = w.numel()
    npk, nam = (n + 1) // 2, (n + blocksize - 1) // blocksize
    hole = torch.empty(npk, dtype=torch.uint8, device=w.device)
    plug = torch.empty(npk, dtype=torch.uint8, device=w.device)
    am = torch.empty(nam, dtype=torch.float32, device=w.device)
    _check(encode_lib().glint_encode_f32_device(_p(w), n, blocksize, _p(hole), _p(plug), _p(am), _stream(stream)),
           "glint_encode_f32_device")
    return hole, plug, am


def expand_f32(hole, plug, absmax, n: int, blocksize: int = 64, out=None, stream=None):
    torch = _torch()
    out = torch.empty(n, dtype=torch.float32, device=hole.device) if out is None else out
    _check(encode_lib().glint_expand_packed_to_f32_device(_p(hole), _p(plug), _p(absmax), n, blocksize, _p(out),
                                                          _stream(stream)), "glint_expand_packed_to_f32_device")
    return out


def expand_bf16(hole, plug, absmax, n: int, blocksize: int = 64, out=None, stream=None):
    torch = _torch()
    out = torch.empty(n, dtype=torch.bfloat16, device=hole.device) if out is None else out
    _check(encode_lib().glint_expand_packed_to_bf16_device(_p(hole), _p(plug), _p(absmax), n, blocksize, _p(out),
                                                           _stream(stream)), "glint_expand_packed_to_bf16_device")
    return out


def htile_f32(hole, plug, absmax, x, N: int, K: int, blocksize: int = 64, out=None, stream=None):
    """y[M, N] f32 = x[M, K] (bf16) @ W^T via launch_glint_htile_s3_f32_stream."""
    torch = _torch()
    x = _as_u16(x)
    M = x.numel() // K
    y = torch.empty((M, N), dtype=torch.float32, device=x.device) if out is None else out
    _check(encode_lib().launch_glint_htile_s3_f32_stream(_p(hole), _p(plug), _p(absmax), _p(x), _p(y), M, N, K,
                                                         blocksize, _stream(stream)), "launch_glint_htile_s3_f32_stream")
    return y


def htile_bf16(hole, plug, absmax, x, N: int, K: int, blocksize: int = 64, out=None, stream=None):
    """y[M, N] bf16 (f32 accumulation) via launch_glint_htile_bf16_stream."""
    torch = _torch()
    x = _as_u16(x)
    M = x.numel() // K
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if out is None else out
    _check(encode_lib().launch_glint_htile_bf16_stream(_p(hole), _p(plug), _p(absmax), _p(x), _p(y), M, N, K,
                                                       blocksize, _stream(stream)), "launch_glint_htile_bf16_stream")
    return y


# ------------------------------------------------------- K-major decode path (glint_select.h)
def kmajor_pack(hole, plug, absmax, N: int, K: int, stream=None):
    """Row-major pin planes -> (hole_k, plug_k, scales_k) device tensors."""
    torch = _torch()
    hk = torch.empty(K * N // 2, dtype=torch.uint8, device=hole.device)
    pk = torch.empty(K * N // 2, dtype=torch.uint8, device=hole.device)
    sk = torch.empty(N * K // 64, dtype=torch.float32, device=hole.device)
    _check(encode_lib().glint_kmajor_pack(_p(hole), _p(plug), _p(absmax), N, K, _p(hk), _p(pk), _p(sk),
                                          _stream(stream)), "glint_kmajor_pack")
    return hk, pk, sk


def gemv_km_fold(hole_k, scales_k, x, N: int, K: int, ksg: int = 1, y=None, part=None, stream=None):
    """Parent-only GEMV over the K-major hole: x bf16 [K] -> y f32 [N]."""
    torch = _torch()
    y = torch.empty(N, dtype=torch.float32, device=hole_k.device) if y is None else y
    if ksg > 1 and part is None:
        part = torch.empty(ksg * N, dtype=torch.float32, device=hole_k.device)
    _check(encode_lib().glint_gemv_km_fold(_p(hole_k), _p(scales_k), _p(_as_u16(x)), _p(y), N, K, ksg,
                                           _p(part) if part is not None else None, _stream(stream)),
           "glint_gemv_km_fold")
    return y


def select_topk(x, nsel: int, idx=None, cnt=None, stream=None, tkey: int = 0, nfloor: int = 0, cnt_log=None,
                slot: int = 0):
    """Kept channels of x (ascending) and their count, both on the device (the rank rule,
    and the price / relational / floor rules when tkey or nfloor is given)."""
    torch = _torch()
    x = _as_u16(x)
    K = x.numel()
    idx = torch.empty(K, dtype=torch.int32, device=x.device) if idx is None else idx
    cnt = torch.empty(1, dtype=torch.int32, device=x.device) if cnt is None else cnt
    if tkey == 0 and nfloor == 0 and cnt_log is None:
        _check(encode_lib().glint_select_topk(_p(x), K, nsel, _p(idx), _p(cnt), _stream(stream)), "glint_select_topk")
    else:
        _check(encode_lib().glint_select_topk_ex(_p(x), K, nsel, tkey, nfloor, _p(idx), _p(cnt),
                                                 _p(cnt_log) if cnt_log is not None else None, slot,
                                                 _stream(stream)), "glint_select_topk_ex")
    return idx, cnt


def apply_corr_km(hole_k, plug_k, scales_k, x, idx, cnt, y, N: int, K: int, ks: int = 1, part=None, stream=None):
    """y += the plug correction over the selected channels (in place)."""
    torch = _torch()
    if ks > 1 and part is None:
        part = torch.empty(ks * N, dtype=torch.float32, device=y.device)
    _check(encode_lib().glint_apply_corr_km(_p(hole_k), _p(plug_k), _p(scales_k), _p(_as_u16(x)), _p(idx), _p(cnt),
                                            _p(y), N, K, ks, _p(part) if part is not None else None,
                                            _stream(stream)), "glint_apply_corr_km")
    return y


def int8_mma_gemm(x, q, scale, n_out: int, k_in: int, xq=None, sx=None, stream=None):
    """The attach ABI's W8A8 GEMM: x bf16 [m, k_in] -> y f32 [m, n_out] (also returns xq, sx)."""
    torch = _torch()
    x = _as_u16(x)
    m = x.numel() // k_in
    y = torch.empty((m, n_out), dtype=torch.float32, device=x.device)
    xq = torch.empty(m * k_in, dtype=torch.int8, device=x.device) if xq is None else xq
    sx = torch.empty(m * (k_in // 64), dtype=torch.float32, device=x.device) if sx is None else sx
    lin = Int8MmaLinear(q.data_ptr(), scale.data_ptr(), n_out, k_in)
    _check(p7_lib().int8_mma_gemm(_p(x), lin, _p(y), m, _p(xq), _p(sx), _stream(stream)), "int8_mma_gemm")
    return y, xq, sx


def int8_tile_gemm(x, q, scale, n_out: int, k_in: int, m: Optional[int] = None, y=None, stream=None):
    """W8A16 over an INT8 pin linear: x bf16 [m, k_in] -> y f32 [m, n_out] (int8_tile_gemm_bf16).
    x, q and scale may be views at any offset; the call takes their data pointers as they are."""
    torch = _torch()
    x = _as_u16(x)
    m = x.numel() // k_in if m is None else m
    if y is None:
        y = torch.empty((m, n_out), dtype=torch.float32, device=x.device)
    lin = Int8PinLinear(q.data_ptr(), scale.data_ptr(), n_out, k_in)
    _check(p7_lib().int8_tile_gemm_bf16(_p(x), lin, _p(y), m, _stream(stream)), "int8_tile_gemm_bf16")
    return y


def int8_mma_gemm_plug(x, q, scale, plug_q4, plug_scale, n_out: int, k_in: int, fused: bool = False, stream=None):
    """The late-plug forms: two passes through int8 scratch (int8_mma_gemm_plug) or one fused
    kernel (int8_mma_gemm_plug_fused). Returns y f32 [m, n_out]."""
    torch = _torch()
    x = _as_u16(x)
    m = x.numel() // k_in
    y = torch.empty((m, n_out), dtype=torch.float32, device=x.device)
    xq = torch.empty(m * k_in, dtype=torch.int8, device=x.device)
    sx = torch.empty(m * (k_in // 64), dtype=torch.float32, device=x.device)
    lin = Int8MmaLinear(q.data_ptr(), scale.data_ptr(), n_out, k_in)
    lib = p7_lib()
    if fused:
        _check(lib.int8_mma_gemm_plug_fused(_p(x), lin, _p(plug_q4), _p(plug_scale), _p(y), m, _p(xq), _p(sx),
                                            _stream(stream)), "int8_mma_gemm_plug_fused")
    else:
        pi8 = torch.empty(n_out * k_in, dtype=torch.int8, device=x.device)
        _check(lib.int8_mma_gemm_plug(_p(x), lin, _p(plug_q4), _p(plug_scale), _p(y), m, _p(xq), _p(sx), _p(pi8),
                                      _stream(stream)), "int8_mma_gemm_plug")
    return y


def int8_mma_gemm_resolve(x, q, scale, n_out: int, k_in: int, plug_q4=None, plug_scale=None, stream=None):
    """int8_mma_gemm_resolve: base (+ plug) plus the re-quantized activation residual.
    Returns (y, xq, sx, rq, sr)."""
    torch = _torch()
    x = _as_u16(x)
    m = x.numel() // k_in
    dev = x.device
    y = torch.empty((m, n_out), dtype=torch.float32, device=dev)
    xq = torch.empty(m * k_in, dtype=torch.int8, device=dev)
    sx = torch.empty(m * (k_in // 64), dtype=torch.float32, device=dev)
    rq = torch.empty_like(xq)
    sr = torch.empty_like(sx)
    pi8 = torch.empty(n_out * k_in, dtype=torch.int8, device=dev) if plug_q4 is not None else None
    lin = Int8MmaLinear(q.data_ptr(), scale.data_ptr(), n_out, k_in)
    opt = lambda t: VP(t.data_ptr()) if t is not None else VP(None)
    _check(p7_lib().int8_mma_gemm_resolve(_p(x), lin, opt(plug_q4), opt(plug_scale), _p(y), m, _p(xq), _p(sx),
                                          _p(rq), _p(sr), opt(pi8), _stream(stream)), "int8_mma_gemm_resolve")
    return y, xq, sx, rq, sr


class PlugStreamer:
    """The 2-slot plug ring (include/glint_plug_streamer.h) over raw device pointers.
    Methods return the C return codes unchanged."""

    def __init__(self, layer_bytes, copy_stream, compute_stream):
        self.lib = p7_lib()
        self.h = VP()
        n = len(layer_bytes)
        arr = (ctypes.c_uint64 * n)(*layer_bytes)
        rc = self.lib.glint_plug_streamer_create(ctypes.byref(self.h), n, arr, VP(copy_stream.cuda_stream),
                                                 VP(compute_stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"glint_plug_streamer_create rc={rc}")

    def set_host_data(self, layer: int, data: bytes) -> int:
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        return self.lib.glint_plug_streamer_set_host_data(self.h, layer, buf, len(data))

    def start(self) -> int:
        return self.lib.glint_plug_streamer_start(self.h)

    def acquire(self, layer: int):
        p = VP()
        rc = self.lib.glint_plug_streamer_acquire(self.h, layer, ctypes.byref(p))
        return rc, p.value

    def release(self, layer: int) -> int:
        return self.lib.glint_plug_streamer_release(self.h, layer)

    def stats(self) -> GlintStreamerStats:
        st = GlintStreamerStats()
        _check(self.lib.glint_plug_streamer_get_stats(self.h, ctypes.byref(st)), "glint_plug_streamer_get_stats")
        return st

    def close(self) -> None:
        if self.h:
            self.lib.glint_plug_streamer_destroy(self.h)
            self.h = VP()


def p7_selftest():
    """p7_abi_selftest: (rc, message)."""
    msg = ctypes.create_string_buffer(512)
    rc = p7_lib().p7_abi_selftest(msg, 512)
    return rc, msg.value.decode()


def int8_gemm_i32(A, B, stream=None):
    torch = _torch()
    M, K = A.shape
    N = B.shape[0]
    C = torch.empty((M, N), dtype=torch.int32, device=A.device)
    _check(p7_lib().glint_int8_gemm_i32(_p(A), _p(B), _p(C), M, N, K, _stream(stream)), "glint_int8_gemm_i32")
    return C


def int8_gemm_scaled_bf16(A, B, sa, sb, out=None, stream=None):
    torch = _torch()
    M, K = A.shape
    N = B.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=A.device) if out is None else out
    _check(p7_lib().glint_int8_gemm_scaled_bf16(_p(A), _p(B), _p(sa), _p(sb), _p(out), M, N, K, _stream(stream)),
           "glint_int8_gemm_scaled_bf16")
    return out


# ------------------------------------------------------------- host-pointer wrappers
def encode_bf16_host(raw_bf16: bytes, n: int, blocksize: int = 64) -> Tuple[bytes, bytes, bytes]:
    """Same contract as the reference's glint_cuda.encode_bf16_cuda (glint_cuda.py:52-65)."""
    lib = encode_lib()
    n_am = lib.glint_encode_n_absmax(n, blocksize)
    n_pk = lib.glint_encode_n_packed(n)
    hole = (_c.c_uint8 * n_pk)()
    plug = (_c.c_uint8 * n_pk)()
    am = (_c.c_float * n_am)()
    buf = (_c.c_uint16 * n).from_buffer_copy(raw_bf16[: n * 2])
    rc = lib.glint_encode_bf16_host(_c.byref(buf), n, blocksize, hole, plug, am)
    if rc != 0:
        raise RuntimeError(f"glint_encode_bf16_host rc={rc}")
    return bytes(hole), bytes(plug), bytes(_c.string_at(_c.addressof(am), n_am * 4))


def expand_host(hole: bytes, plug: bytes, absmax_f32: bytes, n: int, blocksize: int = 64) -> bytes:
    """Same contract as the reference's glint_cuda.expand_cuda (glint_cuda.py:66-78)."""
    lib = encode_lib()
    out = (_c.c_float * n)()
    h = _c.create_string_buffer(bytes(hole), len(hole))
    p = _c.create_string_buffer(bytes(plug), len(plug))
    a = _c.create_string_buffer(bytes(absmax_f32), len(absmax_f32))
    rc = lib.glint_expand_packed_to_f32_host(h, p, a, n, blocksize, out)
    if rc != 0:
        raise RuntimeError(f"glint_expand_packed_to_f32_host rc={rc}")
    return bytes(_c.string_at(_c.addressof(out), n * 4))


def expand_bf16_host(hole: bytes, plug: bytes, absmax_f32: bytes, n: int, blocksize: int = 64) -> bytes:
    lib = encode_lib()
    out = (_c.c_uint16 * n)()
    h = _c.create_string_buffer(bytes(hole), len(hole))
    p = _c.create_string_buffer(bytes(plug), len(plug))
    a = _c.create_string_buffer(bytes(absmax_f32), len(absmax_f32))
    rc = lib.glint_expand_packed_to_bf16_host(h, p, a, n, blocksize, out)
    if rc != 0:
        raise RuntimeError(f"glint_expand_packed_to_bf16_host rc={rc}")
    return bytes(_c.string_at(_c.addressof(out), n * 2))
