"""CPU checks of the C-ABI boundary: the libraries load, export every function their
headers declare, and reject bad arguments before touching a GPU (no compute here)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from glint_amd import glint_hip

ROOT = Path(__file__).resolve().parent.parent
HEADERS = {
    "libglint_encode.so": ["glint_encode.h", "glint_htile.h", "glint_select.h"],
    "libp7_kernels.so": ["int8_mma_gemm.h", "int8_tile_gemm.h", "p7_attach.h", "glint_plug_streamer.h"],
}


def declared_functions(header: str):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = []
    for stmt in re.findall(r"^(?!\s*(?:static|#|typedef))[^;{}#]*?\b(\w+)\s*\([^;{}]*\)\s*;", text, flags=re.M):
        names.append(stmt)
    return names


def exported(lib: Path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("lib", sorted(HEADERS))
def test_library_exports_every_declared_function(lib):
    path = glint_hip.LIB_DIR / lib
    assert path.is_file(), f"{path} not built"
    ctypes.CDLL(str(path))  # loads
    syms = exported(path)
    declared = [f for h in HEADERS[lib] for f in declared_functions(h)]
    assert declared, "header parse found nothing"
    missing = [f for f in declared if f not in syms]
    assert not missing, missing
    # and nothing but the declared C ABI leaks out
    assert syms <= set(declared), sorted(syms - set(declared))


def test_reference_symbol_set_present():
    """The names the reference's callers bind (glint_cuda.py:28-49, glint_encode.h,
    glint_htile.h, attach/CONTRACT.md)."""
    enc = exported(glint_hip.LIB_DIR / "libglint_encode.so")
    for s in ("glint_encode_bf16_host", "glint_encode_f32_host", "glint_encode_n_absmax", "glint_encode_n_packed",
              "glint_expand_packed_to_f32_host", "glint_expand_packed_to_f32_device",
              "launch_glint_htile_s3_f32_stream", "launch_glint_htile_s3_f32"):
        assert s in enc, s
    p7 = exported(glint_hip.LIB_DIR / "libp7_kernels.so")
    # the twelve symbols cuda/p7_attach_check.c:11-14 requires, plus the rest of the attach contract
    for s in ("p7_abi_version", "p7_abi_selftest", "int8_mma_gemm", "glint_plug_streamer_create",
              "glint_plug_streamer_set_host_data", "glint_plug_streamer_start", "glint_plug_streamer_acquire",
              "glint_plug_streamer_release", "glint_plug_streamer_get_stats", "glint_plug_streamer_destroy",
              "p7_int8_gemm_flat", "p7_int8_gemm_plug_flat",
              "int8_mma_gemm_plug", "int8_mma_gemm_plug_fused", "int8_mma_gemm_resolve",
              "glint_plug_streamer_reset_stats"):
        assert s in p7, s


def test_size_helpers_match_reference_semantics():
    lib = glint_hip.encode_lib()
    assert lib.glint_encode_n_absmax(4096 * 4096, 64) == 262144
    assert lib.glint_encode_n_absmax(100, 23) == 5
    assert lib.glint_encode_n_absmax(100, 0) == 0 and lib.glint_encode_n_absmax(100, -3) == 0
    assert lib.glint_encode_n_packed(4096 * 4096) == 8388608
    assert lib.glint_encode_n_packed(7) == 4 and lib.glint_encode_n_packed(0) == 0


def test_bad_arguments_rejected_without_a_device():
    lib = glint_hip.encode_lib()
    null = None
    assert lib.glint_encode_bf16_device(null, 10, 64, null, null, null, null) == -1
    assert lib.glint_encode_bf16_device(null, 10, 0, null, null, null, null) == -1
    assert lib.glint_encode_bf16_host(null, -1, 64, null, null, null) == -1
    assert lib.glint_encode_bf16_host(null, 0, 64, null, null, null) == 0  # empty input: nothing to do
    assert lib.glint_expand_packed_to_f32_device(null, null, null, 10, 64, null, null) == -1
    assert lib.launch_glint_htile_s3_f32(null, null, null, null, null, 1, 1, 1, 64) == -1
    one = ctypes.c_void_p(8)
    assert lib.launch_glint_htile_s3_f32(one, one, one, one, one, 1, 1, 1, 0) == -2
    p7 = glint_hip.p7_lib()
    assert p7.p7_abi_version() == b"p7_attach_abi_v1"
    bad = glint_hip.Int8MmaLinear(8, 8, 64, 96)  # k_in % 64 != 0 (test_int8_mma_gemm.cu:201-205)
    assert p7.int8_mma_gemm(one, bad, one, 1, one, one, null) == 1
    assert p7.p7_int8_gemm_flat(one, one, one, 64, 96, one, 1, one, one, null) == 1
    assert p7.glint_int8_gemm_i32(one, one, one, 4, 4, 100, null) == 1
    ok = glint_hip.Int8MmaLinear(16, 16, 64, 128)
    x16 = ctypes.c_void_p(16)
    assert p7.int8_mma_gemm_plug(x16, ok, null, one, one, 1, x16, one, x16, null) == 1  # plug missing
    assert p7.int8_mma_gemm_plug_fused(one, bad, one, one, one, 1, one, one, null) == 1
    assert p7.p7_int8_gemm_plug_flat(one, one, one, one, one, 64, 96, one, 1, one, one, null) == 1
    # resolve: the three plug pointers must be all set or all NULL (int8_mma_gemm.h:56-61)
    assert p7.int8_mma_gemm_resolve(x16, ok, one, null, one, 1, x16, one, x16, one, x16, null) == 1
    # W8A16: a pending error (here: no device) or a bad argument returns nonzero, launching nothing
    assert p7.int8_tile_gemm_bf16(null, glint_hip.Int8PinLinear(16, 16, 64, 128), one, 1, null) != 0
    # streamer argument checks come before any device call (glint_plug_streamer.h codes)
    h = ctypes.c_void_p()
    sizes = (ctypes.c_uint64 * 1)(16)
    assert p7.glint_plug_streamer_create(ctypes.byref(h), 0, sizes, null, null) == -1
    assert p7.glint_plug_streamer_create(ctypes.byref(h), 65, sizes, null, null) == -1
    assert p7.glint_plug_streamer_start(null) == -1
    assert p7.glint_plug_streamer_release(null, 0) == -1
    p = ctypes.c_void_p()
    assert p7.glint_plug_streamer_acquire(null, 0, ctypes.byref(p)) == -1
    assert p7.glint_plug_streamer_set_host_data(null, 0, one, 16) == -1


def test_drop_in_module_surface():
    from glint_amd import glint_cuda
    for name in ("lib_path", "load", "encode_bf16_cuda", "expand_cuda", "gpu_ok"):
        assert callable(getattr(glint_cuda, name))
    assert glint_cuda.lib_path() == glint_hip.LIB_DIR / "libglint_encode.so"


def test_loaders_header_semantics():
    """include/glint_htile_load.h restates the reference's tail-safe loaders: compile a
    small host program against it and check rows/columns outside the matrix read 0."""
    src = r'''
#include "glint_htile_load.h"
#include <stdio.h>
int main(void) {
    /* 3 x 5 matrix, element i has nibble (i % 15) + 1 */
    uint8_t pk[8] = {0};
    for (int i = 0; i < 15; ++i) pk[i >> 1] |= (uint8_t)(((i % 15) + 1) << ((i & 1) * 4));
    int bad = 0;
    for (int row = 0; row < 4; ++row)
        for (int k = 0; k < 6; ++k) {
            uint8_t b = glint_packed_tile_byte(pk, row, 3, 5, k);
            int lo = (row < 3 && k < 5) ? (row * 5 + k) % 15 + 1 : 0;
            int hi = (row < 3 && k + 1 < 5) ? (row * 5 + k + 1) % 15 + 1 : 0;
            bad += b != (uint8_t)(lo | (hi << 4));
        }
    printf("%d\n", bad);
    return bad != 0;
}
'''
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        c = Path(td) / "t.c"
        c.write_text(src)
        exe = Path(td) / "t"
        subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(c), "-o", str(exe)], check=True)
        r = subprocess.run([str(exe)], capture_output=True, text=True)
        assert r.returncode == 0 and r.stdout.strip() == "0"
