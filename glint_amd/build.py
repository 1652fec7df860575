"""Build the GLINT HIP libraries in-tree for gfx950.

    python -m glint_amd.build            # libraries + oracle
    python -m glint_amd.build --only-libs

Outputs (git-ignored, shipped with the tree):
    glint_amd/lib/libglint_encode.so   encode / expand / H-TILE (include/glint_encode.h, glint_htile.h)
    glint_amd/lib/libp7_kernels.so     attach ABI: INT8 GEMM (include/int8_mma_gemm.h, p7_attach.h)
    glint_amd/lib/libglint_probe.so    bench.py's HBM read ceiling (measurement only)
    glint_amd/lib/libglint_encode_tl.so  libglint_encode.so with the decode GEMV's per-wave
                                       timeline stamps (bench.py --timeline; measurement only)
    oracle/liboracle.so                CPU oracle (tests only)
    tests/native/bin/abi_caller        C++ caller of the C ABI, linked with -lglint_encode (tests only)
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
BUILD = ROOT / "_build"
ARCH = os.environ.get("GLINT_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-ffp-contract=off",  # every fused multiply-add in the kernels is an explicit fmaf
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]

LIBS = {
    "libglint_encode.so": ["glint_encode.hip", "glint_htile.hip", "glint_select.hip", "glint_noalloc.hip"],
    "libp7_kernels.so": ["int8_mma_gemm.hip", "int8_tile_gemm.hip", "p7_abi.cpp", "glint_plug_streamer.cpp", "p7_selftest.cpp"],
    # measurement only (bench.py's read ceiling), not part of the GLINT ABI
    "libglint_probe.so": ["hbm_probe.hip"],
    # measurement only (bench.py --timeline): libglint_encode.so with the decode GEMV's
    # per-wave stamps compiled in
    "libglint_encode_tl.so": ["glint_encode.hip", "glint_htile.hip+tl", "glint_select.hip", "glint_noalloc.hip"],
}
# source variants: "<file>+<tag>" compiles <file> with these extra flags
VARIANT_FLAGS = {"tl": ["-DGLINT_TIMELINE=1"]}


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(str, cmd))}\n{r.stdout}\n{r.stderr}")
    return r


def gen_code_table() -> None:
    """Regenerate glint_code_table.inc from the codebook (deterministic)."""
    BUILD.mkdir(exist_ok=True)
    exe = BUILD / "gen_code_table"
    _run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", f"-I{ROOT / 'include'}", f"-I{CSRC}",
          str(CSRC / "gen_code_table.c"), "-lm", "-o", str(exe)])
    tmp = BUILD / "glint_code_table.inc"
    _run([str(exe), str(tmp)])
    dst = CSRC / "glint_code_table.inc"
    if not dst.is_file() or dst.read_bytes() != tmp.read_bytes():
        shutil.copyfile(tmp, dst)


def _compile(src: str) -> Path:
    file, _, tag = src.partition("+")
    obj = BUILD / (file + (f".{tag}" if tag else "") + ".o")
    lang = ["-x", "hip"] if file.endswith(".hip") else []
    _run([HIPCC, *HIP_FLAGS, *VARIANT_FLAGS.get(tag, []), *lang, "-c", str(CSRC / file), "-o", str(obj)])
    return obj


def build_libs() -> None:
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    srcs = list(dict.fromkeys(s for files in LIBS.values() for s in files if (CSRC / s.partition("+")[0]).is_file()))
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    for lib, files in LIBS.items():
        present = [objs[f] for f in files if f in objs]
        if not present:
            continue
        out = LIB / lib
        tmp = LIB / (lib + ".tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, present)])
        os.replace(tmp, out)


NATIVE = ROOT / "tests" / "native"


def build_native_tests() -> None:
    """The C++ ABI caller: compiled against include/*.h only and linked with
    -lglint_encode (rpath to glint_amd/lib), as a reference C/C++ test links the library."""
    out = NATIVE / "bin"
    out.mkdir(exist_ok=True)
    exe = out / "abi_caller"
    tmp = out / "abi_caller.tmp"
    _run([HIPCC, "-O2", "-std=c++17", f"-I{ROOT / 'include'}", str(NATIVE / "abi_caller.cpp"),
          f"-L{LIB}", "-lglint_encode", "-Wl,-rpath,$ORIGIN/../../../glint_amd/lib", "-o", str(tmp)])
    os.replace(tmp, exe)


def build_oracle() -> None:
    _run(["make", "-C", str(ROOT / "oracle"), "-j4"])
    if Path("/root/reference").is_dir():
        _run(["make", "-C", str(ROOT / "oracle"), "ref"])


def build(only_libs: bool = False) -> None:
    gen_code_table()
    build_libs()
    build_native_tests()
    if not only_libs:
        build_oracle()


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--only-libs", action="store_true")
    args = ap.parse_args()
    build(args.only_libs)
    print("built:", ", ".join(sorted(p.name for p in LIB.glob("*.so"))))
    sys.exit(0)
