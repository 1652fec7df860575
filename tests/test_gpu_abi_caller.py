"""The C ABI from a C++ caller (no ctypes): tests/native/abi_caller.cpp is compiled against
include/glint_encode.h and include/glint_htile.h and linked with -lglint_encode by
`python -m glint_amd.build`, as the reference's own C/C++ tests link the library. Each
suite runs the binary in its own process and must print PASS for every case; the suites
restate reference tests/test_htile_k_bounds_device.cu:40-118 and tests/test_glint_htile.cu:
63-153, the glint_cuda.gpu_ok probe and the device/host expand pair."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
EXE = ROOT / "tests" / "native" / "bin" / "abi_caller"


def _exe():
    if not EXE.is_file():
        pytest.fail("tests/native/bin/abi_caller is not built: run `python -m glint_amd.build`")
    return EXE


def test_caller_links_the_c_abi():
    """CPU check: the binary names the ABI entry points as undefined symbols resolved from
    libglint_encode.so, not from a copy of its own."""
    out = subprocess.run(["nm", "-D", "--undefined-only", str(_exe())], capture_output=True, text=True, check=True)
    for sym in ("glint_encode_bf16_host", "glint_expand_packed_to_f32_device", "glint_expand_packed_to_f32_host",
                "launch_glint_htile_s3_f32", "launch_glint_htile_s3_f32_stream", "glint_encode_n_absmax"):
        assert sym in out.stdout, sym
    ldd = subprocess.run(["ldd", str(_exe())], capture_output=True, text=True).stdout
    assert "libglint_encode.so" in ldd


@pytest.mark.gpu
@pytest.mark.parametrize("suite", ["gpu_ok", "expand", "kbounds", "ten", "prefill"])
def test_c_caller_suite(suite):
    print(f"abi_caller {suite}", flush=True)
    r = subprocess.run([str(_exe()), suite], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
    assert "PASS abi_caller suites=1 failed=0" in r.stdout
    assert "FAIL" not in r.stdout
