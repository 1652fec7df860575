"""Exhaustive CPU proofs behind the fast encode (built from this repo's sources with gcc):

* the bucket table reproduces the reference's first-minimum scan for every float in
  [-1, 1] and for NaN (glint_amd/csrc/gen_code_table.c --verify);
* the committed glint_code_table.inc is what the generator produces;
* the fast path's one-multiply quotient q = RN(w * RN(1/s)), with RN(1/s) from the
  128-entry reciprocal table, stays in [-1, 1] and gives the code of the IEEE quotient
  w / s for every bf16 (w, absmax) pair the fast path sees, both signs, also with a
  flush-to-zero multiply (tests/native/check_encode_quotient.c);
* the three-plane BF16 split of the f32-out H-TILE on MFMA is exact for every f32 weight
  (tests/native/check_split3.c);
* the host C (the CPU oracle, the code-table generator and both checkers) runs clean under
  AddressSanitizer and UndefinedBehaviorSanitizer (the reference's CI runs its host C the
  same way, .github/workflows/ci.yml:62-65).
"""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "glint_amd" / "csrc"


def _build(tmp_path, src, name):
    exe = tmp_path / name
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", f"-I{ROOT / 'include'}", f"-I{CSRC}", str(src),
                    "-lm", "-o", str(exe)], check=True, capture_output=True)
    return exe


def test_code_table_is_generated_and_exhaustively_correct(tmp_path):
    exe = _build(tmp_path, CSRC / "gen_code_table.c", "gen")
    out = tmp_path / "t.inc"
    subprocess.run([str(exe), str(out)], check=True, timeout=300)
    assert out.read_bytes() == (CSRC / "glint_code_table.inc").read_bytes()
    r = subprocess.run([str(exe), "--verify"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "verify: 0 mismatches" in r.stdout


def test_fast_quotient_exhaustive_over_bf16_pairs(tmp_path):
    exe = _build(tmp_path, ROOT / "tests" / "native" / "check_encode_quotient.c", "quot")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "749099520 pairs" in r.stdout
    assert ("0 reciprocal mismatches, 0 |q| > 1, 0 code mismatches, 0 flush-to-zero code mismatches"
            in r.stdout)


def test_three_plane_split_exhaustive(tmp_path):
    exe = _build(tmp_path, ROOT / "tests" / "native" / "check_split3.c", "split3")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 sums differ, 0 lo not BF16, 0 special mismatches" in r.stdout


SAN = ["-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _build_san(tmp_path, srcs, name):
    exe = tmp_path / name
    subprocess.run(["gcc", *SAN, "-fopenmp", "-ffp-contract=off", f"-I{ROOT / 'include'}", f"-I{CSRC}",
                    *map(str, srcs), "-lm", "-o", str(exe)], check=True, capture_output=True)
    return exe


def test_host_c_under_sanitizers(tmp_path):
    """The oracle driven over every function and edge path (tests/native/oracle_sanitize.c),
    the code-table generator, and sampled runs of the two exhaustive checkers, each built
    with -fsanitize=address,undefined -fno-sanitize-recover=all: any report ends the run
    with a nonzero status."""
    env = dict(os.environ, OMP_NUM_THREADS="4", ASAN_OPTIONS="abort_on_error=0:detect_leaks=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    run = lambda args, t: subprocess.run(args, capture_output=True, text=True, timeout=t, env=env)
    exe = _build_san(tmp_path, [ROOT / "oracle" / "glint_oracle.c", ROOT / "tests" / "native" / "oracle_sanitize.c"],
                     "oracle_san")
    r = run([str(exe)], 120)
    assert r.returncode == 0 and "oracle under sanitizers" in r.stdout, r.stdout + r.stderr
    gen = _build_san(tmp_path, [CSRC / "gen_code_table.c"], "gen_san")
    out = tmp_path / "t.inc"
    r = run([str(gen), str(out)], 300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert out.read_bytes() == (CSRC / "glint_code_table.inc").read_bytes()
    quot = _build_san(tmp_path, [ROOT / "tests" / "native" / "check_encode_quotient.c"], "quot_san")
    r = run([str(quot), "--stride", "97"], 300)
    assert r.returncode == 0 and "0 code mismatches" in r.stdout, r.stdout + r.stderr
    split3 = _build_san(tmp_path, [ROOT / "tests" / "native" / "check_split3.c"], "split3_san")
    r = run([str(split3), "--stride", "65537"], 300)
    assert r.returncode == 0 and "0 sums differ" in r.stdout, r.stdout + r.stderr
