"""Exhaustive CPU proofs behind the fast encode (built from this repo's sources with gcc):

* the bucket table reproduces the reference's first-minimum scan for every float in
  [-1, 1] and for NaN (glint_amd/csrc/gen_code_table.c --verify);
* the committed glint_code_table.inc is what the generator produces;
* the fast path's one-multiply quotient q = RN(w * RN(1/s)), with RN(1/s) from the
  128-entry reciprocal table, stays in [-1, 1] and gives the code of the IEEE quotient
  w / s for every bf16 (w, absmax) pair the fast path sees, both signs, also with a
  flush-to-zero multiply (tests/native/check_encode_quotient.c);
* the three-plane BF16 split of the f32-out H-TILE on MFMA is exact for every f32 weight
  (tests/native/check_split3.c).
"""
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
