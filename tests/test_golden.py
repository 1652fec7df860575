"""The committed fixture for the CPU-reference configuration (tests/golden/): the C oracle
re-derives it exactly, and the numpy restatement (searchsorted nearest, a different
algorithm from the C oracle's linear scan) produces the same pin bytes."""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "golden"))
import make_golden  # noqa: E402

FIXTURE = json.loads((ROOT / "tests" / "golden" / "encode_4096x4096_outliers.json").read_text())


def test_oracle_reproduces_committed_fixture(oracle):
    got = make_golden.compute(oracle)
    for k in ("input_bf16_sha256", "hole_sha256", "plug_sha256", "absmax_sha256", "expand_bf16_sha256"):
        assert got[k] == FIXTURE[k], k
    assert abs(got["expand_rmse"] - FIXTURE["expand_rmse"]) <= 1e-12


def test_numpy_restatement_matches_fixture():
    from oracle import glint_oracle as G
    u16 = make_golden.config0_input()
    hole, plug, am = G.encode_bf16(u16, 64)
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert sha(hole) == FIXTURE["hole_sha256"]
    assert sha(plug) == FIXTURE["plug_sha256"]
    assert sha(am) == FIXTURE["absmax_sha256"]
    assert sha(G.expand_bf16(hole, plug, am, u16.size, 64)) == FIXTURE["expand_bf16_sha256"]
