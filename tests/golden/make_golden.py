#!/usr/bin/env python3
"""Writes tests/golden/encode_4096x4096_outliers.json: the CPU-reference configuration
(4096 x 4096 BF16 weights ~ N(0, 0.02^2) from numpy default_rng(1001), 0.1% of entries
scaled x10 before BF16 rounding, blocksize 64) with SHA-256 digests of its GLINT pin
(hole and plug planes, absmax) and of the BF16 expand, plus the expand RMSE.

Expected outputs come from the C oracle (oracle/glint_oracle.c), which the CPU tests pin
to the reference's known answers, header hash and linear-scan definition. The fixture lets
the GPU tests check the full-size encode and expand against committed digests, and a CPU
test re-derives it (catching drift in the oracle or the input generator).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
OUT = Path(__file__).resolve().parent / "encode_4096x4096_outliers.json"
N_ROWS = N_COLS = 4096
SEED = 1001
BS = 64


def config0_input() -> np.ndarray:
    """BF16 bits of the CPU-reference configuration's weight matrix (flattened)."""
    from oracle import glint_oracle as G
    rng = np.random.default_rng(SEED)
    n = N_ROWS * N_COLS
    w = rng.normal(0.0, 0.02, n).astype(np.float32)
    idx = rng.choice(n, n // 1000, replace=False)
    w[idx] *= np.float32(10.0)
    return G.f32_to_bf16_bits(w)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def compute(oracle) -> dict:
    from oracle import glint_oracle as G
    u16 = config0_input()
    n = u16.size
    hole, plug, am = oracle.encode_bf16(u16, BS)
    out16 = oracle.expand_bf16(hole, plug, am, n, BS)
    w = G.bf16_bits_to_f32(u16).astype(np.float64)
    e = G.bf16_bits_to_f32(out16).astype(np.float64)
    return {
        "config": "BASELINE configs[0]: W[4096x4096] ~ N(0,0.02^2), default_rng(1001), "
                  "rng.choice(n, n//1000, replace=False) entries x10, f32 -> BF16 RNE, blocksize 64",
        "n": int(n), "blocksize": BS,
        "input_bf16_sha256": sha(u16),
        "hole_sha256": sha(hole), "plug_sha256": sha(plug), "absmax_sha256": sha(am),
        "expand_bf16_sha256": sha(out16),
        "expand_rmse": float(np.sqrt(np.mean((w - e) ** 2))),
        "hole_head": hole[:16].tolist(), "plug_head": plug[:16].tolist(),
        "absmax_head": [float(v) for v in am[:4]],
    }


def main() -> int:
    from oracle import glint_oracle as G
    OUT.write_text(json.dumps(compute(G.Oracle()), indent=1) + "\n")
    print(OUT.read_text())
    return 0


if __name__ == "__main__":
    sys.exit(main())
