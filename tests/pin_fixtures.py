"""Toy models for the pin-tool tests, shaped like the reference's own fixtures
(test_glint_tools.py:28-76): two shards, a BF16 linear, a norm, an odd-sized F32
linear whose blocks straddle rows, a linear with an all-zero block, a bias, and a
config.json sidecar. An F16 linear is added to cover the third source dtype."""
import json
import random
import struct
from pathlib import Path

import numpy as np

from glint_amd.tensorfile import save


def gauss(n, seed, scale=0.02):
    """random.Random(seed).gauss(0, scale), the reference tests' generator."""
    rng = random.Random(seed)
    return [rng.gauss(0.0, scale) for _ in range(n)]


def bf16_bytes(vals) -> bytes:
    u = np.asarray(vals, dtype=np.float32).view(np.uint32)
    r = ((u + (np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1)))) >> 16).astype("<u2")
    return r.tobytes()


def toy_shards():
    a = gauss(16 * 64, 1)
    b = gauss(8 * 63, 2)  # odd numel, blocks straddle rows
    c = gauss(4 * 128, 3)
    c[:64] = [0.0] * 64  # an all-zero block
    d = gauss(6 * 96, 4, scale=0.5)
    return {
        "model-00001-of-00002.safetensors": [
            ("layers.0.q.weight", "BF16", (16, 64), bf16_bytes(a)),
            ("layers.0.norm.weight", "BF16", (64,), bf16_bytes([1.0] * 64)),
            ("layers.0.o.weight", "F32", (8, 63), struct.pack("<" + "f" * len(b), *b)),
        ],
        "model-00002-of-00002.safetensors": [
            ("layers.1.up.weight", "BF16", (4, 128), bf16_bytes(c)),
            ("layers.1.up.bias", "BF16", (4,), bf16_bytes([0.5] * 4)),
            ("layers.1.down.weight", "F16", (6, 96), np.asarray(d, dtype="<f2").tobytes()),
        ],
    }


def write_model(root: Path, shards: dict, index: bool = True) -> None:
    root.mkdir(parents=True, exist_ok=True)
    weight_map = {}
    for shard, tensors in shards.items():
        save(root / shard, tensors)
        for t in tensors:
            weight_map[t[0]] = shard
    if index:
        (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    (root / "config.json").write_text('{"model_type": "toy"}')


def dense_f32(dtype: str, raw: bytes) -> np.ndarray:
    if dtype == "BF16":
        return (np.frombuffer(raw, "<u2").astype(np.uint32) << 16).view(np.float32)
    if dtype == "F16":
        return np.frombuffer(raw, "<f2").astype(np.float32)
    return np.frombuffer(raw, "<f4").astype(np.float32)
