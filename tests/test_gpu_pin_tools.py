"""GPU tests of the pin tools' device path (glint_amd.pin_tools).

This restates the reference's tool tests (test_glint_tools.py:77-106, 133-148, 216-228,
240-251) with the encode and expand on the MI355X:
- convert writes the oracle's bytes for every linear (BF16, F16 and F32 sources), with
  the reference's file set, index and report fields;
- verify passes with both gates (host re-encode parity and device-vs-host expand);
- unpin gives the oracle's BF16, F32 and F16 expansions;
- the official safetensors reader opens every file.
A larger two-shard model exercises the copy/compute overlap and prints its rate.
"""
import json
import tempfile
import time
from pathlib import Path

import numpy as np
import pytest

from glint_amd import pin_tools as P
from glint_amd.tensorfile import TensorFile, save
from tests.gpu_util import torch_cuda
from tests.pin_fixtures import bf16_bytes, dense_f32, toy_shards, write_model

pytestmark = pytest.mark.gpu


def _module_bytes(pin_dir: Path, stem: str):
    with P.Pin(pin_dir) as pin:
        return pin.module(stem)


def test_convert_writes_the_oracle_pin(oracle):
    torch_cuda()
    print("pin tools: convert toy shards", flush=True)
    with tempfile.TemporaryDirectory() as td:
        src, pin_dir = Path(td) / "src", Path(td) / "pin"
        write_model(src, toy_shards(), index=True)
        got = P.convert(src, pin_dir)
        pin = got["pin"]
        assert pin["schema"] == "glint_pin_v1" and pin["n_converted"] == 4
        assert pin["backends"] == ["hip_bf16", "hip_f32"] and pin["backend"] == "mixed"
        assert pin["sidecar"] == ["config.json"] and (pin_dir / "config.json").is_file()
        assert pin["rmse_max"] is not None and pin["rmse_max"] < 1e-2
        index = json.loads((pin_dir / P.INDEX_NAME).read_text())
        assert index["weight_map"]["_glint_cells"] == "model-00001-of-00002.safetensors"
        assert index["weight_map"]["layers.1.up.weight.glint_plug"] == "model-00002-of-00002.safetensors"
        assert index["weight_map"]["layers.0.norm.weight"] == "model-00001-of-00002.safetensors"
        report = json.loads((pin_dir / "CONVERT_REPORT.json").read_text())
        assert [m["src"] for m in report["modules"]] == ["layers.0.q", "layers.0.o", "layers.1.up", "layers.1.down"]
        for shard, tensors in toy_shards().items():
            for name, dtype, shape, raw in tensors:
                if not name.endswith(".weight") or "norm" in name:
                    continue
                stem = name[:-7]
                state, hole, plug, am = _module_bytes(pin_dir, stem)
                assert state == {"quant_type": "glint", "blocksize": 64, "shape": list(shape), "src_dtype": dtype}
                w = dense_f32(dtype, raw)
                oh, op, oam = oracle.encode_f32(w, 64)
                assert hole == oh.tobytes() and plug == op.tobytes() and am == oam.tobytes(), stem
                rec = oracle.expand_f32(oh, op, oam, w.size, 64)
                want = float(np.sqrt(np.mean((w.astype(np.float64) - rec.astype(np.float64)) ** 2)))
                row = next(m for m in report["modules"] if m["src"] == stem)
                assert row["rmse"] == pytest.approx(want, rel=1e-9, abs=1e-12), stem
                assert row["shard"] == shard
        with P.Pin(pin_dir) as p, TensorFile(src / "model-00001-of-00002.safetensors") as s:
            assert p.blob("layers.0.norm.weight") == s.blob("layers.0.norm.weight")
            assert p.entry("layers.0.q.weight").shape == (512, 1)


def test_verify_gates_and_unpin(oracle):
    torch_cuda()
    print("pin tools: verify --parity --cuda, unpin", flush=True)
    with tempfile.TemporaryDirectory() as td:
        src, pin_dir = Path(td) / "src", Path(td) / "pin"
        write_model(src, toy_shards(), index=True)
        P.convert(src, pin_dir)
        ev = P.verify(pin_dir, src, parity=True, cuda=True)
        assert ev["ok"], ev["failures"]
        assert ev["n_modules"] == 4
        assert all(m["parity"]["plug_bytes_differ"] == 0 and m["cuda_expand_max_abs"] == 0.0 for m in ev["modules"])
        for dt in ("BF16", "F32", "F16"):
            back = Path(td) / f"back_{dt}"
            res = P.unpin(pin_dir, back, dt)
            assert res["n_expanded"] == 4 and len(res["shards"]) == 2
            assert (back / "config.json").is_file() and (back / P.INDEX_NAME).is_file()
            with P.Pin(pin_dir) as pin:
                for stem in pin.stems():
                    state, hole, plug, am = pin.module(stem)
                    n = int(np.prod(state["shape"]))
                    hh, pp = np.frombuffer(hole, np.uint8), np.frombuffer(plug, np.uint8)
                    aa = np.frombuffer(am, np.float32)
                    shard = pin.where[stem + ".weight"]
                    with TensorFile(back / shard) as st:
                        info = st.entries[stem + ".weight"]
                        assert info.dtype == dt and list(info.shape) == state["shape"]
                        got = st.blob(stem + ".weight")
                        assert "_glint_cells" not in st.entries
                    if dt == "BF16":
                        want = oracle.expand_bf16(hh, pp, aa, n, 64).tobytes()
                    else:
                        f = oracle.expand_f32(hh, pp, aa, n, 64)
                        want = (f if dt == "F32" else f.astype("<f2")).tobytes()
                    assert got == want, (dt, stem)
        with TensorFile(Path(td) / "back_BF16" / "model-00002-of-00002.safetensors") as st, \
                TensorFile(src / "model-00002-of-00002.safetensors") as s:
            assert st.blob("layers.1.up.bias") == s.blob("layers.1.up.bias")


def test_files_load_in_the_official_reader():
    safetensors = pytest.importorskip("safetensors")
    torch_cuda()
    with tempfile.TemporaryDirectory() as td:
        src, pin_dir = Path(td) / "src", Path(td) / "pin"
        write_model(src, toy_shards(), index=True)
        P.convert(src, pin_dir)
        P.unpin(pin_dir, Path(td) / "back", "F32")
        files = list(pin_dir.glob("*.safetensors")) + list((Path(td) / "back").glob("*.safetensors"))
        assert len(files) == 4
        for f in files:
            with safetensors.safe_open(str(f), "np") as h:
                for k in h.keys():
                    if h.get_slice(k).get_dtype() != "BF16":  # numpy has no bfloat16
                        h.get_tensor(k)


def test_pipeline_on_a_larger_model(oracle):
    """Two shards of 4096-wide BF16 linears (about 200 MB): every module's bytes equal the
    oracle's on a row sample, and the unpin round trip equals the oracle's BF16 expand."""
    torch = torch_cuda()
    rng = np.random.default_rng(77)
    shards = {}
    for s in range(2):
        tensors = []
        for l in range(3):
            w = (rng.standard_normal((4096, 4096), dtype=np.float32) * 0.02)
            tensors.append((f"layers.{3 * s + l}.mlp.weight", "BF16", (4096, 4096), bf16_bytes(w)))
            tensors.append((f"layers.{3 * s + l}.norm.weight", "F32", (4096,), np.ones(4096, np.float32).tobytes()))
        shards[f"model-0000{s + 1}-of-00002.safetensors"] = tensors
    with tempfile.TemporaryDirectory() as td:
        src, pin_dir = Path(td) / "src", Path(td) / "pin"
        write_model(src, shards, index=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        got = P.convert(src, pin_dir)
        dt = time.perf_counter() - t0
        mb = 6 * 4096 * 4096 * 2 / 1e6
        print(f"pin tools: convert {mb:.0f} MB BF16 in {dt:.2f} s ({mb / dt:.0f} MB/s, file I/O and PCIe inclusive)",
              flush=True)
        assert got["pin"]["n_converted"] == 6
        for shard, tensors in shards.items():
            for name, dtype, shape, raw in tensors:
                if "mlp" not in name:
                    continue
                state, hole, plug, am = _module_bytes(pin_dir, name[:-7])
                rows = slice(1000 * 4096, 1064 * 4096)  # 64 rows, block aligned
                oh, op, oam = oracle.encode_bf16(np.frombuffer(raw, "<u2")[rows], 64)
                assert hole[1000 * 2048:1064 * 2048] == oh.tobytes()
                assert plug[1000 * 2048:1064 * 2048] == op.tobytes()
                assert am[1000 * 256:1064 * 256] == oam.tobytes()
        t0 = time.perf_counter()
        P.unpin(pin_dir, Path(td) / "back")
        print(f"pin tools: unpin {mb:.0f} MB BF16 in {time.perf_counter() - t0:.2f} s", flush=True)
        with TensorFile(Path(td) / "back" / "model-00002-of-00002.safetensors") as st:
            state, hole, plug, am = _module_bytes(pin_dir, "layers.5.mlp")
            n = 4096 * 4096
            want = oracle.expand_bf16(np.frombuffer(hole, np.uint8), np.frombuffer(plug, np.uint8),
                                      np.frombuffer(am, np.float32), n, 64)
            assert st.blob("layers.5.mlp.weight") == want.tobytes()
