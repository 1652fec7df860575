"""CPU checks of the pin tools (glint_amd.pin_tools, glint_amd.tensorfile, glint_amd.host_codec).

The container format is checked against the safetensors specification and the official
reader. The host codec that verify's gates use is pinned against the oracle. Dry-run
plans, layout checks and the parity gate run on a pin assembled here from oracle bytes.
Encoding and expanding need the GPU: without one, convert and unpin must refuse (tested
here); with one they are tested in test_gpu_pin_tools.py.
"""
import json
import struct
import tempfile
from pathlib import Path

import numpy as np
import pytest

from glint_amd import codebook, host_codec, pin_tools as P
from glint_amd.tensorfile import TensorFile, save
from tests.pin_fixtures import bf16_bytes, dense_f32, gauss, toy_shards, write_model


def test_container_offsets_are_contiguous_and_header_aligned():
    """Specification: the data section is fully indexed with no holes
    (test_glint_tools.py:229-238) and starts on an 8-byte boundary."""
    with tempfile.TemporaryDirectory() as td:
        f = Path(td) / "m.safetensors"
        n = save(f, [("a", "U8", (3,), b"abc"), ("b", "F32", (1,), b"\0" * 4), ("c", "U8", (1,), b"z")],
                 meta={"format": "pt"})
        assert n == 8
        raw = f.read_bytes()
        (hlen,) = struct.unpack("<Q", raw[:8])
        assert (8 + hlen) % 8 == 0
        header = json.loads(raw[8:8 + hlen])
        assert list(header)[0] == "__metadata__" and header["__metadata__"] == {"format": "pt"}
        spans = sorted(tuple(v["data_offsets"]) for k, v in header.items() if k != "__metadata__")
        assert spans[0][0] == 0 and all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
        assert 8 + hlen + spans[-1][1] == len(raw)
        with TensorFile(f) as tf:
            assert tf.blob("c") == b"z" and tf.blob("a") == b"abc" and tf.meta == {"format": "pt"}
            assert tf.entries["b"].count == 1 and tf.array("a", np.uint8).tolist() == [97, 98, 99]
            assert list(tf) == ["a", "b", "c"]
        assert [p.name for p in Path(td).iterdir()] == ["m.safetensors"]  # no temporary file left


def test_saved_file_mode_follows_the_umask():
    """save() writes through a temporary file (mkstemp, mode 0600) and renames it; the file
    it leaves has the mode a plain open(path, "wb") would give: 0666 less the umask."""
    import os
    old = os.umask(0o022)
    try:
        with tempfile.TemporaryDirectory() as d:
            for mask in (0o022, 0o002, 0o077):
                os.umask(mask)
                path = Path(d) / f"m{mask:o}.safetensors"
                save(path, [("w", "F32", [2], np.zeros(2, np.float32))])
                assert (path.stat().st_mode & 0o777) == (0o666 & ~mask), (oct(mask), oct(path.stat().st_mode))
    finally:
        os.umask(old)


def test_official_reader_accepts_our_files():
    safetensors = pytest.importorskip("safetensors")
    with tempfile.TemporaryDirectory() as td:
        f = Path(td) / "m.safetensors"
        vals = np.arange(12, dtype=np.float32)
        save(f, [("w", "F32", (3, 4), vals.tobytes()), ("u", "U8", (5, 1), bytes(range(5)))])
        with safetensors.safe_open(str(f), "np") as h:
            assert np.array_equal(h.get_tensor("w"), vals.reshape(3, 4))
            assert h.get_tensor("u").reshape(-1).tolist() == [0, 1, 2, 3, 4]


def _raw_file(f: Path, header: dict, data: bytes) -> None:
    hb = json.dumps(header).encode()
    hb += b" " * ((-(len(hb) + 8)) % 8)
    f.write_bytes(struct.pack("<Q", len(hb)) + hb + data)


def test_reader_rejects_bad_ranges_and_writer_bad_sizes():
    with tempfile.TemporaryDirectory() as td:
        f = Path(td) / "bad.safetensors"
        _raw_file(f, {"x": {"dtype": "U8", "shape": [10], "data_offsets": [0, 10]}}, b"abc")
        with pytest.raises(ValueError, match="spans"):
            TensorFile(f)
        _raw_file(f, {"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"abcd")
        with pytest.raises(ValueError, match="holds"):
            TensorFile(f)
        f.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
        with pytest.raises(ValueError, match="does not fit"):
            TensorFile(f)
        with pytest.raises(ValueError, match="bytes for shape"):
            save(Path(td) / "w.safetensors", [("y", "F32", (3,), b"\0" * 8)])
        with pytest.raises(ValueError, match="not a safetensors dtype"):
            save(Path(td) / "w.safetensors", [("y", "Q4", (3,), b"\0" * 3)])
        assert not (Path(td) / "w.safetensors").exists()


def test_resolve_shards_rules():
    with tempfile.TemporaryDirectory() as td:
        root = Path(td)
        write_model(root / "sharded", toy_shards(), index=True)
        got = P.resolve_shards(root / "sharded")
        assert [p.name for p in got] == sorted(toy_shards())
        one = root / "one"
        one.mkdir()
        save(one / "weights.safetensors", [("a.weight", "BF16", (2, 64), bf16_bytes(gauss(128, 7)))])
        assert [p.name for p in P.resolve_shards(one)] == ["weights.safetensors"]
        save(one / "other.safetensors", [("b", "U8", (1,), b"x")])
        with pytest.raises(FileNotFoundError):
            P.resolve_shards(one)
        (root / "sharded" / "model-00002-of-00002.safetensors").unlink()
        with pytest.raises(FileNotFoundError):
            P.resolve_shards(root / "sharded")


def test_dry_run_plan():
    """Headers only: the linears are the dense 2-D .weight tensors that are not norms,
    biases or rotary tables (glint_pin.py:100-122)."""
    with tempfile.TemporaryDirectory() as td:
        src = Path(td) / "src"
        write_model(src, toy_shards(), index=True)
        plan = P.convert(src, Path(td) / "pin", dry_run=True)
        assert plan["schema"] == "glint_pin_v1"
        assert plan["linears"] == ["layers.0.q.weight", "layers.0.o.weight", "layers.1.up.weight",
                                   "layers.1.down.weight"]
        assert plan["n_keep"] == 2 and plan["shards"] == sorted(toy_shards())
        assert not (Path(td) / "pin").exists()


def test_convert_and_unpin_refuse_without_a_gpu():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with tempfile.TemporaryDirectory() as td:
        src = Path(td) / "src"
        write_model(src, toy_shards(), index=True)
        with pytest.raises(RuntimeError, match="GPU"):
            P.convert(src, Path(td) / "pin")
        with pytest.raises(NotImplementedError):
            P.convert(src, Path(td) / "pin", force_python=True)


# ------------------------------------------------------------- host codec vs the oracle
def test_host_codec_matches_the_oracle(oracle):
    """verify's gates compare against the host codec, so it must give the oracle's bytes:
    seeded Gaussians with a zero block, NaN, inf and an odd length."""
    w = np.asarray(gauss(64 * 41 + 7, 5), dtype=np.float32)
    w[128:192] = 0.0
    w[300], w[301], w[777] = np.nan, np.inf, -np.inf
    h, p, am = host_codec.encode_f32(w, 64)
    oh, op, oam = oracle.encode_f32(w, 64)
    assert h == oh.tobytes() and p == op.tobytes() and am.tobytes() == oam.tobytes()
    rec = host_codec.expand(h, p, am, w.size, 64)
    assert rec.tobytes() == oracle.expand_f32(oh, op, oam, w.size, 64).tobytes()
    every = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)  # every bf16 pattern, specials included
    h, p, am = host_codec.encode_f32(every, 64)
    oh, op, oam = oracle.encode_f32(every, 64)
    assert h == oh.tobytes() and p == op.tobytes() and am.tobytes() == oam.tobytes()
    for bs in (23, 128):
        h, p, am = host_codec.encode_f32(w, bs, block_chunk=3)
        oh, op, oam = oracle.encode_f32(w, bs)
        assert h == oh.tobytes() and p == op.tobytes() and am.tobytes() == oam.tobytes()


def test_host_codec_tables_are_the_pinned_ones():
    assert host_codec.CELLS.tobytes() == codebook.cells_f32_bytes()
    assert host_codec.PARENT.tobytes() == codebook.parent_f32_bytes()


# ------------------------------------------- verify on a pin assembled from oracle bytes
def _assemble_pin(oracle, src: Path, pin: Path, bs: int = 64):
    """A pin laid out as convert lays it out, with the oracle's encode."""
    shards = P.resolve_shards(src)
    pin.mkdir(parents=True)
    weight_map, n_conv = {}, 0
    for si, wf in enumerate(shards):
        items = []
        with TensorFile(wf) as tf:
            for name, e in tf.entries.items():
                raw = tf.blob(name)
                if P.is_linear(name, e.dtype, e.shape):
                    h, p, am = oracle.encode_f32(dense_f32(e.dtype, raw), bs)
                    t = P.module_names(name[:-7])
                    state = json.dumps({"quant_type": "glint", "blocksize": bs, "shape": list(e.shape),
                                        "src_dtype": e.dtype}, separators=(",", ":")).encode()
                    items += [(t["hole"], "U8", (h.size, 1), h.tobytes()),
                              (t["plug"], "U8", (p.size, 1), p.tobytes()),
                              (t["absmax"], "F32", (am.size,), am.tobytes()),
                              (t["state"], "U8", (len(state),), state)]
                    n_conv += 1
                else:
                    items.append((name, e.dtype, e.shape, raw))
        if si == 0:
            items.append(("_glint_cells", "F32", (16, 16), codebook.cells_f32_bytes()))
        weight_map.update(dict.fromkeys((it[0] for it in items), wf.name))
        save(pin / wf.name, items, meta={"format": "pt", "quantization": "glint"})
    (pin / P.INDEX_NAME).write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    (pin / "pin.json").write_text(json.dumps({"schema": "glint_pin_v1", "n_converted": n_conv, "backend": "test"}))


def test_verify_layout_rmse_and_parity_on_oracle_pin(oracle):
    with tempfile.TemporaryDirectory() as td:
        src, pin = Path(td) / "src", Path(td) / "pin"
        write_model(src, toy_shards(), index=True)
        _assemble_pin(oracle, src, pin)
        ev = P.verify(pin, src, parity=True)
        assert ev["ok"], ev["failures"]
        assert ev["n_modules"] == 4 and ev["rmse_max"] < 1e-2
        assert all(m["parity"]["hole_bytes_differ"] == 0 and m["parity"]["plug_bytes_differ"] == 0
                   for m in ev["modules"])


def test_verify_catches_corrupt_plug_and_pad(oracle):
    """One flipped plug byte is found by the parity gate at its offset
    (test_glint_tools.py:133-148); a nonzero pad nibble on odd n fails the layout check."""
    with tempfile.TemporaryDirectory() as td:
        src, pin = Path(td) / "src", Path(td) / "pin"
        write_model(src, {"model.safetensors": [("lin.weight", "BF16", (8, 64), bf16_bytes(gauss(512, 4))),
                                                ("odd.weight", "BF16", (3, 21), bf16_bytes(gauss(63, 9)))]},
                    index=False)
        _assemble_pin(oracle, src, pin)
        (pin / P.INDEX_NAME).unlink()
        f = pin / "model.safetensors"
        with TensorFile(f) as tf:
            off_plug = tf.entries["lin.weight.glint_plug"].begin + 3
            off_pad = tf.entries["odd.weight"].end - 1
        raw = bytearray(f.read_bytes())
        raw[off_plug] ^= 0x11
        raw[off_pad] |= 0x50
        f.write_bytes(bytes(raw))
        ev = P.verify(pin, src, parity=True)
        assert not ev["ok"]
        lin = next(m for m in ev["modules"] if m["module"] == "lin")
        assert lin["parity"]["plug_first_diff"] == 3 and lin["parity"]["plug_bytes_differ"] == 1
        odd = next(m for m in ev["modules"] if m["module"] == "odd")
        assert any("pad nibble" in q for q in odd["problems"])


def test_verify_flags_missing_cells_and_count(oracle):
    with tempfile.TemporaryDirectory() as td:
        src, pin = Path(td) / "src", Path(td) / "pin"
        write_model(src, toy_shards(), index=True)
        _assemble_pin(oracle, src, pin)
        meta = json.loads((pin / "pin.json").read_text())
        meta["n_converted"] = 7
        (pin / "pin.json").write_text(json.dumps(meta))
        ev = P.verify(pin)
        assert not ev["ok"] and any("n_converted=7" in f for f in ev["failures"])
