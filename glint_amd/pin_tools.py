"""GLINT pin tools on the MI355X device path: convert, verify, unpin.

    python -m glint_amd.pin_tools convert --src MODEL --out PIN [--blocksize 64] [--dry-run]
    python -m glint_amd.pin_tools verify  --pin PIN [--src MODEL] [--parity] [--cuda] [--out F] [--quiet]
    python -m glint_amd.pin_tools unpin   --pin PIN --out DIR [--dtype BF16|F16|F32]

Interface kept from the reference's tools, so pins move between the two: the pin layout
(per linear "<stem>.weight" U8 [ceil(n/2), 1] hole plane, ".weight.glint_plug" U8 plug
plane, ".weight.absmax" F32 [ceil(n/bs)], ".weight.glint_state" JSON bytes; one
"_glint_cells" F32 [16, 16] in the first shard), the file set (shards named as the
source's, "model.safetensors.index.json" when sharded, "pin.json", "CONVERT_REPORT.json",
the copied sidecar files) and the JSON keys of every report (glint_pin.py:87-193,
glint_verify.py:48-144, glint_unpin.py:45-85).

Device path: each tensor to encode is copied from the shard's memory map into pinned
host memory, moved on a copy stream and encoded on a compute stream (BF16 from its bits,
F16 widened on the device, F32 as is); its RMSE comes from a device expand, and the planes
return through pinned memory. Work is queued one tensor ahead, so reading and staging the
next tensor overlaps the device work of the current one. unpin expands on the device the
same way. Without the HIP library or a GPU, convert and unpin raise RuntimeError; dry runs
and verify's layout checks need neither.
"""
from __future__ import annotations

import argparse
import json
import shutil
import sys
from collections import deque
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, Iterable, Iterator, List, Optional, Tuple

import numpy as np

from . import codebook
from . import host_codec as hc
from .tensorfile import TensorFile, save

# ---------------------------------------------------------------- format names
PIN_SCHEMA = "glint_pin_v1"
VERIFY_SCHEMA = "glint_verify_v1"
INDEX_NAME = "model.safetensors.index.json"
SINGLE_SHARD = "model.safetensors"
CELLS_TENSOR = "_glint_cells"
STATE_SUFFIX = ".weight.glint_state"
DENSE_DTYPES = ("BF16", "F16", "F32")
# files that make a pin (or an unpinned model) loadable, copied when present
SIDECAR = ("config.json", "generation_config.json", "tokenizer.json", "tokenizer_config.json",
           "special_tokens_map.json", "tokenizer.model", "vocab.json", "merges.txt", "added_tokens.json",
           "chat_template.jinja")
# substrings of tensor names that stay dense (normalisation, biases, rotary tables)
DENSE_KEEP = ("norm", "bias", "rotary", "cos_cached", "sin_cached")
EXPAND_GATE = 1e-5  # verify --cuda: largest |device - host| expand difference allowed (glint_verify.py:29)


def module_names(stem: str) -> Dict[str, str]:
    """The four tensors a converted linear becomes."""
    w = stem + ".weight"
    return {"hole": w, "plug": w + ".glint_plug", "absmax": w + ".absmax", "state": stem + STATE_SUFFIX}


def is_linear(name: str, dtype: str, shape) -> bool:
    """A tensor the pin encodes: a dense 2-D ".weight" that is not a norm, bias or rotary table."""
    low = name.lower()
    kept = name.endswith(".bias") or any(k in low for k in DENSE_KEEP)
    return dtype in DENSE_DTYPES and len(shape) == 2 and name.endswith(".weight") and not kept


def element_count(shape) -> int:
    return int(np.prod([int(d) for d in shape], dtype=np.int64)) if len(shape) else 1


def table_values() -> List[float]:
    return np.frombuffer(codebook.cells_f32_bytes(), dtype="<f4").tolist()


# ------------------------------------------------------------------- the source
class ModelSource:
    """Where a model's tensors live: a .safetensors file, or a directory holding
    model.safetensors, an index naming its shards, or a single .safetensors file."""

    def __init__(self, path: Path):
        root = Path(path).expanduser().resolve()
        self.sharded = False
        if not root.is_dir():
            self.dir, self.files = root.parent, [root]
            return
        self.dir = root
        if (root / SINGLE_SHARD).is_file():
            self.files = [root / SINGLE_SHARD]
        elif (root / INDEX_NAME).is_file():
            wanted = sorted(set(json.loads((root / INDEX_NAME).read_text())["weight_map"].values()))
            absent = [s for s in wanted if not (root / s).is_file()]
            if absent:
                raise FileNotFoundError(f"{root / INDEX_NAME} lists shards that are not there: {', '.join(absent)}")
            self.files = [root / s for s in wanted]
        else:
            found = sorted(root.glob("*.safetensors"))
            if len(found) != 1:
                raise FileNotFoundError(f"{root}: expected {SINGLE_SHARD}, {INDEX_NAME} or a single .safetensors "
                                        f"file, found {len(found)} .safetensors files")
            self.files = found
        self.sharded = len(self.files) > 1

    def lookup(self) -> Dict[str, TensorFile]:
        """Every tensor name -> its open file (the caller closes them: close_all)."""
        table: Dict[str, TensorFile] = {}
        for f in self.files:
            tf = TensorFile(f)
            table.update(dict.fromkeys(tf.entries, tf))
        return table


def resolve_shards(src: Path) -> List[Path]:
    """The source's shard files in order (see ModelSource)."""
    return ModelSource(src).files


def close_all(files: Iterable[TensorFile]) -> None:
    for tf in {id(f): f for f in files}.values():
        tf.close()


# ---------------------------------------------------------------------- the pin
class Pin:
    """An open pin directory: pin.json, every shard mapped, tensors found by name."""

    def __init__(self, root: Path):
        self.root = Path(root).expanduser().resolve()
        meta = self.root / "pin.json"
        if not meta.is_file():
            raise FileNotFoundError(f"{self.root} is not a pin: pin.json is missing")
        self.meta = json.loads(meta.read_text())
        idx = self.root / INDEX_NAME
        names = sorted(set(json.loads(idx.read_text())["weight_map"].values())) if idx.is_file() else [SINGLE_SHARD]
        self.shards: Dict[str, TensorFile] = {s: TensorFile(self.root / s) for s in names}
        self.where: Dict[str, str] = {t: s for s, tf in self.shards.items() for t in tf.entries}

    def close(self) -> None:
        close_all(self.shards.values())

    def __enter__(self) -> "Pin":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def entry(self, name: str):
        return self.shards[self.where[name]].entries[name]

    def blob(self, name: str) -> bytes:
        return self.shards[self.where[name]].blob(name)

    def stems(self) -> List[str]:
        return [t[:-len(STATE_SUFFIX)] for t in self.where if t.endswith(STATE_SUFFIX)]

    def table(self) -> Optional[List[float]]:
        return np.frombuffer(self.blob(CELLS_TENSOR), dtype="<f4").tolist() if CELLS_TENSOR in self.where else None

    def module(self, stem: str) -> Tuple[dict, bytes, bytes, bytes]:
        """(state, hole bytes, plug bytes, absmax bytes); KeyError names a missing tensor."""
        t = module_names(stem)
        state = json.loads(self.blob(t["state"]).decode())
        return state, self.blob(t["hole"]), self.blob(t["plug"]), self.blob(t["absmax"])

    def dense_names(self) -> List[str]:
        """Tensors carried over unchanged (not part of a module, not the cell table)."""
        owned = {CELLS_TENSOR}
        for stem in self.stems():
            owned.update(module_names(stem).values())
        return [t for t in self.where if t not in owned]


# ------------------------------------------------------------ device execution
class Ticket:
    """Device work in flight: pinned host outputs, readable after `done` fires."""

    def __init__(self, outputs: Dict[str, object], done):
        self.outputs, self.done = outputs, done

    def result(self) -> Dict[str, bytes]:
        self.done.synchronize()
        return {k: v.numpy().tobytes() for k, v in self.outputs.items()}


class DeviceCodec:
    """Encode and expand jobs on the GPU through the C ABI: host bytes are staged in pinned
    memory and moved on a copy stream, the kernels run on a compute stream that waits for
    the copy, and the outputs come back to pinned memory on the compute stream."""

    def __init__(self):
        try:
            import torch
        except ImportError as exc:  # pragma: no cover - torch is part of the image
            raise RuntimeError("the pin tools use torch for device memory and streams") from exc
        if not torch.cuda.is_available():
            raise RuntimeError("the pin tools encode and expand on the GPU, and no GPU is visible")
        from . import glint_hip
        glint_hip.encode_lib()  # RuntimeError if libglint_encode.so is missing
        self.torch, self.kern = torch, glint_hip
        self.copy_stream, self.work_stream = torch.cuda.Stream(), torch.cuda.Stream()

    def _upload(self, data):
        torch = self.torch
        host = np.frombuffer(data, dtype=np.uint8)
        staging = torch.empty(host.size, dtype=torch.uint8, pin_memory=True)
        staging.numpy()[:] = host
        with torch.cuda.stream(self.copy_stream):
            on_device = staging.to("cuda", non_blocking=True)
        self.work_stream.wait_stream(self.copy_stream)
        on_device.record_stream(self.work_stream)
        return on_device

    def _download(self, t):
        host = self.torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        host.copy_(t, non_blocking=True)
        return host

    def _finish(self, outs) -> Ticket:
        staged = {k: self._download(v) for k, v in outs.items()}
        done = self.torch.cuda.Event()
        done.record(self.work_stream)
        return Ticket(staged, done)

    def encode(self, dtype: str, data, n: int, blocksize: int) -> Ticket:
        """Outputs: hole, plug, absmax (f32) and rmse (f64, of the device expand against the source)."""
        torch, k = self.torch, self.kern
        raw = self._upload(data)
        with torch.cuda.stream(self.work_stream):
            if dtype == "BF16":
                bits = raw.view(torch.int16)[:n]
                hole, plug, am = k.encode_bf16(bits, blocksize, stream=self.work_stream)
                src = bits.view(torch.bfloat16).float()
            else:
                src = raw.view(torch.float16)[:n].float() if dtype == "F16" else raw.view(torch.float32)[:n]
                hole, plug, am = k.encode_f32(src, blocksize, stream=self.work_stream)
            if n:
                back = k.expand_f32(hole, plug, am, n, blocksize, stream=self.work_stream)
                err = (src.double() - back.double()).square().mean().sqrt().reshape(1)
            else:
                err = torch.zeros(1, dtype=torch.float64, device="cuda")
            return self._finish({"hole": hole, "plug": plug, "absmax": am, "rmse": err})

    def expand(self, hole: bytes, plug: bytes, absmax: bytes, n: int, blocksize: int, dtype: str) -> Ticket:
        """Output: out, the n weights as dtype (BF16 bits with the reference's rounding)."""
        torch, k = self.torch, self.kern
        dh, dp, da = self._upload(hole), self._upload(plug), self._upload(absmax)
        with torch.cuda.stream(self.work_stream):
            am = da.view(torch.float32)
            if dtype == "BF16":
                out = k.expand_bf16(dh, dp, am, n, blocksize, stream=self.work_stream).view(torch.int16)
            else:
                out = k.expand_f32(dh, dp, am, n, blocksize, stream=self.work_stream)
                out = out.half() if dtype == "F16" else out
            return self._finish({"out": out})


def lookahead(work: Iterable[Tuple[object, Optional[Callable[[], Ticket]]]], depth: int = 1):
    """Yield (key, result) in input order, starting up to `depth` jobs before waiting on
    the oldest; a None job passes its key through with a None result."""
    queue: deque = deque()
    for key, start in work:
        queue.append((key, start() if start else None))
        if len(queue) > depth:
            k, t = queue.popleft()
            yield k, t.result() if t else None
    while queue:
        k, t = queue.popleft()
        yield k, t.result() if t else None


# -------------------------------------------------------------------- convert
@dataclass
class ShardPlan:
    source: Path
    out_name: str
    tensors: List[str] = field(default_factory=list)


def _state_json(blocksize: int, shape, dtype: str) -> bytes:
    return json.dumps({"quant_type": "glint", "blocksize": blocksize, "shape": [int(d) for d in shape],
                       "src_dtype": dtype}, separators=(",", ":")).encode()


def _copy_sidecars(src_dir: Path, out: Path, names: Iterable[str]) -> List[str]:
    copied = []
    for fname in names:
        f = src_dir / fname
        if f.is_file() and f.resolve() != (out / fname).resolve():
            shutil.copyfile(f, out / fname)
            copied.append(fname)
    return copied


def _stats(values: List[float]) -> Tuple[Optional[float], Optional[float]]:
    return (sum(values) / len(values), max(values)) if values else (None, None)


def convert(src: Path, out: Path, blocksize: int = 64, dry_run: bool = False, allow_cpu: bool = False,
            force_python: bool = False) -> dict:
    """Dense BF16/F16/F32 linears of a model -> a GLINT pin, encoded on the GPU.
    allow_cpu and force_python keep the reference's signature: there is no host encoder
    here, so allow_cpu has no effect and force_python raises NotImplementedError."""
    if blocksize < 1:
        raise ValueError(f"blocksize {blocksize} is not positive")
    if force_python:
        raise NotImplementedError("no pure-Python encoder in this build: GLINT pins are encoded on the GPU")
    source = ModelSource(src)
    out = Path(out).expanduser().resolve()
    plans: List[ShardPlan] = []
    linears: List[str] = []
    n_dense = 0
    for f in source.files:
        plan = ShardPlan(f, f.name if source.sharded else SINGLE_SHARD)
        with TensorFile(f) as tf:
            for name, e in tf.entries.items():
                plan.tensors.append(name)
                if is_linear(name, e.dtype, e.shape):
                    linears.append(name)
                else:
                    n_dense += 1
        plans.append(plan)
    try:
        codec, why = DeviceCodec(), None
    except RuntimeError as exc:
        codec, why = None, str(exc)
    if dry_run:
        return {"schema": PIN_SCHEMA, "n_linears": len(linears), "n_keep": n_dense, "blocksize": blocksize,
                "shards": [f.name for f in source.files], "linears": linears, "cuda": codec is not None,
                "device": "hip", "numpy": True}
    if codec is None:
        raise RuntimeError(f"convert encodes on the GPU (libglint_encode.so): {why}")
    to_encode = set(linears)
    out.mkdir(parents=True, exist_ok=True)
    modules, weight_map, total = [], {}, 0
    for shard_no, plan in enumerate(plans):
        items = []
        with TensorFile(plan.source) as tf:
            def work():
                for name in plan.tensors:
                    e = tf.entries[name]
                    if name in to_encode:
                        yield name, (lambda e=e, name=name: codec.encode(e.dtype, tf.buffer(name), e.count, blocksize))
                    else:
                        yield name, None
            for name, res in lookahead(work()):
                e = tf.entries[name]
                if res is None:
                    items.append((name, e.dtype, e.shape, tf.blob(name)))
                    continue
                stem = name[:-len(".weight")]
                t = module_names(stem)
                state = _state_json(blocksize, e.shape, e.dtype)
                items += [(t["hole"], "U8", (len(res["hole"]), 1), res["hole"]),
                          (t["plug"], "U8", (len(res["plug"]), 1), res["plug"]),
                          (t["absmax"], "F32", (len(res["absmax"]) // 4,), res["absmax"]),
                          (t["state"], "U8", (len(state),), state)]
                modules.append({"src": stem, "rmse": float(np.frombuffer(res["rmse"], np.float64)[0]),
                                "shape": [int(d) for d in e.shape],
                                "backend": "hip_bf16" if e.dtype == "BF16" else "hip_f32", "shard": plan.out_name})
        if shard_no == 0:
            items.append((CELLS_TENSOR, "F32", (16, 16), codebook.cells_f32_bytes()))
        total += save(out / plan.out_name, items, meta={"format": "pt", "quantization": "glint"})
        weight_map.update(dict.fromkeys((it[0] for it in items), plan.out_name))
        del items
    if source.sharded:
        (out / INDEX_NAME).write_text(json.dumps({"metadata": {"total_size": total, "quantization": "glint"},
                                                  "weight_map": weight_map}, indent=2) + "\n")
    sidecars = _copy_sidecars(source.dir, out, SIDECAR)
    mean, worst = _stats([m["rmse"] for m in modules if m["rmse"] is not None])
    kinds = sorted({m["backend"] for m in modules})
    pin = {"schema": PIN_SCHEMA, "src": str(source.dir if source.sharded else source.files[0]), "dest": "glint",
           "n_converted": len(modules), "blocksize": blocksize, "rmse_mean": mean, "rmse_max": worst,
           "backend": kinds[0] if len(kinds) == 1 else ("mixed" if kinds else None), "backends": kinds,
           "shards": [f.name for f in source.files] if source.sharded else [SINGLE_SHARD], "sidecar": sidecars,
           "note": "hole = parent (NF4) cell, plug = child index; weight = GLINT_CELLS[hole][plug] * absmax"}
    (out / "pin.json").write_text(json.dumps(pin, indent=2) + "\n")
    (out / "CONVERT_REPORT.json").write_text(json.dumps({"pin": pin, "modules": modules}, indent=2) + "\n")
    return {"pin": pin, "modules": modules}


# --------------------------------------------------------------------- verify
def _first_mismatch(a: bytes, b: bytes) -> Optional[int]:
    """Offset of the first differing byte (the shorter length if only lengths differ)."""
    if a == b:
        return None
    if len(a) != len(b):
        return min(len(a), len(b))
    return int(np.argmax(np.frombuffer(a, np.uint8) != np.frombuffer(b, np.uint8)))


def _pin_level_failures(pin: Pin, cells: Optional[List[float]], n_modules: int) -> List[str]:
    found = []
    if pin.meta.get("schema") != PIN_SCHEMA:
        found.append(f"schema={pin.meta.get('schema')!r}")
    if cells is None:
        found.append(f"{CELLS_TENSOR} missing")
    elif cells != table_values():
        found.append(f"{CELLS_TENSOR} is not the GLINT cell table")
    declared = pin.meta.get("n_converted")
    if declared is not None and declared != n_modules:
        found.append(f"pin.json n_converted={declared}, the pin holds {n_modules} modules")
    return found


def _layout_problems(n: int, bs: int, hole: bytes, plug: bytes, absmax: bytes) -> List[str]:
    planes, scales = (n + 1) // 2, -(-n // bs)
    found = []
    if (len(hole), len(plug)) != (planes, planes):
        found.append(f"planes hold {len(hole)}/{len(plug)} bytes, {planes} expected")
    if len(absmax) != 4 * scales:
        found.append(f"{len(absmax) // 4} absmax values, {scales} expected")
    if n % 2 and planes and (hole[-1] >> 4 or plug[-1] >> 4):
        found.append("the pad nibble of an odd-length module is not zero")
    return found


def _parity(w: np.ndarray, bs: int, hole: bytes, plug: bytes, absmax: bytes) -> dict:
    h2, p2, am2 = hc.encode_f32(w, bs)
    out = {"hole_first_diff": _first_mismatch(hole, h2), "plug_first_diff": _first_mismatch(plug, p2),
           "absmax_first_diff": _first_mismatch(absmax, am2.astype("<f4").tobytes())}
    for key, mine, host in (("hole_bytes_differ", hole, h2), ("plug_bytes_differ", plug, p2)):
        a, b = np.frombuffer(mine, np.uint8), np.frombuffer(host, np.uint8)
        common = min(a.size, b.size)  # bytes past the shorter plane count as differing
        out[key] = int(np.count_nonzero(a[:common] != b[:common])) + abs(a.size - b.size)
    return out


def verify(pin_dir: Path, src: Optional[Path] = None, parity: bool = False, cuda: bool = False) -> dict:
    """Check a pin: its schema and cell table, each module's layout; with src, each
    module's RMSE against the source weights; the --cuda gate (device expand against the
    host expand, max |diff| < 1e-5) and the --parity gate (the pin's bytes against a host
    re-encode of the source). The report's "ok" is False on any failure."""
    if parity and src is None:
        raise ValueError("the parity gate re-encodes the source: pass src")
    codec = DeviceCodec() if cuda else None
    rows: List[dict] = []
    with Pin(pin_dir) as pin:
        cells = pin.table()
        stems = pin.stems()
        failures = _pin_level_failures(pin, cells, len(stems))
        source = ModelSource(src).lookup() if src is not None else {}
        try:
            for stem in stems:
                rows.append(_check_module(pin, stem, cells, source, codec, parity))
        finally:
            close_all(source.values())
        backend = pin.meta.get("backend")
    rated = [r["rmse"] for r in rows if "rmse" in r]
    mean, worst = _stats(rated)
    bad = [r["module"] for r in rows if not r["ok"]]
    return {"schema": VERIFY_SCHEMA, "pin": str(Path(pin_dir).expanduser().resolve()), "backend": backend,
            "n_modules": len(rows), "n_failed": len(bad), "rmse_mean": mean, "rmse_max": worst,
            "parity_checked": parity, "cuda_expand_checked": cuda, "ok": not failures and not bad,
            "failures": failures + [f"module {m}" for m in bad], "modules": rows}


def _check_module(pin: Pin, stem: str, cells, source: Dict[str, TensorFile], codec: Optional[DeviceCodec],
                  parity: bool) -> dict:
    row: dict = {"module": stem}
    problems: List[str] = []
    try:
        state, hole, plug, absmax = pin.module(stem)
    except KeyError as exc:
        return {"module": stem, "ok": False, "problems": [f"tensor {exc} is missing"]}
    n, bs = element_count(state["shape"]), int(state["blocksize"])
    problems += _layout_problems(n, bs, hole, plug, absmax)
    scales = np.frombuffer(absmax, dtype="<f4")
    if not problems and codec is not None:
        host = hc.expand(hole, plug, scales, n, bs, cells)
        device = np.frombuffer(codec.expand(hole, plug, absmax, n, bs, "F32").result()["out"], dtype="<f4")
        gap = float(np.abs(device - host).max()) if n else 0.0
        row["cuda_expand_max_abs"] = gap
        if not gap < EXPAND_GATE:
            problems.append(f"device expand differs from the host expand by {gap:.3g} (gate {EXPAND_GATE})")
    if not problems and source:
        name = module_names(stem)["hole"]
        tf = source.get(name)
        if tf is None:
            problems.append("the source has no such tensor")
        elif list(tf.entries[name].shape) != list(state["shape"]):
            problems.append(f"source shape {list(tf.entries[name].shape)}, pin shape {state['shape']}")
        else:
            w = hc.to_f32(tf.entries[name].dtype, tf.buffer(name), n)
            rec = hc.expand(hole, plug, scales, n, bs, cells)
            row["rmse"] = hc.rms_error(w, rec)
            scale = hc.rms_error(w, np.zeros_like(w))
            row["rel_rmse"] = row["rmse"] / scale if scale else 0.0
            if not np.isfinite(rec[np.isfinite(w)]).all():
                problems.append("finite source weights reconstruct to non-finite values")
            if parity:
                row["parity"] = _parity(w, bs, hole, plug, absmax)
                if any(v is not None for k, v in row["parity"].items() if k.endswith("_first_diff")):
                    problems.append("the pin's bytes differ from a host re-encode of the source")
    row["ok"] = not problems
    if problems:
        row["problems"] = problems
    return row


# ---------------------------------------------------------------------- unpin
def unpin(pin_dir: Path, out: Path, dtype: str = "BF16") -> dict:
    """A pin -> dense safetensors under the original tensor names and shapes (the GLINT
    reconstruction, expanded on the GPU), plus the pin's sidecar files."""
    if dtype not in DENSE_DTYPES:
        raise ValueError(f"unpin writes one of {', '.join(DENSE_DTYPES)}, not {dtype}")
    out = Path(out).expanduser().resolve()
    with Pin(pin_dir) as pin:
        if pin.meta.get("schema") != PIN_SCHEMA:
            raise ValueError(f"{pin.root} holds schema {pin.meta.get('schema')!r}, not {PIN_SCHEMA}")
        cells = pin.table()
        if cells is not None and cells != table_values():
            raise ValueError(f"{pin.root}: its {CELLS_TENSOR} is not the table the device kernels expand with")
        codec = DeviceCodec()
        out.mkdir(parents=True, exist_ok=True)
        hole_of = {module_names(s)["hole"]: s for s in pin.stems()}
        carried = set(pin.dense_names())

        def work():
            for name in pin.where:
                if name in hole_of:
                    state, hole, plug, absmax = pin.module(hole_of[name])
                    n, bs = element_count(state["shape"]), int(state["blocksize"])
                    yield (name, state), (lambda h=hole, p=plug, a=absmax, n=n, bs=bs: codec.expand(h, p, a, n, bs,
                                                                                                     dtype))
                elif name in carried:
                    yield (name, None), None

        shards: Dict[str, list] = {s: [] for s in pin.shards}
        expanded = 0
        for (name, state), res in lookahead(work()):
            if res is None:
                e = pin.entry(name)
                shards[pin.where[name]].append((name, e.dtype, e.shape, pin.blob(name)))
            else:
                shards[pin.where[name]].append((name, dtype, tuple(state["shape"]), res["out"]))
                expanded += 1
        weight_map, total = {}, 0
        for shard, items in shards.items():
            total += save(out / shard, items, meta={"format": "pt", "unpinned_from": "glint"})
            weight_map.update(dict.fromkeys((it[0] for it in items), shard))
        if len(shards) > 1:
            (out / INDEX_NAME).write_text(json.dumps({"metadata": {"total_size": total}, "weight_map": weight_map},
                                                     indent=2) + "\n")
        _copy_sidecars(pin.root, out, pin.meta.get("sidecar", []))
    return {"out": str(out), "dtype": dtype, "n_expanded": expanded, "shards": list(shards)}


# ------------------------------------------------------------------------ CLI
def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="GLINT pin tools on the GPU")
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("convert", help="dense BF16/F16/F32 linears -> hole + plug pin")
    c.add_argument("--src", required=True, help=".safetensors file, model dir or sharded model dir")
    c.add_argument("--out", required=True)
    c.add_argument("--blocksize", type=int, default=64)
    c.add_argument("--dry-run", action="store_true")
    c.add_argument("--allow-cpu", action="store_true", help="accepted; this build has no host encoder")
    v = sub.add_parser("verify", help="check a pin; exit status 1 if any check fails")
    v.add_argument("--pin", required=True)
    v.add_argument("--src", help="source model, for per-module RMSE")
    v.add_argument("--parity", action="store_true", help="compare the pin's bytes with a host re-encode of --src")
    v.add_argument("--cuda", action="store_true", help="compare the device expand with the host expand (< 1e-5)")
    v.add_argument("--out", help="write the full report here")
    v.add_argument("--quiet", action="store_true", help="leave the per-module rows out of stdout")
    u = sub.add_parser("unpin", help="pin -> dense safetensors")
    u.add_argument("--pin", required=True)
    u.add_argument("--out", required=True)
    u.add_argument("--dtype", default="BF16", choices=DENSE_DTYPES)
    a = ap.parse_args(argv)
    if a.cmd == "convert":
        res = convert(Path(a.src), Path(a.out), a.blocksize, a.dry_run, a.allow_cpu)
        print(json.dumps(res if a.dry_run else res["pin"], indent=2))
        return 0
    if a.cmd == "verify":
        rep = verify(Path(a.pin), Path(a.src) if a.src else None, a.parity, a.cuda)
        if a.out:
            Path(a.out).write_text(json.dumps(rep, indent=2) + "\n")
        shown = {k: v for k, v in rep.items() if k != "modules"} if a.quiet else rep
        print(json.dumps(shown, indent=2))
        return 0 if rep["ok"] else 1
    print(json.dumps(unpin(Path(a.pin), Path(a.out), a.dtype), indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
