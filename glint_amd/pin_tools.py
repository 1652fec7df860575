"""GLINT pin tools on the MI355X device path: convert, verify and unpin.

    python -m glint_amd.pin_tools convert --src MODEL --out PIN [--blocksize 64] [--dry-run]
    python -m glint_amd.pin_tools verify  --pin PIN [--src MODEL] [--parity] [--cuda] [--out F] [--quiet]
    python -m glint_amd.pin_tools unpin   --pin PIN --out DIR [--dtype BF16|F16|F32]

The pin format, the file set (shards, index, sidecar files, pin.json,
CONVERT_REPORT.json) and the verify evidence follow the reference's tools
(glint_pin.py:23-193, glint_verify.py:29-144, glint_unpin.py:24-85,
glint_pinfile.py:8-61), so a pin made here reads in the reference's tools and back.

What runs where:
- convert reads each shard through a memory map. For every dense 2-D ".weight" it
  stages the bytes in pinned host memory, copies them on a copy stream and encodes on a
  compute stream: BF16 straight from its bits, F16 widened to f32 on the device, F32
  as is. It then expands the pin on the device for the module's RMSE and copies the
  planes back. Staging of tensor i + 1 on the host overlaps the device work of tensor i.
- unpin expands on the device (BF16 with the reference's rounding and NaN rule, F32, or
  F16 from the f32 expand), with the same overlap.
- verify checks layout on the host. Its gates compare against the host codec
  (glint_amd.host_codec): --cuda is the device expand vs the host expand at
  max_abs < 1e-5; --parity is the pin's bytes vs a host re-encode of the source.
There is no host encode or expand path: without the HIP library and a GPU, convert and
unpin raise RuntimeError (dry runs and the layout checks still work).
"""
from __future__ import annotations

import argparse
import json
import shutil
import sys
from pathlib import Path
from typing import Dict, Iterator, List, Optional, Tuple

import numpy as np

from . import codebook
from . import host_codec as HC
from .safetensors_io import SafeTensorsFile, write_safetensors

PARENT_KEEP = ("norm", "bias", "rotary", "cos_cached", "sin_cached")
INDEX_NAME = "model.safetensors.index.json"
STATE_SUFFIX = ".weight.glint_state"
SIDECAR = ("config.json", "generation_config.json", "tokenizer.json", "tokenizer_config.json",
           "special_tokens_map.json", "tokenizer.model", "vocab.json", "merges.txt", "added_tokens.json",
           "chat_template.jinja")
CUDA_EXPAND_TOL = 1e-5  # glint_verify.py:29
DENSE = ("BF16", "F16", "F32")


def numel_of(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def _is_keep(name: str) -> bool:
    low = name.lower()
    return any(k in low for k in PARENT_KEEP) or name.endswith(".bias")


def resolve_shards(src: Path) -> List[Path]:
    """A file, or a dir with model.safetensors, an index, or exactly one .safetensors
    (glint_pin.py:41-60)."""
    src = Path(src).expanduser().resolve()
    if not src.is_dir():
        return [src]
    if (src / "model.safetensors").is_file():
        return [src / "model.safetensors"]
    index = src / INDEX_NAME
    if index.is_file():
        names = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        missing = [n for n in names if not (src / n).is_file()]
        if missing:
            raise FileNotFoundError(f"{INDEX_NAME} names missing shards: {missing}")
        return [src / n for n in names]
    shards = sorted(src.glob("*.safetensors"))
    if len(shards) != 1:
        raise FileNotFoundError(f"need model.safetensors, {INDEX_NAME}, or exactly one .safetensors in {src}")
    return shards


class Pin:
    """A pin dir, every shard open, tensors looked up by name (glint_pinfile.py:10-61)."""

    def __init__(self, root: Path):
        self.root = Path(root).expanduser().resolve()
        pj = self.root / "pin.json"
        if not pj.is_file():
            raise FileNotFoundError(f"no pin.json in {self.root}")
        self.meta = json.loads(pj.read_text())
        index = self.root / INDEX_NAME
        names = (sorted(set(json.loads(index.read_text())["weight_map"].values())) if index.is_file()
                 else ["model.safetensors"])
        self.shards: Dict[str, SafeTensorsFile] = {n: SafeTensorsFile(self.root / n) for n in names}
        self.where: Dict[str, str] = {t: s for s, st in self.shards.items() for t in st.tensors}

    def close(self) -> None:
        for st in self.shards.values():
            st.close()

    def __enter__(self) -> "Pin":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def info(self, name: str):
        return self.shards[self.where[name]].tensors[name]

    def read(self, name: str) -> bytes:
        return self.shards[self.where[name]].read_bytes(name)

    def stems(self) -> List[str]:
        return [n[: -len(STATE_SUFFIX)] for n in self.where if n.endswith(STATE_SUFFIX)]

    def state(self, stem: str) -> dict:
        return json.loads(self.read(stem + STATE_SUFFIX).decode())

    def cells(self) -> Optional[List[float]]:
        if "_glint_cells" not in self.where:
            return None
        return np.frombuffer(self.read("_glint_cells"), dtype="<f4").tolist()

    def module(self, stem: str) -> Tuple[dict, bytes, bytes, bytes]:
        w = stem + ".weight"
        return self.state(stem), self.read(w), self.read(w + ".glint_plug"), self.read(w + ".absmax")

    @staticmethod
    def module_names(stem: str) -> Tuple[str, ...]:
        w = stem + ".weight"
        return (w, w + ".glint_plug", w + ".absmax", w + ".glint_state")


# ------------------------------------------------------------------ device pipeline
class _Device:
    """Copy stream + compute stream; a job's outputs land in pinned host buffers and are
    read once its completion event has fired."""

    def __init__(self):
        try:
            import torch
        except ImportError as e:  # pragma: no cover - torch is part of the image
            raise RuntimeError("the pin tools need torch for device memory and streams") from e
        if not torch.cuda.is_available():
            raise RuntimeError("GLINT encode/expand run on the GPU: no GPU is visible (this build has no host path)")
        from . import glint_hip
        glint_hip.encode_lib()  # raises if libglint_encode.so is missing
        self.torch, self.H = torch, glint_hip
        self.copy_s = torch.cuda.Stream()
        self.comp_s = torch.cuda.Stream()

    def _to_device(self, raw) -> "object":
        """Host bytes -> pinned staging -> device (uint8), ordered before the compute stream."""
        torch = self.torch
        src = np.frombuffer(raw, dtype=np.uint8)
        pinned = torch.empty(src.size, dtype=torch.uint8, pin_memory=True)
        pinned.numpy()[:] = src  # host copy (pages the memory map in)
        with torch.cuda.stream(self.copy_s):
            dev = pinned.to("cuda", non_blocking=True)
        self.comp_s.wait_stream(self.copy_s)
        dev.record_stream(self.comp_s)
        return dev

    def _to_host(self, t):
        host = self.torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        host.copy_(t, non_blocking=True)
        return host

    def encode_job(self, dtype: str, raw, n: int, bs: int) -> dict:
        torch, H = self.torch, self.H
        dev = self._to_device(raw)
        with torch.cuda.stream(self.comp_s):
            if dtype == "BF16":
                src16 = dev.view(torch.int16)[:n]
                hole, plug, am = H.encode_bf16(src16, bs, stream=self.comp_s)
                w32 = src16.view(torch.bfloat16).float()
            else:
                w32 = (dev.view(torch.float16)[:n].float() if dtype == "F16" else dev.view(torch.float32)[:n])
                hole, plug, am = H.encode_f32(w32, bs, stream=self.comp_s)
            if n:
                rec = H.expand_f32(hole, plug, am, n, bs, stream=self.comp_s)
                d = w32.double() - rec.double()
                err = torch.sqrt(torch.mean(d * d)).reshape(1)
            else:
                err = torch.zeros(1, dtype=torch.float64, device="cuda")
            job = {"hole": self._to_host(hole), "plug": self._to_host(plug), "am": self._to_host(am),
                   "rmse": self._to_host(err), "event": torch.cuda.Event()}
            job["event"].record(self.comp_s)
        return job

    def expand_job(self, hole: bytes, plug: bytes, am: bytes, n: int, bs: int, dtype: str) -> dict:
        torch, H = self.torch, self.H
        dh, dp, da = self._to_device(hole), self._to_device(plug), self._to_device(am)
        with torch.cuda.stream(self.comp_s):
            amf = da.view(torch.float32)
            if dtype == "BF16":
                out = H.expand_bf16(dh, dp, amf, n, bs, stream=self.comp_s).view(torch.int16)
            else:
                out = H.expand_f32(dh, dp, amf, n, bs, stream=self.comp_s)
                if dtype == "F16":
                    out = out.half()
            job = {"out": self._to_host(out), "event": torch.cuda.Event()}
            job["event"].record(self.comp_s)
        return job

    @staticmethod
    def finish(job: dict) -> dict:
        job["event"].synchronize()
        return {k: (v.numpy().tobytes() if k != "event" else None) for k, v in job.items()}


def _pipelined(dev_jobs: Iterator[Tuple[object, Optional[callable]]]):
    """Run (key, make_job) pairs one deep: job i + 1 is staged and enqueued before job i is
    waited on. make_job None passes the key through untouched, in order."""
    pending = []
    for key, make in dev_jobs:
        pending.append((key, make() if make is not None else None))
        while len(pending) > 1:
            k, j = pending.pop(0)
            yield k, (_Device.finish(j) if j is not None else None)
    for k, j in pending:
        yield k, (_Device.finish(j) if j is not None else None)


def _device_or_none():
    try:
        return _Device(), None
    except RuntimeError as e:
        return None, str(e)


# ------------------------------------------------------------------------ convert
def _state_bytes(bs: int, shape, dtype: str) -> bytes:
    return json.dumps({"quant_type": "glint", "blocksize": bs, "shape": list(shape), "src_dtype": dtype},
                      separators=(",", ":")).encode()


def convert(src: Path, out: Path, blocksize: int = 64, dry_run: bool = False, allow_cpu: bool = False,
            force_python: bool = False) -> dict:
    """BF16/F16/F32 dense linears -> GLINT pin (glint_pin.py:87-193), encoded on the GPU.
    allow_cpu and force_python exist for call compatibility: this build has no host
    encoder, so force_python raises and allow_cpu changes nothing."""
    if blocksize <= 0:
        raise ValueError("blocksize must be positive")
    if force_python:
        raise NotImplementedError("this build encodes on the GPU only (no pure-Python encoder)")
    shards = resolve_shards(src)
    out = Path(out).expanduser().resolve()
    sharded = len(shards) > 1
    linears: List[str] = []
    keep: List[str] = []
    for wf in shards:
        with SafeTensorsFile(wf) as st:
            for name, info in st.tensors.items():
                dense = info.dtype in DENSE and len(info.shape) == 2
                (linears if dense and name.endswith(".weight") and not _is_keep(name) else keep).append(name)
    dev, why = _device_or_none()
    if dry_run:
        return {"schema": "glint_pin_v1", "n_linears": len(linears), "n_keep": len(keep), "blocksize": blocksize,
                "shards": [s.name for s in shards], "linears": linears, "hip": dev is not None, "numpy": True}
    if dev is None:
        raise RuntimeError(f"GLINT encode runs on the GPU (libglint_encode.so): {why}")
    out.mkdir(parents=True, exist_ok=True)
    linear_set = set(linears)
    reports, weight_map, total = [], {}, 0
    for si, wf in enumerate(shards):
        out_name = wf.name if sharded else "model.safetensors"
        tensors = []
        with SafeTensorsFile(wf) as st:
            def jobs():
                for name, info in st.tensors.items():
                    if name not in linear_set:
                        yield (name, info), None
                    else:
                        n = numel_of(info.shape)
                        yield (name, info), (lambda i=info, nm=name, nn=n: dev.encode_job(i.dtype, st.view(nm), nn,
                                                                                         blocksize))
            for (name, info), res in _pipelined(jobs()):
                if res is None:
                    tensors.append((name, info.dtype, info.shape, st.read_bytes(name)))
                    continue
                stem = name[: -len(".weight")]
                hole, plug, am = res["hole"], res["plug"], res["am"]
                state = _state_bytes(blocksize, info.shape, info.dtype)
                tensors += [(stem + ".weight", "U8", (len(hole), 1), hole),
                            (stem + ".weight.glint_plug", "U8", (len(plug), 1), plug),
                            (stem + ".weight.absmax", "F32", (len(am) // 4,), am),
                            (stem + STATE_SUFFIX, "U8", (len(state),), state)]
                backend = "hip_bf16" if info.dtype == "BF16" else "hip_f32"
                err = float(np.frombuffer(res["rmse"], dtype=np.float64)[0])
                reports.append({"src": stem, "rmse": err, "shape": list(info.shape), "backend": backend,
                                "shard": out_name})
        if si == 0:
            tensors.append(("_glint_cells", "F32", (16, 16), codebook.cells_f32_bytes()))
        for t in tensors:
            weight_map[t[0]] = out_name
            total += len(t[3])
        write_safetensors(out / out_name, tensors, metadata={"format": "pt", "quantization": "glint"})
        del tensors
    if sharded:
        index = {"metadata": {"total_size": total, "quantization": "glint"}, "weight_map": weight_map}
        (out / INDEX_NAME).write_text(json.dumps(index, indent=2) + "\n")
    src_dir = shards[0].parent
    copied = []
    for side in SIDECAR:
        p = src_dir / side
        if p.is_file() and p.resolve() != (out / side).resolve():
            shutil.copyfile(p, out / side)
            copied.append(side)
    rated = [r["rmse"] for r in reports if r["rmse"] is not None]
    backends = sorted({r["backend"] for r in reports})
    pin = {"schema": "glint_pin_v1", "src": str(shards[0] if not sharded else src_dir), "dest": "glint",
           "n_converted": len(reports), "blocksize": blocksize,
           "rmse_mean": (sum(rated) / len(rated)) if rated else None, "rmse_max": max(rated) if rated else None,
           "backend": backends[0] if len(backends) == 1 else ("mixed" if backends else None), "backends": backends,
           "shards": [s.name for s in shards] if sharded else ["model.safetensors"], "sidecar": copied,
           "note": "hole = parent (NF4) cell, plug = child index; weight = GLINT_CELLS[hole][plug] * absmax"}
    (out / "pin.json").write_text(json.dumps(pin, indent=2) + "\n")
    (out / "CONVERT_REPORT.json").write_text(json.dumps({"pin": pin, "modules": reports}, indent=2) + "\n")
    return {"pin": pin, "modules": reports}


# ------------------------------------------------------------------------- verify
def _first_diff(a: bytes, b: bytes) -> Optional[int]:
    if len(a) != len(b):
        return min(len(a), len(b))
    if a == b:
        return None
    return int(np.flatnonzero(np.frombuffer(a, np.uint8) != np.frombuffer(b, np.uint8))[0])


def verify(pin_dir: Path, src: Optional[Path] = None, parity: bool = False, cuda: bool = False) -> dict:
    """Layout of every module, optional RMSE against the source, and the two gates
    (glint_verify.py:48-144). Exit status of the CLI: 1 on any failure."""
    if parity and src is None:
        raise ValueError("--parity needs --src")
    dev = _Device() if cuda else None
    fails, modules = [], []
    with Pin(pin_dir) as pin:
        if pin.meta.get("schema") != "glint_pin_v1":
            fails.append(f"schema={pin.meta.get('schema')!r}")
        cells = pin.cells()
        if cells is None:
            fails.append("_glint_cells missing")
        elif cells != np.frombuffer(codebook.cells_f32_bytes(), dtype="<f4").tolist():
            fails.append("_glint_cells differs from the GLINT table")
        src_ix: Dict[str, SafeTensorsFile] = {}
        if src is not None:
            for wf in resolve_shards(src):
                st = SafeTensorsFile(wf)
                for name in st.tensors:
                    src_ix[name] = st
        stems = pin.stems()
        if pin.meta.get("n_converted") not in (None, len(stems)):
            fails.append(f"pin.json n_converted={pin.meta.get('n_converted')} but {len(stems)} modules")
        for stem in stems:
            row = {"module": stem, "ok": True, "problems": []}
            try:
                state, hole, plug, am = pin.module(stem)
            except KeyError as e:
                row["problems"].append(f"missing tensor {e}")
                row["ok"] = False
                modules.append(row)
                continue
            n = numel_of(tuple(state["shape"]))
            bs = int(state["blocksize"])
            npk, nam = (n + 1) // 2, (n + bs - 1) // bs
            if len(hole) != npk or len(plug) != npk:
                row["problems"].append(f"hole/plug bytes {len(hole)}/{len(plug)} != {npk}")
            if len(am) != 4 * nam:
                row["problems"].append(f"absmax {len(am) // 4} floats != {nam}")
            if n & 1 and npk and ((hole[-1] >> 4) or (plug[-1] >> 4)):
                row["problems"].append("odd n but pad nibble is not zero")
            amf = np.frombuffer(am, dtype="<f4") if len(am) == 4 * nam else None
            if not row["problems"] and cuda:
                host = HC.expand(hole, plug, amf, n, bs, cells)
                got = np.frombuffer(_Device.finish(dev.expand_job(hole, plug, am, n, bs, "F32"))["out"], dtype="<f4")
                row["cuda_expand_max_abs"] = float(np.max(np.abs(got - host))) if n else 0.0
                if not row["cuda_expand_max_abs"] < CUDA_EXPAND_TOL:
                    row["problems"].append(f"cuda expand max_abs {row['cuda_expand_max_abs']:.3g} >= {CUDA_EXPAND_TOL}")
            if not row["problems"] and src is not None:
                name = stem + ".weight"
                st = src_ix.get(name)
                if st is None:
                    row["problems"].append("not in --src")
                else:
                    info = st.tensors[name]
                    if list(info.shape) != list(state["shape"]):
                        row["problems"].append(f"shape {state['shape']} != src {list(info.shape)}")
                    else:
                        w = HC.dense_to_f32(info.dtype, st.view(name), n)
                        rec = HC.expand(hole, plug, amf, n, bs, cells)
                        row["rmse"] = HC.rmse(w, rec)
                        ref = float(np.sqrt(np.mean(w.astype(np.float64) ** 2))) if n else 0.0
                        row["rel_rmse"] = row["rmse"] / ref if ref else 0.0
                        if not np.all(np.isfinite(rec[np.isfinite(w)])):
                            row["problems"].append("non-finite reconstruction of finite weights")
                        if parity:
                            h2, p2, am2 = HC.encode_f32(w, bs)
                            par = {"hole_first_diff": _first_diff(hole, h2), "plug_first_diff": _first_diff(plug, p2),
                                   "absmax_first_diff": _first_diff(am, am2.astype("<f4").tobytes())}
                            hb, pb = np.frombuffer(hole, np.uint8), np.frombuffer(plug, np.uint8)
                            par["hole_bytes_differ"] = int(np.count_nonzero(hb != np.frombuffer(h2, np.uint8)))
                            par["plug_bytes_differ"] = int(np.count_nonzero(pb != np.frombuffer(p2, np.uint8)))
                            row["parity"] = par
                            if any(v is not None for k, v in par.items() if k.endswith("first_diff")):
                                row["problems"].append("host re-encode bytes differ")
            row["ok"] = not row["problems"]
            if not row["problems"]:
                del row["problems"]
            modules.append(row)
        for st in {id(s): s for s in src_ix.values()}.values():
            st.close()
        backend = pin.meta.get("backend")
    rated = [m["rmse"] for m in modules if "rmse" in m]
    bad = [m["module"] for m in modules if not m["ok"]]
    return {"schema": "glint_verify_v1", "pin": str(Path(pin_dir).expanduser().resolve()), "backend": backend,
            "n_modules": len(modules), "n_failed": len(bad), "rmse_mean": sum(rated) / len(rated) if rated else None,
            "rmse_max": max(rated) if rated else None, "parity_checked": parity, "cuda_expand_checked": cuda,
            "ok": not fails and not bad, "failures": fails + [f"module {b}" for b in bad], "modules": modules}


# -------------------------------------------------------------------------- unpin
def unpin(pin_dir: Path, out: Path, dtype: str = "BF16") -> dict:
    """Pin -> dense safetensors with the original names and shapes (glint_unpin.py:45-85),
    expanded on the GPU with the pin's own table."""
    if dtype not in DENSE:
        raise ValueError(f"dtype must be one of {DENSE}")
    out = Path(out).expanduser().resolve()
    with Pin(pin_dir) as pin:
        if pin.meta.get("schema") != "glint_pin_v1":
            raise ValueError(f"not a glint_pin_v1 pin: {pin.meta.get('schema')}")
        cells = pin.cells()
        if cells is not None and cells != np.frombuffer(codebook.cells_f32_bytes(), dtype="<f4").tolist():
            raise ValueError("the pin's _glint_cells differ from the table the device kernels use")
        dev = _Device()
        out.mkdir(parents=True, exist_ok=True)
        per_shard: Dict[str, list] = {s: [] for s in pin.shards}
        stem_of = {stem + ".weight": stem for stem in pin.stems()}
        owned = set()
        for stem in pin.stems():
            owned.update(pin.module_names(stem))

        def jobs():
            for name, shard in pin.where.items():
                if name in stem_of:
                    state, hole, plug, am = pin.module(stem_of[name])
                    n, bs = numel_of(tuple(state["shape"])), int(state["blocksize"])
                    yield (name, shard, state), (lambda h=hole, p=plug, a=am, nn=n, b=bs:
                                                 dev.expand_job(h, p, a, nn, b, dtype))
                elif name not in owned and name != "_glint_cells":
                    yield (name, shard, None), None

        n_expanded = 0
        for (name, shard, state), res in _pipelined(jobs()):
            if res is not None:
                per_shard[shard].append((name, dtype, tuple(state["shape"]), res["out"]))
                n_expanded += 1
            else:
                info = pin.info(name)
                per_shard[shard].append((name, info.dtype, info.shape, pin.read(name)))
        weight_map, total = {}, 0
        for shard, tensors in per_shard.items():
            write_safetensors(out / shard, tensors, metadata={"format": "pt", "unpinned_from": "glint"})
            for t in tensors:
                weight_map[t[0]] = shard
                total += len(t[3])
        if len(per_shard) > 1:
            (out / INDEX_NAME).write_text(json.dumps({"metadata": {"total_size": total}, "weight_map": weight_map},
                                                     indent=2) + "\n")
        for side in pin.meta.get("sidecar", []):
            p = pin.root / side
            if p.is_file():
                shutil.copyfile(p, out / side)
    return {"out": str(out), "dtype": dtype, "n_expanded": n_expanded, "shards": list(per_shard)}


# ---------------------------------------------------------------------------- CLI
def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="GLINT pin tools (MI355X device path)")
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("convert", help="BF16/F16/F32 -> hole+plug pin")
    c.add_argument("--src", required=True)
    c.add_argument("--out", required=True)
    c.add_argument("--blocksize", type=int, default=64)
    c.add_argument("--dry-run", action="store_true")
    v = sub.add_parser("verify", help="check a pin; exit 1 on any failure")
    v.add_argument("--pin", required=True)
    v.add_argument("--src")
    v.add_argument("--parity", action="store_true", help="pin bytes vs a host re-encode of --src")
    v.add_argument("--cuda", action="store_true", help="device expand vs host expand, max_abs < 1e-5")
    v.add_argument("--out")
    v.add_argument("--quiet", action="store_true")
    u = sub.add_parser("unpin", help="pin -> dense safetensors")
    u.add_argument("--pin", required=True)
    u.add_argument("--out", required=True)
    u.add_argument("--dtype", default="BF16", choices=DENSE)
    a = ap.parse_args(argv)
    if a.cmd == "convert":
        got = convert(Path(a.src), Path(a.out), a.blocksize, a.dry_run)
        print(json.dumps(got if a.dry_run else got["pin"], indent=2))
        return 0
    if a.cmd == "verify":
        got = verify(Path(a.pin), Path(a.src) if a.src else None, a.parity, a.cuda)
        text = json.dumps(got, indent=2) + "\n"
        if a.out:
            Path(a.out).write_text(text)
        print(json.dumps({k: v for k, v in got.items() if k != "modules"} if a.quiet else got, indent=2))
        return 0 if got["ok"] else 1
    print(json.dumps(unpin(Path(a.pin), Path(a.out), a.dtype), indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
