"""Safetensors containers for the pin tools: memory-mapped reading, atomic writing.

The container format is fixed by the safetensors specification (and is what the
reference's pin tools read and write): an unsigned 64-bit little-endian length, that
many bytes of UTF-8 JSON, then the data section. The JSON maps each tensor name to its
"dtype", "shape" and "data_offsets" (a [begin, end) byte range relative to the data
section); an optional "__metadata__" entry holds string pairs. Writers pad the JSON with
spaces so the data section starts on an 8-byte boundary and pack the tensors back to back.

Reading maps the whole file once and keeps absolute byte ranges, so a tensor is handed
out as a zero-copy view (a pinned staging copy reads straight from the page cache).
Every range is checked against the file size and against its dtype and shape. Writing
goes to a temporary file in the destination directory that replaces the destination
only when complete, so a reader never sees a half-written shard.
"""
from __future__ import annotations

import json
import mmap
import os
import tempfile
from itertools import accumulate
from pathlib import Path
from typing import Dict, Iterator, Mapping, NamedTuple, Optional, Sequence, Tuple

import numpy as np

# Element sizes of the specification's dtypes.
ELEM_BYTES: Dict[str, int] = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E5M2": 1, "F8_E4M3": 1,
    "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
    "I32": 4, "U32": 4, "F32": 4,
    "F64": 8, "I64": 8, "U64": 8,
}
HEADER_LIMIT = 1 << 27  # a JSON header larger than this is treated as corruption


class Entry(NamedTuple):
    """One tensor of a container: absolute byte range [begin, end) in the file."""
    dtype: str
    shape: Tuple[int, ...]
    begin: int
    end: int

    @property
    def nbytes(self) -> int:
        return self.end - self.begin

    @property
    def count(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1


class TensorFile:
    """A read-only safetensors file. `entries` maps names to Entry in header order;
    `meta` is the "__metadata__" dict (empty when absent)."""

    def __init__(self, path: str | os.PathLike):
        self.path = Path(path)
        with open(self.path, "rb") as fh:
            size = os.fstat(fh.fileno()).st_size
            if size < 8:
                raise ValueError(f"{self.path}: {size} bytes is too short for a safetensors file")
            self._mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self.meta, self.entries = self._parse(size)
        except Exception:
            self._mm.close()
            raise

    def _parse(self, size: int):
        hlen = int.from_bytes(self._mm[:8], "little")
        if hlen > HEADER_LIMIT or 8 + hlen > size:
            raise ValueError(f"{self.path}: header of {hlen} bytes does not fit a {size}-byte file")
        doc = json.loads(self._mm[8:8 + hlen].decode("utf-8"))
        if not isinstance(doc, dict):
            raise ValueError(f"{self.path}: header is not a JSON object")
        meta = doc.pop("__metadata__", None) or {}
        base = 8 + hlen
        entries: Dict[str, Entry] = {}
        for name, spec in doc.items():
            dtype = str(spec["dtype"])
            shape = tuple(int(d) for d in spec["shape"])
            lo, hi = (int(v) for v in spec["data_offsets"])
            e = Entry(dtype, shape, base + lo, base + hi)
            if not (0 <= lo <= hi and e.end <= size):
                raise ValueError(f"{self.path}: '{name}' spans bytes {lo}..{hi} of a {size - base}-byte data section")
            if dtype in ELEM_BYTES and e.nbytes != e.count * ELEM_BYTES[dtype]:
                raise ValueError(f"{self.path}: '{name}' holds {e.nbytes} bytes for {e.count} x {dtype}")
            entries[name] = e
        return meta, entries

    # -- access
    def __contains__(self, name: str) -> bool:
        return name in self.entries

    def __iter__(self) -> Iterator[str]:
        return iter(self.entries)

    def buffer(self, name: str) -> memoryview:
        """Zero-copy view of a tensor's bytes, valid until close()."""
        e = self.entries[name]
        return memoryview(self._mm)[e.begin:e.end]

    def array(self, name: str, np_dtype) -> np.ndarray:
        """Zero-copy numpy view of a tensor's bytes as `np_dtype` (flat)."""
        return np.frombuffer(self.buffer(name), dtype=np_dtype)

    def blob(self, name: str) -> bytes:
        return bytes(self.buffer(name))

    # -- lifetime
    def close(self) -> None:
        if not self._mm.closed:
            self._mm.close()

    def __enter__(self) -> "TensorFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def _umask() -> int:
    """The process umask, read without changing it (Linux /proc); elsewhere set and restored."""
    try:
        with open("/proc/self/status") as fh:
            for line in fh:
                if line.startswith("Umask:"):
                    return int(line.split()[1], 8)
    except OSError:
        pass
    mask = os.umask(0o022)
    os.umask(mask)
    return mask


def save(path: str | os.PathLike, items: Sequence[Tuple[str, str, Sequence[int], object]],
         meta: Optional[Mapping[str, str]] = None) -> int:
    """Write (name, dtype, shape, bytes-like) items in order; returns the data bytes
    written. The dtype must be one of the specification's, and each item's length must
    match its shape."""
    sizes = []
    for name, dtype, shape, data in items:
        if dtype not in ELEM_BYTES:
            raise ValueError(f"'{name}': dtype {dtype!r} is not a safetensors dtype")
        nb = memoryview(data).nbytes
        want = int(np.prod(tuple(shape), dtype=np.int64)) * ELEM_BYTES[dtype] if len(shape) else ELEM_BYTES[dtype]
        if nb != want:
            raise ValueError(f"'{name}': {nb} bytes for shape {tuple(shape)} of {dtype}")
        sizes.append(nb)
    bounds = [0, *accumulate(sizes)]
    doc: dict = {}
    if meta:
        doc["__metadata__"] = {str(k): str(v) for k, v in meta.items()}
    for i, (name, dtype, shape, _data) in enumerate(items):
        doc[name] = {"dtype": dtype, "shape": [int(d) for d in shape], "data_offsets": [bounds[i], bounds[i + 1]]}
    head = json.dumps(doc, separators=(",", ":")).encode("utf-8")
    head = head.ljust(len(head) + (-(8 + len(head)) % 8), b" ")
    dest = Path(path)
    dest.parent.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=dest.name + ".", suffix=".part", dir=dest.parent)
    try:
        # mkstemp creates the file 0600; give it the mode open(path, "wb") would (0666 less
        # the umask), so a pin converted by one user stays readable by the serving user
        os.fchmod(fd, 0o666 & ~_umask())
        with os.fdopen(fd, "wb") as fh:
            fh.write(len(head).to_bytes(8, "little"))
            fh.write(head)
            for _name, _dtype, _shape, data in items:
                fh.write(memoryview(data).cast("B"))
        os.replace(tmp, dest)
    except BaseException:
        try:
            os.unlink(tmp)
        except FileNotFoundError:
            pass
        raise
    return bounds[-1]
