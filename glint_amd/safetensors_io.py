"""safetensors files for the pin tools: a memory-mapped reader and a spec-contiguous writer.

Format (the one the reference's pin tools read and write, safetensors_io.py:1-104):
8-byte little-endian header length, a JSON header mapping each tensor name to
{"dtype", "shape", "data_offsets": [start, end]} (offsets relative to the data section)
plus an optional "__metadata__" of string pairs, then the data. The writer emits the
header compactly (no spaces), "__metadata__" first, padded with spaces so the data
section starts on an 8-byte boundary, and the tensors back to back with no gaps or tail,
so official readers accept it and the reference's writer would produce the same bytes.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass
from typing import Dict, Iterable, List, Mapping, Optional, Tuple

DTYPE_WIDTH = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E5M2": 1, "F8_E4M3": 1,
    "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
    "I32": 4, "U32": 4, "F32": 4,
    "F64": 8, "I64": 8, "U64": 8,
}
MAX_HEADER = 100_000_000


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype: str
    shape: Tuple[int, ...]
    data_offsets: Tuple[int, int]  # relative to the data section

    @property
    def nbytes(self) -> int:
        return int(self.data_offsets[1] - self.data_offsets[0])


class SafeTensorsFile:
    """Header parsed once; tensor bytes are served from a read-only memory map, so a
    tensor can be handed to a device copy without an intermediate file read."""

    def __init__(self, path: str | os.PathLike):
        self.path = str(path)
        self._fp = open(self.path, "rb")
        head = self._fp.read(8)
        if len(head) != 8:
            raise ValueError(f"{self.path}: truncated header length")
        (hlen,) = struct.unpack("<Q", head)
        if hlen > MAX_HEADER:
            raise ValueError(f"{self.path}: implausible header length {hlen}")
        header = json.loads(self._fp.read(hlen).decode("utf-8"))
        self.metadata: Dict[str, str] = header.pop("__metadata__", {}) or {}
        self.data_start = 8 + hlen
        size = os.fstat(self._fp.fileno()).st_size
        self.tensors: Dict[str, TensorInfo] = {}
        for name, spec in header.items():
            off = spec["data_offsets"]
            info = TensorInfo(name, str(spec["dtype"]), tuple(int(d) for d in spec["shape"]), (int(off[0]), int(off[1])))
            if info.data_offsets[0] > info.data_offsets[1] or self.data_start + info.data_offsets[1] > size:
                raise ValueError(f"{self.path}: tensor {name} lies outside the file")
            self.tensors[name] = info
        self._map = mmap.mmap(self._fp.fileno(), 0, access=mmap.ACCESS_READ) if size > 0 else None

    def close(self) -> None:
        if self._map is not None:
            self._map.close()
            self._map = None
        self._fp.close()

    def __enter__(self) -> "SafeTensorsFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def view(self, name: str) -> memoryview:
        """Zero-copy view of a tensor's bytes (valid until close())."""
        info = self.tensors[name]
        a = self.data_start + info.data_offsets[0]
        return memoryview(self._map)[a:a + info.nbytes]

    def read_bytes(self, name: str) -> bytes:
        return bytes(self.view(name))

    def names(self) -> List[str]:
        return list(self.tensors)


def write_safetensors(path: str | os.PathLike, tensors: Iterable[Tuple[str, str, Tuple[int, ...], bytes]],
                      metadata: Optional[Mapping[str, str]] = None) -> None:
    """Write (name, dtype, shape, raw bytes) tensors in the given order."""
    planned = []
    cursor = 0
    for name, dtype, shape, blob in tensors:
        if dtype not in DTYPE_WIDTH:
            raise ValueError(f"unsupported dtype {dtype}")
        planned.append((name, dtype, tuple(shape), blob, cursor, cursor + len(blob)))
        cursor += len(blob)
    header: dict = {}
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    for name, dtype, shape, _blob, start, end in planned:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [start, end]}
    hb = json.dumps(header, separators=(",", ":")).encode("utf-8")
    hb += b" " * ((-(len(hb) + 8)) % 8)
    parent = os.path.dirname(str(path))
    if parent:
        os.makedirs(parent, exist_ok=True)
    with open(path, "wb") as fp:
        fp.write(struct.pack("<Q", len(hb)))
        fp.write(hb)
        for _name, _dtype, _shape, blob, _start, _end in planned:
            fp.write(blob)
