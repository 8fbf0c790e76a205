"""`.cimage` container (TRB_CIMG) reader and writer.

Restates src/quantization/cimage.rs: magic ``TRB_CIMG`` (8 B), u64 LE JSON
header size, JSON header ``{"tensors": {name: {tensor_type, offset, size,
dim_m, dim_n}}, "execution_plan": str|null}`` at offset 16, 128 KB reserved
for the header (HEADER_PAGES = 8 x 16 KB, :24-26), every payload starting on
a 16 KB boundary (:23, :102-125, :210-222).

Extension: tensor type ``Palettized8Bit`` for the 8-bit split-block payload
(the reference defines only StandardFP16 / Palettized4Bit / Blob, :34-39).
"""
from __future__ import annotations

import json
import mmap
import os
import struct

import numpy as np

PAGE_SIZE = 16384
HEADER_PAGES = 8
MAGIC = b"TRB_CIMG"
TENSOR_TYPES = ("StandardFP16", "Palettized4Bit", "Palettized8Bit", "Blob")


class CImageWriter:
    """Streaming writer (cimage.rs:69-208)."""

    def __init__(self, path: str):
        self.path = path
        self.f = open(path, "wb")
        self.f.write(b"\0" * (HEADER_PAGES * PAGE_SIZE))
        self.tensors: dict[str, dict] = {}
        self.execution_plan: str | None = None

    def set_execution_plan(self, plan_json: str) -> None:
        self.execution_plan = plan_json

    def _align(self) -> None:
        pos = self.f.tell()
        rem = pos % PAGE_SIZE
        if rem:
            self.f.write(b"\0" * (PAGE_SIZE - rem))

    def _append(self, name: str, payload, ttype: str, dim_m: int, dim_n: int) -> None:
        self._align()
        off = self.f.tell()
        data = bytes(np.asarray(payload, dtype=np.uint8).reshape(-1)) if not isinstance(payload, bytes) else payload
        self.f.write(data)
        self.tensors[name] = {"tensor_type": ttype, "offset": off, "size": len(data), "dim_m": int(dim_m),
                              "dim_n": int(dim_n)}

    def append_palettized(self, name: str, payload, dim_m: int, dim_n: int, bits: int = 4) -> None:
        """Palettized split-block payload (cimage.rs:97-125; 8-bit is the extension)."""
        self._append(name, payload, "Palettized4Bit" if bits == 4 else "Palettized8Bit", dim_m, dim_n)

    def append_fp16(self, name: str, payload, dim_m: int, dim_n: int) -> None:
        self._append(name, payload, "StandardFP16", dim_m, dim_n)

    def append_blob(self, name: str, payload) -> None:
        self._append(name, payload, "Blob", 0, 0)

    def finalize(self) -> None:
        hdr = {"tensors": self.tensors, "execution_plan": self.execution_plan}
        hb = json.dumps(hdr, separators=(",", ":")).encode()
        if 16 + len(hb) > HEADER_PAGES * PAGE_SIZE:
            raise ValueError(f"header ({16 + len(hb)} B) exceeds reserved {HEADER_PAGES * PAGE_SIZE} B")
        self.f.seek(0)
        self.f.write(MAGIC)
        self.f.write(struct.pack("<Q", len(hb)))
        self.f.write(hb)
        self.f.close()


class CImageReader:
    """Header parser plus zero-copy payload views (cimage.rs:240-303); the
    payloads are memory-mapped instead of read whole (engine_impl.rs:600)."""

    def __init__(self, path: str, populate: bool = False):
        """populate: map every page up front (MAP_POPULATE), for a reader
        that will touch the whole file, such as a loader."""
        self.path = path
        with open(path, "rb") as f:
            magic = f.read(8)
            if magic != MAGIC:
                raise ValueError(f"Invalid magic: expected TRB_CIMG, got {magic!r}")
            (hsize,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(hsize))
        self._f = open(path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if not size:
            self._mm = None
        elif populate and hasattr(mmap, "MAP_POPULATE"):
            self._mm = mmap.mmap(self._f.fileno(), 0, flags=mmap.MAP_SHARED | mmap.MAP_POPULATE,
                                 prot=mmap.PROT_READ)
        else:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)

    @property
    def tensors(self) -> dict:
        return self.header.get("tensors", {})

    @property
    def execution_plan(self):
        return self.header.get("execution_plan")

    def tensor(self, name: str):
        return self.tensors.get(name)

    def payload(self, name: str) -> np.ndarray:
        rec = self.tensor(name)
        if rec is None:
            raise KeyError(f"tensor {name} not found")
        return np.frombuffer(self._mm, dtype=np.uint8, count=rec["size"], offset=rec["offset"])

    def close(self) -> None:
        if self._mm is not None:
            self._mm.close()
            self._mm = None
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def bits_of(tensor_type: str) -> int:
    if tensor_type == "Palettized4Bit":
        return 4
    if tensor_type == "Palettized8Bit":
        return 8
    raise ValueError(f"{tensor_type} is not a palettized tensor")
