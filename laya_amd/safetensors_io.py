"""Safetensors reading and writing on the host.

Reading widens F32/F16/BF16/F64/I64 to fp32, as ``SafetensorsFile.Read``
(src/StructuredDecisions.Base/Io/SafetensorsFile.cs:101-156) does; an implausible or short header
raises ``ValueError`` (SafetensorsFile.cs:47-50, 185-193). Writing stores F32, F16 or BF16 with
round-to-nearest-even, as ``SafetensorsWriter`` (SafetensorsWriter.cs:16-97) does. The file is
memory-mapped, nothing in it is executed.
"""
from __future__ import annotations

import json
import os
import struct
from typing import Dict, Iterable, List, Tuple

import numpy as np

_WIDTH = {"F32": 4, "F16": 2, "BF16": 2, "F64": 8, "I64": 8}


class SafetensorsFile:
    def __init__(self, path: str):
        self.path = path
        self._map = np.memmap(path, dtype=np.uint8, mode="r")
        if self._map.size < 8:
            raise ValueError(f"{path}: too short for a safetensors header")
        n = struct.unpack("<Q", bytes(self._map[:8]))[0]
        if n <= 0 or n > 100_000_000 or 8 + n > self._map.size:
            raise ValueError(f"{path}: implausible safetensors header length {n}")
        header = json.loads(bytes(self._map[8:8 + n]).decode("utf-8"))
        self._data_start = 8 + n
        self.entries: Dict[str, dict] = {k: v for k, v in header.items() if k != "__metadata__"}

    def names_in_file_order(self) -> List[str]:
        return sorted(self.entries, key=lambda k: self.entries[k]["data_offsets"][0])

    def shape(self, name: str) -> Tuple[int, ...]:
        return tuple(self.entries[name]["shape"])

    def dtype(self, name: str) -> str:
        return self.entries[name]["dtype"]

    def read_float32(self, name: str) -> np.ndarray:
        if name not in self.entries:
            raise KeyError(f"{self.path}: no tensor named '{name}'")
        e = self.entries[name]
        dt = e["dtype"]
        if dt not in _WIDTH:
            raise ValueError(f"{name}: unsupported safetensors dtype '{dt}'")
        count = int(np.prod(e["shape"], dtype=np.int64)) if e["shape"] else 1
        start, end = e["data_offsets"]
        if end - start != count * _WIDTH[dt]:
            raise ValueError(f"{name}: {end - start} bytes for {count} {dt} elements")
        raw = self._map[self._data_start + start:self._data_start + end]
        if dt == "F32":
            out = np.frombuffer(raw, dtype="<f4").astype(np.float32)
        elif dt == "F16":
            out = np.frombuffer(raw, dtype="<f2").astype(np.float32)
        elif dt == "BF16":
            out = (np.frombuffer(raw, dtype="<u2").astype(np.uint32) << 16).view(np.float32)
        elif dt == "F64":
            out = np.frombuffer(raw, dtype="<f8").astype(np.float32)
        else:
            out = np.frombuffer(raw, dtype="<i8").astype(np.float32)
        return out.reshape(e["shape"])


def _to_bf16_bits(x: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = bits + (np.uint32(0x7FFF) + ((bits >> 16) & 1))
    out = (rounded >> 16).astype(np.uint16)
    nan = np.isnan(x)
    out[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def write(path: str, tensors: Iterable[Tuple[str, Tuple[int, ...], np.ndarray, str]]) -> None:
    """Writes ``(name, shape, fp32 values, dtype)`` tuples; dtype is F32, F16 or BF16."""
    header, blobs, offset = {}, [], 0
    for name, shape, values, dtype in tensors:
        v = np.asarray(values, dtype=np.float32).reshape(-1)
        if dtype == "F32":
            blob = v.astype("<f4").tobytes()
        elif dtype == "F16":
            blob = v.astype("<f2").tobytes()
        elif dtype == "BF16":
            blob = _to_bf16_bits(v).astype("<u2").tobytes()
        else:
            raise ValueError(f"{name}: cannot write dtype '{dtype}'")
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(blob)]}
        blobs.append(blob)
        offset += len(blob)
    text = json.dumps(header, separators=(",", ":")).encode("utf-8")
    text += b" " * ((8 - len(text) % 8) % 8)
    # Written beside the target and moved over it once complete (as SafetensorsWriter does with its .tmp
    # file, SafetensorsWriter.cs:46-58): a crash mid-write never leaves a truncated file under `path`.
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)
