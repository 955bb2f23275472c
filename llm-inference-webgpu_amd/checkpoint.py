"""Safetensors checkpoints for the load path.

The container, as the safetensors format defines it: an unsigned 64-bit little-endian
byte count N, N bytes of UTF-8 JSON, then one byte buffer. The JSON object maps each
tensor name to ``{"dtype": <element type>, "shape": [dims], "data_offsets": [start,
stop]}`` with the offsets counted from the start of the buffer; an optional
``"__metadata__"`` entry maps strings to strings.

``Safetensors.open`` checks the whole header against the file before anything is read
and reports every defect it finds in one error (a checkpoint with a bad record usually
has more than one). The buffer is then memory-mapped read-only, so a tensor's bytes go
to the device loader (qh_model_load_tensor) straight from the page cache, one tensor at
a time. The reader's methods carry the names of the reference's reader that callers use
(names / has / info / read_raw, src/core/safetensors.js); the checks and messages are
this module's own.
"""
from __future__ import annotations

import json
import math
import os
from dataclasses import dataclass

import numpy as np

# Bytes per element of each element type of the format.
ELEMENT_BYTES = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1,
    "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
    "I32": 4, "U32": 4, "F32": 4,
    "I64": 8, "U64": 8, "F64": 8,
}
# How the loader hands on the element types it reads: 16-bit floats as their bits.
LOADER_VIEWS = {"BF16": np.uint16, "F16": np.uint16, "F32": np.float32}
# Headers beyond this are refused outright (the format's own readers cap them too).
HEADER_LIMIT = 100 << 20


class SafetensorsError(ValueError):
    pass


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype: str
    shape: tuple
    begin: int   # offset of the first byte within the buffer
    end: int     # one past the last byte

    @property
    def numel(self) -> int:
        return math.prod(self.shape)  # exact Python integers: a huge shape cannot wrap to a small count

    @property
    def byte_length(self) -> int:
        return self.end - self.begin


def _is_count(v) -> bool:
    """A non-negative integer (JSON booleans are not counts)."""
    return isinstance(v, int) and not isinstance(v, bool) and v >= 0


def _record_defects(name, record, buffer_bytes):
    """(TensorInfo or None, [defects]) for one header record."""
    if not isinstance(record, dict):
        return None, [f"'{name}': the record is a JSON {type(record).__name__}, not an object"]
    defects = []
    dtype, shape, span = record.get("dtype"), record.get("shape"), record.get("data_offsets")
    if dtype not in ELEMENT_BYTES:
        defects.append(f"'{name}': {dtype!r} is not a safetensors element type")
    if not (isinstance(shape, list) and all(_is_count(d) for d in shape)):
        defects.append(f"'{name}': dimensions {shape!r} are not a list of non-negative integers")
    if not (isinstance(span, list) and len(span) == 2 and all(_is_count(v) for v in span) and span[0] <= span[1]):
        defects.append(f"'{name}': data_offsets {span!r} is not [start, stop] with 0 <= start <= stop")
    if defects:
        return None, defects
    info = TensorInfo(name, dtype, tuple(shape), span[0], span[1])
    if info.end > buffer_bytes:
        return None, [f"'{name}': bytes [{info.begin}, {info.end}) extend past the {buffer_bytes}-byte buffer"]
    need = info.numel * ELEMENT_BYTES[dtype]
    if info.byte_length != need:
        return None, [f"'{name}': {info.numel} x {dtype} is {need} bytes, the record spans {info.byte_length}"]
    return info, []


class Safetensors:
    """A checked, memory-mapped safetensors file."""

    def __init__(self, path, records, buffer_start, metadata, file_bytes):
        self.path, self.metadata = path, metadata
        self._records, self._buffer_start, self._file_bytes = records, buffer_start, file_bytes
        self._map = None

    @staticmethod
    def open(path: str) -> "Safetensors":
        file_bytes = os.path.getsize(path)
        where = os.path.basename(path)
        if file_bytes < 8:
            raise SafetensorsError(f"{where}: {file_bytes} bytes is too short for a safetensors length prefix")
        with open(path, "rb") as f:
            n = int.from_bytes(f.read(8), "little")
            if n == 0 or n > min(file_bytes - 8, HEADER_LIMIT):
                raise SafetensorsError(f"{where}: the length prefix declares a {n}-byte header, but "
                                       f"{file_bytes - 8} bytes follow it (and headers are limited to "
                                       f"{HEADER_LIMIT} bytes)")
            text = f.read(n)
        try:
            header = json.loads(text.decode("utf-8"))
        except (UnicodeDecodeError, ValueError) as e:
            raise SafetensorsError(f"{where}: the header is not UTF-8 JSON ({e})") from e
        if not isinstance(header, dict):
            raise SafetensorsError(f"{where}: the header is a JSON {type(header).__name__}, "
                                   "not an object of tensor records")
        buffer_start = 8 + n
        buffer_bytes = file_bytes - buffer_start
        defects = []
        metadata = header.pop("__metadata__", None)
        if metadata is not None and not (isinstance(metadata, dict)
                                         and all(isinstance(v, str) for v in metadata.values())):
            defects.append("__metadata__ is not an object of strings")
        records = {}
        for name, record in header.items():
            info, found = _record_defects(name, record, buffer_bytes)
            defects += found
            if info is not None:
                records[name] = info
        # Two records must never claim the same byte.
        by_start = sorted((r for r in records.values() if r.byte_length), key=lambda r: (r.begin, r.end))
        for a, b in zip(by_start, by_start[1:]):
            if b.begin < a.end:
                defects.append(f"'{b.name}' [{b.begin}, {b.end}) overlaps '{a.name}' [{a.begin}, {a.end})")
        if defects:
            raise SafetensorsError(f"{where}: {len(defects)} defect{'s' if len(defects) > 1 else ''} in the "
                                   "header: " + "; ".join(defects))
        return Safetensors(path, records, buffer_start, metadata, file_bytes)

    def __len__(self) -> int:
        return len(self._records)

    def names(self) -> list:
        return list(self._records)

    def has(self, name: str) -> bool:
        return name in self._records

    def info(self, name: str) -> TensorInfo:
        try:
            return self._records[name]
        except KeyError:
            raise SafetensorsError(f"{os.path.basename(self.path)} holds no tensor {name!r}") from None

    def read_raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as stored: a read-only view of the file mapping."""
        t = self.info(name)
        if t.byte_length == 0:
            return np.zeros(0, np.uint8)
        if self._map is None:
            self._map = np.memmap(self.path, np.uint8, "r", offset=self._buffer_start,
                                  shape=(self._file_bytes - self._buffer_start,))
        return self._map[t.begin:t.end]

    def array(self, name: str) -> np.ndarray:
        """The tensor in the loader's view, shaped: BF16 and F16 as uint16 bits, F32 as float32."""
        t = self.info(name)
        view = LOADER_VIEWS.get(t.dtype)
        if view is None:
            raise SafetensorsError(f"{name}: the loader reads BF16, F16 and F32 tensors, not {t.dtype}")
        raw = self.read_raw(name)
        if raw.ctypes.data % np.dtype(view).itemsize:
            raw = raw.copy()   # the format does not promise aligned tensors
        return raw.view(view).reshape(t.shape)

    def close(self) -> None:
        self._map = None


def write(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """Write {name: (dtype, array)} as a safetensors file, tensors back to back in the given
    order and the header padded with spaces to a multiple of 8 bytes (for tests and tools that
    make checkpoints)."""
    header, blobs, offset = {}, [], 0
    for name, (dtype, a) in tensors.items():
        a = np.ascontiguousarray(a)
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [offset, offset + a.nbytes]}
        blobs.append(a)
        offset += a.nbytes
    if metadata is not None:
        header["__metadata__"] = metadata
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little"))
        f.write(text)
        for a in blobs:
            f.write(a.tobytes())
