"""Safetensors checkpoints for the load path (src/core/safetensors.js:1-160).

The container: a little-endian u64 header length, a JSON header mapping tensor names
to {dtype, shape, data_offsets}, then the tensor bytes back to back. ``Safetensors.open``
validates the header against the file the way the reference does (safetensors.js:56-125)
and maps the data section read-only, so a tensor's bytes are handed to the device
loader (qh_model_load_tensor) straight from the page cache: nothing is widened or copied
on the host, and at most one tensor's pages are touched at a time.
"""
from __future__ import annotations

import json
import os

import numpy as np

# Bytes per element of every dtype safetensors defines (safetensors.js:15-21).
DTYPE_SIZE = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1,
    "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
    "I32": 4, "U32": 4, "F32": 4,
    "I64": 8, "U64": 8, "F64": 8,
}
# The element views the loader hands on: bf16 and f16 as their bits.
VIEW = {"BF16": np.uint16, "F16": np.uint16, "F32": np.float32}


class SafetensorsError(ValueError):
    pass


class TensorInfo:
    __slots__ = ("name", "dtype", "shape", "begin", "end")

    def __init__(self, name, dtype, shape, begin, end):
        self.name, self.dtype, self.shape, self.begin, self.end = name, dtype, tuple(shape), begin, end

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def byte_length(self) -> int:
        return self.end - self.begin


def _int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


class Safetensors:
    """Safetensors.open / names / has / info / readRaw (safetensors.js:36-160)."""

    def __init__(self, path, tensors, data_start, metadata, file_size):
        self.path, self.metadata = path, metadata
        self._tensors, self._data_start, self._file_size = tensors, data_start, file_size
        self._map = None

    @staticmethod
    def open(path: str) -> "Safetensors":
        size = os.path.getsize(path)
        if size < 8:
            raise SafetensorsError(f"not a safetensors file: {size} bytes")
        with open(path, "rb") as f:
            header_len = int.from_bytes(f.read(8), "little")
            if header_len <= 0 or header_len > 2 ** 53 - 1 or 8 + header_len > size:
                raise SafetensorsError(f"header length {header_len} does not fit in a {size}-byte file")
            raw = f.read(header_len)
        try:
            header = json.loads(raw.decode("utf-8"))
        except (UnicodeDecodeError, ValueError) as e:
            raise SafetensorsError(f"header is not valid UTF-8 JSON: {e}") from e
        if not isinstance(header, dict):
            raise SafetensorsError("header must be a JSON object")
        metadata = header.pop("__metadata__", None)
        data_start = 8 + header_len
        data_size = size - data_start
        tensors = {}
        for name, entry in header.items():
            entry = entry if isinstance(entry, dict) else {}
            dtype, shape, offsets = entry.get("dtype"), entry.get("shape"), entry.get("data_offsets")
            if dtype not in DTYPE_SIZE:
                raise SafetensorsError(f"{name}: unknown dtype {json.dumps(dtype)}")
            if not isinstance(shape, list) or not all(_int(d) and d >= 0 for d in shape):
                raise SafetensorsError(f"{name}: shape must be an array of non-negative integers")
            if not isinstance(offsets, list) or len(offsets) != 2:
                raise SafetensorsError(f"{name}: data_offsets must be a pair")
            begin, end = offsets
            if not (_int(begin) and _int(end)) or begin < 0 or end < begin:
                raise SafetensorsError(f"{name}: bad data_offsets [{begin}, {end}]")
            if end > data_size:
                raise SafetensorsError(f"{name}: ends at {end} but the data section is only {data_size} bytes")
            info = TensorInfo(name, dtype, shape, begin, end)
            if end - begin != info.numel * DTYPE_SIZE[dtype]:
                raise SafetensorsError(f"{name}: shape {list(shape)} of {dtype} needs "
                                       f"{info.numel * DTYPE_SIZE[dtype]} bytes but the header reserves "
                                       f"{end - begin}")
            tensors[name] = info
        ranges = sorted(tensors.values(), key=lambda t: t.begin)
        for a, b in zip(ranges, ranges[1:]):
            if b.begin < a.end:
                raise SafetensorsError(f"{b.name} overlaps {a.name}")
        return Safetensors(path, tensors, data_start, metadata, size)

    def __len__(self) -> int:
        return len(self._tensors)

    def names(self) -> list:
        return list(self._tensors)

    def has(self, name: str) -> bool:
        return name in self._tensors

    def info(self, name: str) -> TensorInfo:
        t = self._tensors.get(name)
        if t is None:
            raise SafetensorsError(f"no tensor named {json.dumps(name)}")
        return t

    def read_raw(self, name: str) -> np.ndarray:
        """The tensor's bytes exactly as stored (a read-only view of the file mapping)."""
        t = self.info(name)
        if t.byte_length == 0:
            return np.zeros(0, np.uint8)
        if self._map is None:
            self._map = np.memmap(self.path, np.uint8, "r", offset=self._data_start,
                                  shape=(self._file_size - self._data_start,))
        return self._map[t.begin:t.end]

    def array(self, name: str) -> np.ndarray:
        """The tensor as its element view, shaped: BF16 and F16 as uint16 bits, F32 as float32."""
        t = self.info(name)
        view = VIEW.get(t.dtype)
        if view is None:
            raise SafetensorsError(f"{name}: dtype {t.dtype} is not a weight format the loader reads")
        raw = self.read_raw(name)
        if raw.ctypes.data % np.dtype(view).itemsize:
            raw = raw.copy()   # a misaligned tensor (the format does not promise alignment)
        return raw.view(view).reshape(t.shape)

    def close(self) -> None:
        self._map = None


def write(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """Write {name: (dtype, array)} as a safetensors file: the header padded with spaces to a
    multiple of 8 bytes, tensors back to back in the given order. (For tests and tools that
    make checkpoints; the reference only reads them.)"""
    header, offset = {}, 0
    blobs = []
    for name, (dtype, a) in tensors.items():
        a = np.ascontiguousarray(a)
        n = a.nbytes
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [offset, offset + n]}
        blobs.append(a)
        offset += n
    if metadata is not None:
        header["__metadata__"] = metadata
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little"))
        f.write(text)
        for a in blobs:
            f.write(a.tobytes())
