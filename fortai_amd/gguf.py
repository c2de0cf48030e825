"""GGUF v3 writer and reader (numpy, memory-mapped).

The reader follows the subset of GGUF v3 the reference loader accepts
(``src/fortai_gguf_runtime.f90:106-197``): little-endian header ``GGUF``,
version 3, int64 tensor and metadata counts, typed metadata values
(``:590-658``), tensor infos (name, rank <= 4, int64 dims, ggml type, int64
offset), data start aligned to ``general.alignment`` (default 32,
``:151-152,183-184``).  Tensor byte sizes follow ``tensor_bytes``
(``:739-762``): F32 4 B, F16 2 B, Q8_0 34 B per 32 values with the first
dimension a multiple of 32.

Dimension order is GGUF's: ``shape[0]`` is the fastest-varying (input width),
``shape[1]`` the row count, as the reference reads it
(``fortai_gguf_runtime.f90:336-337``).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

# GGUF metadata value types.
GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16 = 0, 1, 2, 3
GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL = 4, 5, 6, 7
GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = 8, 9, 10, 11, 12

# ggml tensor types used on the decode path.
GGML_TYPE_F32 = 0
GGML_TYPE_F16 = 1
GGML_TYPE_Q8_0 = 8

Q8_BLOCK = 32
Q8_BLOCK_BYTES = 34

_SCALAR_FMT = {
    GGUF_UINT8: "<B", GGUF_INT8: "<b", GGUF_UINT16: "<H", GGUF_INT16: "<h",
    GGUF_UINT32: "<I", GGUF_INT32: "<i", GGUF_FLOAT32: "<f", GGUF_BOOL: "<?",
    GGUF_UINT64: "<Q", GGUF_INT64: "<q", GGUF_FLOAT64: "<d",
}


def tensor_nbytes(ggml_type: int, shape: Tuple[int, ...]) -> int:
    elements = int(np.prod(shape, dtype=np.int64))
    if ggml_type == GGML_TYPE_F32:
        return 4 * elements
    if ggml_type == GGML_TYPE_F16:
        return 2 * elements
    if ggml_type == GGML_TYPE_Q8_0:
        if shape[0] <= 0 or shape[0] % Q8_BLOCK:
            raise ValueError("Q8_0 tensor width is not a multiple of 32")
        return (elements // shape[0]) * (shape[0] // Q8_BLOCK) * Q8_BLOCK_BYTES
    raise ValueError(f"unsupported ggml type {ggml_type}")


def _align(value: int, alignment: int) -> int:
    return ((value + alignment - 1) // alignment) * alignment


@dataclass
class TensorInfo:
    name: str
    shape: Tuple[int, ...]
    ggml_type: int
    offset: int
    nbytes: int
    data: Optional[np.ndarray] = None  # uint8 view into the mapped file

    @property
    def rows(self) -> int:
        return int(np.prod(self.shape[1:], dtype=np.int64)) if len(self.shape) > 1 else 1

    @property
    def width(self) -> int:
        return int(self.shape[0])

    def as_f32(self) -> np.ndarray:
        if self.ggml_type != GGML_TYPE_F32:
            raise TypeError(f"{self.name} is not F32")
        return self.data.view(np.float32)

    def as_f16_bits(self) -> np.ndarray:
        if self.ggml_type != GGML_TYPE_F16:
            raise TypeError(f"{self.name} is not F16")
        return self.data.view(np.uint16)


@dataclass
class GGUFFile:
    path: str
    version: int
    metadata: Dict[str, Any]
    tensors: List[TensorInfo]
    alignment: int
    data_start: int
    _map: Optional[np.memmap] = field(default=None, repr=False)

    def tensor(self, name: str) -> Optional[TensorInfo]:
        for t in self.tensors:
            if t.name == name:
                return t
        return None

    def meta_int(self, key: str, default: int = 0) -> int:
        value = self.metadata.get(key, default)
        return int(value) if isinstance(value, (int, np.integer, bool)) else default

    def meta_real(self, key: str, default: float) -> float:
        value = self.metadata.get(key, default)
        return float(value) if isinstance(value, (float, np.floating)) else default


class _Reader:
    def __init__(self, buf: memoryview):
        self.buf = buf
        self.pos = 0

    def take(self, fmt: str):
        size = struct.calcsize(fmt)
        (value,) = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += size
        return value

    def string(self) -> str:
        length = self.take("<Q")
        raw = bytes(self.buf[self.pos:self.pos + length])
        self.pos += length
        return raw.decode("utf-8", errors="replace")

    def value(self, value_type: int):
        if value_type in _SCALAR_FMT:
            return self.take(_SCALAR_FMT[value_type])
        if value_type == GGUF_STRING:
            return self.string()
        if value_type == GGUF_ARRAY:
            element_type = self.take("<I")
            count = self.take("<Q")
            return [self.value(element_type) for _ in range(count)]
        raise ValueError(f"bad GGUF metadata type {value_type}")


def read(path: str) -> GGUFFile:
    """Parse a GGUF v3 file; tensor payloads are memory-mapped, not loaded."""
    mapped = np.memmap(path, dtype=np.uint8, mode="r")
    reader = _Reader(memoryview(mapped))
    magic = bytes(reader.buf[0:4])
    reader.pos = 4
    version = reader.take("<I")
    if magic != b"GGUF" or version != 3:
        raise ValueError("unsupported or malformed GGUF header")
    tensor_count = reader.take("<q")
    metadata_count = reader.take("<q")
    if tensor_count < 0 or metadata_count < 0:
        raise ValueError("GGUF counts cannot be negative")
    metadata: Dict[str, Any] = {}
    for _ in range(metadata_count):
        key = reader.string()
        value_type = reader.take("<I")
        metadata[key] = reader.value(value_type)
    alignment = int(metadata.get("general.alignment", 32) or 32)
    if alignment <= 0:
        alignment = 32
    infos = []
    for _ in range(tensor_count):
        name = reader.string()
        rank = reader.take("<I")
        if rank <= 0 or rank > 4:
            raise ValueError("invalid GGUF tensor rank")
        shape = tuple(reader.take("<q") for _ in range(rank))
        ggml_type = reader.take("<I")
        offset = reader.take("<q")
        infos.append(TensorInfo(name, shape, ggml_type, offset, tensor_nbytes(ggml_type, shape)))
    data_start = _align(reader.pos, alignment)
    for info in infos:
        begin = data_start + info.offset
        if begin + info.nbytes > mapped.size:
            raise ValueError(f"tensor {info.name} runs past the end of the file")
        info.data = mapped[begin:begin + info.nbytes]
    return GGUFFile(path, version, metadata, infos, alignment, data_start, mapped)


class Writer:
    """Streaming GGUF v3 writer: declare tensors, then stream their payloads."""

    def __init__(self, path: str, alignment: int = 32):
        self.path = path
        self.alignment = alignment
        self.metadata: List[Tuple[str, int, Any]] = []
        self.tensors: List[Tuple[str, Tuple[int, ...], int]] = []

    def add_meta(self, key: str, value_type: int, value: Any) -> None:
        self.metadata.append((key, value_type, value))

    def add_tensor(self, name: str, shape: Tuple[int, ...], ggml_type: int) -> None:
        self.tensors.append((name, tuple(int(s) for s in shape), ggml_type))

    @staticmethod
    def _string(text: str) -> bytes:
        raw = text.encode("utf-8")
        return struct.pack("<Q", len(raw)) + raw

    def _value(self, value_type: int, value: Any) -> bytes:
        if value_type in _SCALAR_FMT:
            return struct.pack(_SCALAR_FMT[value_type], value)
        if value_type == GGUF_STRING:
            return self._string(value)
        raise ValueError("array metadata is not written by this writer")

    def write(self, payload) -> None:
        """``payload(name) -> bytes-like`` is called once per tensor, in order."""
        all_meta = [("general.alignment", GGUF_UINT32, self.alignment)] + self.metadata
        header = bytearray(b"GGUF")
        header += struct.pack("<I", 3)
        header += struct.pack("<q", len(self.tensors))
        header += struct.pack("<q", len(all_meta))
        for key, value_type, value in all_meta:
            header += self._string(key) + struct.pack("<I", value_type) + self._value(value_type, value)
        offset = 0
        offsets = []
        for name, shape, ggml_type in self.tensors:
            offsets.append(offset)
            header += self._string(name) + struct.pack("<I", len(shape))
            for dim in shape:
                header += struct.pack("<q", dim)
            header += struct.pack("<I", ggml_type) + struct.pack("<q", offset)
            offset = _align(offset + tensor_nbytes(ggml_type, shape), self.alignment)
        header += b"\0" * (_align(len(header), self.alignment) - len(header))
        with open(self.path, "wb") as handle:
            handle.write(header)
            written = 0
            for (name, shape, ggml_type), start in zip(self.tensors, offsets):
                if written < start:
                    handle.write(b"\0" * (start - written))
                    written = start
                data = payload(name)
                view = memoryview(np.ascontiguousarray(data)).cast("B")
                if len(view) != tensor_nbytes(ggml_type, shape):
                    raise ValueError(f"payload for {name} has {len(view)} bytes")
                handle.write(view)
                written += len(view)
