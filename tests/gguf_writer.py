"""A small GGUF v3 writer for the tests: synthetic model files with chosen metadata, tensors and faults.

The layout is the published GGUF v3 format (the one the reference reader parses, include/strata/artifact/
gguf_reader.hpp:447-501): magic "GGUF", u32 version, u64 tensor count, u64 metadata count, the metadata
(key string, u32 value type, value), the tensor directory (name, u32 n_dims, u64 dims, u32 type, u64 offset from the
data section), zero padding to general.alignment (32 when absent), then the payloads at their offsets.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
        F64: "<d"}


def gguf_str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def value(t: int, v, elem: int | None = None) -> bytes:
    """A metadata value of type t (ARRAY: v a list of items of type elem, or of (type, items) for nested arrays)."""
    if t == STRING:
        return gguf_str(v)
    if t == ARRAY:
        out = struct.pack("<IQ", elem, len(v))
        for item in v:
            out += value(elem, item[1], item[0]) if elem == ARRAY else value(elem, item)
        return out
    return struct.pack(_FMT[t], v)


@dataclass
class Tensor:
    name: str
    type: int
    shape: tuple[int, ...]   # GGUF order: dim 0 fastest
    data: bytes
    offset: int | None = None  # None: placed after the previous tensor, aligned


@dataclass
class GgufFile:
    meta: list[tuple[str, int, object, int | None]] = field(default_factory=list)  # key, type, value, elem type
    tensors: list[Tensor] = field(default_factory=list)
    version: int = 3
    magic: bytes = b"GGUF"
    alignment: int = 32

    def kv(self, key: str, t: int, v, elem: int | None = None) -> "GgufFile":
        self.meta.append((key, t, v, elem))
        if key == "general.alignment":
            self.alignment = int(v)
        return self

    def add(self, name: str, ggml_type: int, shape: tuple[int, ...], data: bytes | np.ndarray,
            offset: int | None = None) -> "GgufFile":
        self.tensors.append(Tensor(name, ggml_type, tuple(shape), bytes(np.asarray(data).tobytes() if
                                                                            isinstance(data, np.ndarray) else data),
                                   offset))
        return self

    def to_bytes(self) -> bytes:
        out = self.magic + struct.pack("<IQQ", self.version, len(self.tensors), len(self.meta))
        for key, t, v, elem in self.meta:
            out += gguf_str(key) + struct.pack("<I", t) + value(t, v, elem)
        offs, pos = [], 0
        for tn in self.tensors:
            if tn.offset is None:
                pos = (pos + self.alignment - 1) // self.alignment * self.alignment
                offs.append(pos)
                pos += len(tn.data)
            else:
                offs.append(tn.offset)
                pos = max(pos, tn.offset + len(tn.data))
        for tn, off in zip(self.tensors, offs):
            out += gguf_str(tn.name) + struct.pack("<I", len(tn.shape))
            out += b"".join(struct.pack("<Q", d) for d in tn.shape)
            out += struct.pack("<IQ", tn.type, off)
        out += b"\0" * ((self.alignment - len(out) % self.alignment) % self.alignment)
        data = bytearray(pos)
        for tn, off in zip(self.tensors, offs):
            data[off: off + len(tn.data)] = tn.data
        return out + bytes(data)

    def write(self, path) -> str:
        with open(path, "wb") as f:
            f.write(self.to_bytes())
        return str(path)
