"""A small GGUF writer for tests: synthetic model files with no downloaded model.

Layout written (GGUF v2 / v3, little-endian): magic "GGUF", version, tensor count,
key/value count, the key/values, the tensor directory (name, dims innermost first,
ggml type, data offset relative to the data section), padding to the alignment,
then each tensor's bytes at its aligned offset. ``split(parts)`` writes the model
as gguf-split does: the first part holds all metadata, every part carries
split.no / split.count / split.tensors.count and its share of the tensors
(the reference's test writer: dynalm/tests/tiny_gguf.h).
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}

# ggml type ids of the weight types, with (values, bytes) per block
GGML_F32, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 2, 8, 12, 14
GEOMETRY = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


class GgufWriter:
    def __init__(self, version: int = 3, alignment: int | None = None):
        self.version = version
        self.alignment = alignment
        self.kvs: list[tuple[str, int, object]] = []
        self.tensors: list[tuple[str, int, list[int], bytes]] = []
        if alignment is not None:
            self.kv("general.alignment", U32, alignment)

    def kv(self, key: str, vtype: int, value) -> "GgufWriter":
        self.kvs.append((key, vtype, value))
        return self

    def tensor(self, name: str, ggml_type: int, shape: list[int], data: bytes) -> "GgufWriter":
        """shape in engine order (outermost first), as a weight [n, k]."""
        self.tensors.append((name, ggml_type, list(shape), bytes(data)))
        return self

    def to_bytes(self, offsets: dict[str, int] | None = None, raw_dims: dict[str, list[int]] | None = None) -> bytes:
        """The file. `offsets` / `raw_dims` override a tensor's stored offset / GGUF dims (malformed files)."""
        al = self.alignment or 32
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kvs))
        for key, vtype, value in self.kvs:
            head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
        data = b""
        directory = b""
        for name, gtype, shape, blob in self.tensors:
            pad = (-len(data)) % al
            data += b"\0" * pad
            off = len(data)
            if offsets and name in offsets:
                off = offsets[name]
            dims = raw_dims[name] if raw_dims and name in raw_dims else list(reversed(shape))
            directory += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            directory += struct.pack("<IQ", gtype, off)
            data += blob
        body = head + directory
        body += b"\0" * ((-len(body)) % al)
        return body + data

    def split(self, parts: int) -> list[bytes]:
        per = (len(self.tensors) + parts - 1) // parts
        out = []
        for p in range(parts):
            w = GgufWriter(self.version, self.alignment)
            if p == 0:
                w.kvs = list(self.kvs)
            w.kv("split.no", U16, p).kv("split.count", U16, parts).kv("split.tensors.count", I32, len(self.tensors))
            w.tensors = self.tensors[p * per:(p + 1) * per]
            out.append(w.to_bytes())
        return out


def split_names(prefix: str, parts: int) -> list[str]:
    return [f"{prefix}-{i + 1:05d}-of-{parts:05d}.gguf" for i in range(parts)]
