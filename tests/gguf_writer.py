"""A GGUF v2/v3 writer for tests: header, metadata, tensor table, aligned data.

Follows the GGUF container format as the reference reads it
(src/gguf/mod.rs:1091-1310): little-endian, u64 counts and string lengths,
tensor dims innermost first, tensor offsets relative to the data section,
data section at the table end rounded up to general.alignment.  Array
element types other than I32, F32 and String are written with 4 bytes per
element, which is how the reference skips them.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def value_bytes(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _str(value)
    if vtype == ARRAY:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        if etype == STRING:
            return out + b"".join(_str(s) for s in items)
        if etype == I32:
            return out + b"".join(struct.pack("<i", v) for v in items)
        if etype == F32:
            return out + b"".join(struct.pack("<f", v) for v in items)
        return out + b"\0" * (4 * len(items))
    return struct.pack(_SCALAR[vtype], value)


class GgufWriter:
    def __init__(self, version: int = 3, alignment: int | None = None):
        self.version = version
        self.kv = []        # (key, type, value)
        self.tensors = []   # (name, dims, type id, payload bytes)
        self.alignment = alignment
        if alignment is not None:
            self.kv.append(("general.alignment", U32, alignment))

    def add(self, key: str, vtype: int, value):
        self.kv.append((key, vtype, value))

    def add_tensor(self, name: str, dims, type_id: int, payload):
        self.tensors.append((name, [int(d) for d in dims], type_id,
                             np.ascontiguousarray(payload).view(np.uint8).tobytes()))

    def tobytes(self) -> bytes:
        align = 32 if self.alignment is None else max(self.alignment, 1)
        out = bytearray(b"GGUF")
        out += struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv))
        for key, vtype, value in self.kv:
            out += _str(key) + struct.pack("<I", vtype) + value_bytes(vtype, value)
        offsets = []
        off = 0
        for name, dims, tid, data in self.tensors:
            offsets.append(off)
            off += len(data)
            off = (off + align - 1) // align * align
        for (name, dims, tid, data), o in zip(self.tensors, offsets):
            out += _str(name) + struct.pack("<I", len(dims))
            out += b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", tid, o)
        while len(out) % align:
            out += b"\0"
        base = len(out)
        for (name, dims, tid, data), o in zip(self.tensors, offsets):
            out += b"\0" * (base + o - len(out))
            out += data
        return bytes(out)

    def write(self, path) -> None:
        with open(path, "wb") as f:
            f.write(self.tobytes())
