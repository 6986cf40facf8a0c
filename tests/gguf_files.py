"""Writes GGUF files for the tests (format version 2/3: header, metadata
key/values, tensor table, data section at a 32-byte boundary).

Test infrastructure: the files are inputs for the parser tests; each field
is written explicitly so a test can also build malformed files.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}
MAGIC = 0x46554747

# (block elements, block bytes) of the GGML types the reference tables list
# (src/ai/gguf.c:26-94); other numbers below 30 have no entry there.
TYPE_GEO = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
            10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
            24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 29: (1, 2)}


def size_bytes(ggml_type: int, n_elements: int) -> int:
    """Whole blocks only; 0 for types without a table entry or past its end."""
    if ggml_type not in TYPE_GEO:
        return 0
    blk, nb = TYPE_GEO[ggml_type]
    return (n_elements // blk) * nb


def gstr(s: str | bytes, declared_len: int | None = None) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b) if declared_len is None else declared_len) + b


def value(vtype: int, v) -> bytes:
    """type tag + payload; v for ARR is (elem_type, list)."""
    out = struct.pack("<I", vtype)
    if vtype == STR:
        return out + gstr(v)
    if vtype == ARR:
        et, items = v
        out += struct.pack("<IQ", et, len(items))
        if et == STR:
            return out + b"".join(gstr(x) for x in items)
        return out + b"".join(struct.pack(_FMT[et], x) for x in items)
    return out + struct.pack(_FMT[vtype], v)


class Tensor:
    def __init__(self, name, dims, ggml_type, data: bytes | None = None, offset: int | None = None):
        self.name, self.dims, self.type = name, list(dims), ggml_type
        n = int(np.prod(self.dims)) if self.dims else 1
        self.n_elements = n
        self.size = size_bytes(ggml_type, n)
        self.data = data if data is not None else bytes(self.size)
        self.offset = offset


def build(kvs, tensors, version: int = 3, n_kv: int | None = None, n_tensors: int | None = None) -> tuple[bytes, int]:
    """File bytes and the data-section offset.  kvs: list of (key, vtype, value)
    or raw bytes (a pre-encoded entry).  Tensor offsets default to the next
    32-byte boundary of the data section."""
    head = struct.pack("<IIQQ", MAGIC, version, len(tensors) if n_tensors is None else n_tensors,
                       len(kvs) if n_kv is None else n_kv)
    body = b""
    for e in kvs:
        body += e if isinstance(e, bytes) else gstr(e[0]) + value(e[1], e[2])
    off = 0
    for t in tensors:
        if t.offset is None:
            t.offset = (off + 31) // 32 * 32
        off = t.offset + len(t.data)
        body += gstr(t.name) + struct.pack("<I", len(t.dims)) + b"".join(struct.pack("<Q", d) for d in t.dims)
        body += struct.pack("<IQ", t.type, t.offset)
    meta = head + body
    data_offset = (len(meta) + 31) // 32 * 32
    data = bytearray(max((t.offset + len(t.data) for t in tensors), default=0))
    for t in tensors:
        data[t.offset:t.offset + len(t.data)] = t.data
    return meta + bytes(data_offset - len(meta)) + bytes(data), data_offset


def write(path, kvs, tensors, **kw) -> int:
    blob, data_offset = build(kvs, tensors, **kw)
    with open(path, "wb") as f:
        f.write(blob)
    return data_offset
