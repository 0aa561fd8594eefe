"""Writes GGUF files byte by byte from the GGUF specification (little-endian).

Test helper: builds well-formed and deliberately malformed inputs for the
library's GGUF reader.  Layout (GGUF v2/v3): magic "GGUF", u32 version,
u64 tensor count, u64 metadata count, metadata (string key, u32 kind, value),
tensor infos (string name, u32 n_dims, u64 ne[n_dims], u32 type, u64 offset),
padding to the alignment, then the tensor data section.
"""
from __future__ import annotations

import struct

# GGUF metadata value kinds
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def gvalue(kind: int, value) -> bytes:
    if kind == STRING:
        return gstr(value)
    if kind == ARRAY:
        et, items = value
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += gvalue(et, it)
        return out
    if kind not in _SCALAR:  # an unknown kind: its value written as 4 raw bytes
        return struct.pack("<I", value)
    return struct.pack(_SCALAR[kind], value)


def gguf_bytes(metadata=(), tensors=(), version: int = 3, alignment: int = 32, magic: int = 0x46554747,
               tensor_count: int | None = None, metadata_count: int | None = None, trailer: bytes = b"") -> bytes:
    """metadata: (key, kind, value); tensors: (name, ne, storage_type, data, offset or None).

    Offsets left as None are placed one after another, each aligned.  ``data``
    of each tensor is written at its offset in the data section."""
    head = struct.pack("<II", magic, version)
    head += struct.pack("<QQ", len(tensors) if tensor_count is None else tensor_count,
                        len(metadata) if metadata_count is None else metadata_count)
    for key, kind, value in metadata:
        head += gstr(key) + struct.pack("<I", kind) + gvalue(kind, value)
    placed, cursor = [], 0
    for name, ne, st, data, off in tensors:
        if off is None:
            off = (cursor + alignment - 1) // alignment * alignment
        placed.append((name, ne, st, data, off))
        cursor = max(cursor, off + len(data))
    for name, ne, st, data, off in placed:
        head += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", st, off)
    pad = (-len(head)) % alignment
    body = bytearray(cursor)
    for name, ne, st, data, off in placed:
        body[off:off + len(data)] = data
    return head + b"\0" * pad + bytes(body) + trailer
