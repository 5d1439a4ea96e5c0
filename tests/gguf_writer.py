"""Minimal GGUF v3 writer for the tests, following the published GGUF layout
(the same one gguf_loader.rs:1-30 documents): magic, version, tensor and
metadata counts, typed metadata, tensor directory, padding to
general.alignment, then each tensor's bytes at an aligned offset.

Test infrastructure: it writes synthetic files that the library under test
then reads back; nothing here is used by the product path.
"""
from __future__ import annotations

import struct

import numpy as np

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v, elem_type: int | None = None) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARRAY:
        out = struct.pack("<IQ", elem_type, len(v))
        for e in v:
            out += _value(elem_type, e)
        return out
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, metadata: list[tuple], tensors: list[tuple], alignment: int | None = None,
               version: int = 3) -> dict:
    """metadata: (key, vtype, value[, elem_type]); tensors: (name, dims in GGUF
    order, ggml type id, raw bytes).  Returns {name: (offset, data_start)}."""
    align = alignment or 32
    meta = list(metadata)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for m in meta:
        key, vt, val = m[0], m[1], m[2]
        head += _str(key) + struct.pack("<I", vt) + _value(vt, val, m[3] if len(m) > 3 else None)
    offsets, off = {}, 0
    infos = b""
    for name, dims, ttype, data in tensors:
        off = (off + align - 1) // align * align
        offsets[name] = off
        infos += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", ttype, off)
        off += len(data)
    head += infos
    data_start = (len(head) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)))
        pos = 0
        for name, dims, ttype, data in tensors:
            pad = offsets[name] - pos
            f.write(b"\0" * pad + bytes(np.asarray(data, np.uint8).tobytes() if isinstance(data, np.ndarray) else data))
            pos = offsets[name] + len(data)
    return {"offsets": offsets, "data_start": data_start}
