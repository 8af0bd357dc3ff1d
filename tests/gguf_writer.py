"""Writes small GGUF files (the published v3 layout: magic, version, tensor and
key counts, typed key/value pairs, tensor infos, data at general.alignment)
for the GGUF reader's tests.  Test infrastructure only."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v) -> bytes:
    if t == STRING:
        return _str(v)
    return struct.pack(_FMT[t], v)


def write(path, kv: list, tensors: list, alignment: int | None = None, version: int = 3,
          magic: bytes = b"GGUF", offsets: list | None = None) -> None:
    """kv: [(key, type, value)] (ARRAY values as (elem_type, [values]));
    tensors: [(name, ggml_type, dims innermost first, raw bytes)];
    offsets: data offsets to write into the tensor infos in place of the
    computed ones (for files with bad offsets)."""
    if alignment is not None:
        kv = list(kv) + [("general.alignment", U32, alignment)]
    align = alignment or 32
    out = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for key, t, v in kv:
        out += _str(key) + struct.pack("<I", t)
        if t == ARRAY:
            et, vals = v
            out += struct.pack("<IQ", et, len(vals)) + b"".join(_value(et, x) for x in vals)
        else:
            out += _value(t, v)
    computed, off = [], 0
    for _, _, _, raw in tensors:
        computed.append(off)
        off += (len(raw) + align - 1) // align * align
    for (name, gt, dims, _), o in zip(tensors, computed if offsets is None else list(offsets)):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<q", d) for d in dims)
        out += struct.pack("<iQ", gt, o)
    if tensors:
        out += b"\0" * ((-len(out)) % align)
    for _, _, _, raw in tensors:
        out += raw + b"\0" * ((-len(raw)) % align)
    open(path, "wb").write(bytes(out))


def f32(name, a) -> tuple:
    a = np.ascontiguousarray(a, np.float32)
    return (name, 0, tuple(reversed(a.shape)) if a.ndim else (1,), a.tobytes())
