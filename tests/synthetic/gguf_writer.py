"""Minimal GGUF v3 writer (from the GGUF v3 file format: little-endian
header "GGUF", u32 version, u64 tensor and metadata counts, typed metadata,
tensor infos, data section aligned to general.alignment, each tensor's data
at its aligned relative offset). Used to make synthetic weight files for
the reader tests and the load benchmark; knobs produce the malformed
variants the reader must reject.
"""
from __future__ import annotations

import struct

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i",
        F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0 = 0, 1, 2, 3, 8


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _str(value)
    if vtype == ARRAY:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, v) for v in items)
    return struct.pack(_FMT[vtype], value)


def write_gguf(path, metadata, tensors, *, version=3, magic=b"GGUF",
               alignment=None, truncate=0, tensor_count=None, layout_alignment=None):
    """metadata: list of (key, vtype, value); tensors: list of
    (name, dims (GGUF order), ggml_type, raw bytes). `alignment` adds a
    general.alignment u32 entry; data is laid out at `layout_alignment`
    (default: `alignment`, else 32). Returns {name: absolute data offset}."""
    meta = list(metadata)
    align = 32
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
        align = alignment
    if layout_alignment is not None:
        align = layout_alignment
    head = magic + struct.pack("<IQQ", version,
                               len(tensors) if tensor_count is None else tensor_count,
                               len(meta))
    for key, vtype, value in meta:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
    rel, offsets = 0, []
    for name, dims, gtype, raw in tensors:
        offsets.append(rel)
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gtype, rel)
        rel += len(raw)
        rel = (rel + align - 1) // align * align
    data_start = (len(head) + align - 1) // align * align
    body = bytearray(head + b"\0" * (data_start - len(head)))
    for (name, dims, gtype, raw), off in zip(tensors, offsets):
        body += b"\0" * (data_start + off - len(body))
        body += bytes(raw)
    if truncate:
        body = body[:-truncate]
    with open(path, "wb") as f:
        f.write(body)
    return {t[0]: data_start + off for t, off in zip(tensors, offsets)}


def blocks_bytes(blocks: np.ndarray) -> bytes:
    return np.ascontiguousarray(blocks).view(np.uint8).tobytes()
