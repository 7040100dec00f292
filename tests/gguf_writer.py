"""Minimal GGUF v3 writer for the reader's tests -- TEST INFRASTRUCTURE ONLY.

Writes the layout GGUFReader::open parses (src/gguf.rs:321-405): magic, version,
tensor and field counts, typed key/value fields, tensor infos, then the data
section at the next multiple of the alignment, each tensor at an aligned offset
relative to it.  Field values are given as (type_id, value) pairs; arrays as
(9, (element_type_id, [values])).
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, vals = v
        return struct.pack("<IQ", et, len(vals)) + b"".join(_value(et, x) for x in vals)
    return struct.pack(_FMT[t], v)


def gguf_bytes(fields, tensors, alignment=32, version=3, magic=b"GGUF", pad_data=True):
    """fields: [(key, type_id, value)]; tensors: [(name, shape, dtype_id, raw_bytes)].
    `alignment` places the data section and the tensors (general.alignment must be
    among the fields for a reader to use a value other than 32)."""
    head = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(fields)))
    for key, t, v in fields:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for _, _, _, raw in tensors:
        offsets.append(off)
        off += len(raw)
        if pad_data:
            off = (off + alignment - 1) // alignment * alignment
    for (name, shape, dt, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", dt, o)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    out = bytearray(head) + bytes(data_start - len(head))
    for (_, _, _, raw), o in zip(tensors, offsets):
        out += bytes(data_start + o - len(out))
        out += bytes(raw)
    return bytes(out), data_start, offsets


def write_gguf(path, fields, tensors, **kw):
    b, data_start, offsets = gguf_bytes(fields, tensors, **kw)
    with open(path, "wb") as f:
        f.write(b)
    return data_start, offsets


def f32_bytes(a):
    return np.ascontiguousarray(a, np.float32).tobytes()
