"""TEST INFRASTRUCTURE: a writer of GGUF v3 files (the layout the reference
reads in src/gguf.c:131-194), for the loader tests. Builds the bytes of a file
from key/value pairs and tensors, with hooks to corrupt it."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_FMT[t], v)


def gguf_bytes(kvs, tensors, alignment=32, version=3, magic=b"GGUF", offsets=None):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, ne (tuple, ne[0] contiguous), data bytes)].
    Returns the file bytes; tensor data placed at aligned offsets (or `offsets`, a list, when given)."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, pos = [], 0
    for i, (_, _, _, data) in enumerate(tensors):
        o = offsets[i] if offsets is not None else pos
        offs.append(o)
        pos = max(pos, o + len(data))
        pos = (pos + alignment - 1) // alignment * alignment
    for (name, gt, ne, _), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne) + struct.pack("<IQ", gt, o)
    data_off = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(pos)
    for (_, _, _, data), o in zip(tensors, offs):
        body[o:o + len(data)] = data
    return head + bytes(data_off - len(head)) + bytes(body)


def write(path, kvs, tensors, **kw):
    b = gguf_bytes(kvs, tensors, **kw)
    with open(path, "wb") as f:
        f.write(b)
    return b


def np_bytes(a):
    return np.ascontiguousarray(a).tobytes()
