"""A small GGUF v3 writer for the tests: the reader's inputs are files written here from the format (ggml's gguf
layout: header, typed key/value pairs, tensor infos, data aligned to general.alignment), since no model file is on
this machine."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write(path, kv, tensors, alignment=None):
    """kv: [(key, type, value)] (an ARRAY value is (element type, items)); tensors: [(name, ggml type, shape in ggml
    order, uint8 bytes)]. alignment: written as general.alignment when given (the reader's default is 32)."""
    align = 32 if alignment is None else alignment
    kv = list(kv) + ([("general.alignment", U32, alignment)] if alignment is not None else [])
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off += (len(data) + align - 1) // align * align
    for (name, t, shape, _), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", t, o)
    head += b"\0" * ((-len(head)) % align)
    with open(path, "wb") as f:
        f.write(head)
        for (_, _, _, data), o in zip(tensors, offs):
            b = np.ascontiguousarray(data, dtype=np.uint8).tobytes()
            f.write(b + b"\0" * ((len(b) + align - 1) // align * align - len(b)))
