"""A minimal GGUF v3 writer for tests, from the published GGUF layout: magic "GGUF", version, tensor count, key-value
count, key-values (key string, value type, value), tensor infos (name, n_dims, dims innermost first, type, offset),
padding to general.alignment, then the tensor data (each tensor aligned). Strings are u64 length + bytes."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
        F64: "<d"}


def _s(x):
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def _value(t, v, et=None):
    if t == STR:
        return _s(v)
    if t == ARR:
        out = struct.pack("<IQ", et, len(v))
        for x in v:
            out += _s(x) if et == STR else struct.pack(_FMT[et], x)
        return out
    return struct.pack(_FMT[t], v)


def write_gguf(path, kvs, tensors, alignment=32, version=3):
    """kvs: [(key, type, value[, elem_type])]; tensors: [(name, ggml_type, dims (innermost first), bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for kv in kvs:
        key, t, v = kv[:3]
        head += _s(key) + struct.pack("<I", t) + _value(t, v, kv[3] if len(kv) > 3 else None)
    offs, off = [], 0
    for name, gt, dims, data in tensors:
        offs.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, gt, dims, data), o in zip(tensors, offs):
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gt, o)
    head += b"\0" * ((-len(head)) % alignment)
    body = bytearray(off)
    for (name, gt, dims, data), o in zip(tensors, offs):
        body[o:o + len(data)] = bytes(np.asarray(data, dtype=np.uint8).tobytes() if not isinstance(data, bytes) else data)
    with open(path, "wb") as f:
        f.write(head + bytes(body))
    return len(head)
