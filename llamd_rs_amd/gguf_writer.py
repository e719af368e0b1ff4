"""A small GGUF v3 writer (ggml/include/gguf.h layout).

For synthetic models: the tests write files whose every byte they know (and
the malformed headers the reader must refuse), and bench.py writes a
Qwen3-30B-A3B-shaped model whose layers share one copy of their data (tensor
infos may point at the same offset: a data object passed twice, the same
Python object, is stored once).
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        inner, items = v
        return struct.pack("<IQ", inner, len(items)) + b"".join(value(inner, x) for x in items)
    return struct.pack(_FMT[t], v)


def _bytes(data):
    """bytes-like view of a tensor's data (numpy arrays as their raw bytes)."""
    if hasattr(data, "dtype"):
        import numpy as np
        return memoryview(np.ascontiguousarray(data)).cast("B")
    return memoryview(data).cast("B")


def _layout(kvs, tensors, alignment, version, magic, n_kv, n_tensors):
    head = magic + struct.pack("<IQQ", version,
                               len(tensors) if n_tensors is None else n_tensors,
                               len(kvs) if n_kv is None else n_kv)
    body = b"".join(gstr(k) + struct.pack("<I", t) + value(t, v) for k, t, v in kvs)
    infos, datas, off, placed = [], [], 0, {}
    for name, dims, ty, data in tensors:
        at = placed.get(id(data))
        if at is None:
            mv = _bytes(data)
            off = -(-off // alignment) * alignment
            at = placed[id(data)] = off
            datas.append((off, mv))
            off += len(mv)
        infos.append(gstr(name) + struct.pack("<I", len(dims)) +
                     b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, at))
    header = head + body + b"".join(infos)
    return header + b"\0" * (-len(header) % alignment), datas, off


def build(kvs, tensors, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF",
          n_kv=None, n_tensors=None, tail: bytes = b"") -> bytes:
    """kvs: [(key, type, value)] (arrays: value = (inner_type, [items]));
    tensors: [(name, dims, ggml_type, data)] with data bytes or a numpy array,
    laid out in order, each at the next multiple of `alignment` from the data
    section's start."""
    header, datas, size = _layout(kvs, tensors, alignment, version, magic, n_kv, n_tensors)
    section = bytearray(size)
    for o, d in datas:
        section[o:o + len(d)] = d
    return header + bytes(section) + tail


def write(path, kvs, tensors, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF",
          n_kv=None, n_tensors=None, tail: bytes = b"") -> None:
    """build(), streamed to the file (no copy of the data section in memory)."""
    header, datas, size = _layout(kvs, tensors, alignment, version, magic, n_kv, n_tensors)
    with open(path, "wb") as f:
        f.write(header)
        pos = 0
        for o, d in datas:
            f.write(b"\0" * (o - pos))
            f.write(d)
            pos = o + len(d)
        f.write(b"\0" * (size - pos))
        f.write(tail)
