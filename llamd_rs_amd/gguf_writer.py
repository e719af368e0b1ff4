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


def build(kvs, tensors, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF",
          n_kv=None, n_tensors=None, tail: bytes = b"") -> bytes:
    """kvs: [(key, type, value)] (arrays: value = (inner_type, [items]));
    tensors: [(name, dims, ggml_type, data_bytes)], laid out in order, each
    at the next multiple of `alignment` from the data section's start."""
    head = magic + struct.pack("<IQQ", version,
                               len(tensors) if n_tensors is None else n_tensors,
                               len(kvs) if n_kv is None else n_kv)
    body = b"".join(gstr(k) + struct.pack("<I", t) + value(t, v) for k, t, v in kvs)
    infos, datas, off, placed = [], [], 0, {}
    for name, dims, ty, data in tensors:
        at = placed.get(id(data))
        if at is None:
            off = -(-off // alignment) * alignment
            at = placed[id(data)] = off
            datas.append((off, data))
            off += len(data)
        infos.append(gstr(name) + struct.pack("<I", len(dims)) +
                     b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, at))
    header = head + body + b"".join(infos)
    pad = -len(header) % alignment
    section = bytearray(off)
    for o, d in datas:
        section[o:o + len(d)] = d
    return header + b"\0" * pad + bytes(section) + tail


def write(path, *args, **kw) -> None:
    with open(path, "wb") as f:
        f.write(build(*args, **kw))
