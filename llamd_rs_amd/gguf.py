"""GGUF model files: the Python face of the library's reader.

Mirrors crates/llamd-gguf/src/lib.rs (``Gguf::open``, ``get``,
``architecture``, ``tensor``, ``tensor_data``) and the upload side of
crates/llamd-runtime/src/device.rs:224-256 (Q6_K tensors go to the device
verbatim, re-tiled, never dequantized). Parsing and validation happen in the
C++ reader (csrc/host/gguf.cpp); this module decodes its answers.

    g = Gguf("model.gguf")
    g.architecture(), g.get("qwen3moe.expert_used_count")
    t = g.tensor("blk.0.ffn_gate_exps.weight"); raw = g.tensor_data(t)
    w = g.upload_q6k("output.weight")          # rocm.DeviceWeights
    layer = g.moe_layer(0)                     # rocm.MoeLayer

Errors: a malformed or hostile file raises HipError with the reader's reason
(the reference's Error::malformed / Error::unsupported texts).
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from ._lib import HipError, check, check_ptr, lib

# gguf_type (ggml/include/gguf.h), as lib.rs:36-53 mirrors it
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
_SIZE = {U8: 1, I8: 1, U16: 2, I16: 2, U32: 4, I32: 4, F32: 4, BOOL: 1, U64: 8, I64: 8, F64: 8}

# ggml_type of the tensors the path reads (crates/llamd-quant/src/lib.rs:47-52)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q6K = 0, 1, 8, 14


@dataclass
class TensorInfo:
    """lib.rs:99-114. dims in ggml order: dims[0] varies fastest."""
    name: str
    dims: list
    ggml_type: int
    offset: int     # from the start of the data section

    def elems(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


class Gguf:
    def __init__(self, path):
        self._h = check_ptr(lib().llamd_gguf_open(str(Path(path)).encode()), "gguf open")
        v, nt, nkv, al, do, fs = (C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64(),
                                  C.c_uint64(), C.c_uint64())
        check(lib().llamd_gguf_header(self._h, C.byref(v), C.byref(nt), C.byref(nkv), C.byref(al),
                                      C.byref(do), C.byref(fs)), "gguf header")
        self.version, self.alignment, self.data_offset = v.value, al.value, do.value
        self._size = fs.value
        self.metadata = {}
        for i in range(nkv.value):
            key, val = self._kv(i)
            self.metadata[key] = val
        self.tensors = [self._tensor(i) for i in range(nt.value)]

    # -- decoding -------------------------------------------------------------
    def _str(self, i, elem=0) -> str:
        n = C.c_uint64()
        check(lib().llamd_gguf_kv_str(self._h, i, elem, None, 0, C.byref(n)), "gguf string")
        buf = C.create_string_buffer(n.value + 1)
        check(lib().llamd_gguf_kv_str(self._h, i, elem, buf, n.value + 1, None), "gguf string")
        # lossy on purpose, as the reference (lib.rs:324-331)
        return buf.raw[: n.value].decode("utf-8", errors="replace")

    def _num(self, i, t, elem=0):
        bits = C.c_uint64()
        check(lib().llamd_gguf_kv_bits(self._h, i, elem, C.byref(bits)), "gguf value")
        raw = struct.pack("<Q", bits.value)[: _SIZE[t]]
        return struct.unpack(_FMT[t], raw)[0]

    def _kv(self, i):
        key = C.create_string_buffer(65536)
        t, at, n = C.c_uint32(), C.c_uint32(), C.c_uint64()
        check(lib().llamd_gguf_kv(self._h, i, key, len(key), C.byref(t), C.byref(at), C.byref(n)),
              "gguf kv")
        k = key.value.decode("utf-8", errors="replace")
        if t.value == STRING:
            return k, self._str(i)
        if t.value == ARRAY:
            if at.value == STRING:
                return k, [self._str(i, j) for j in range(n.value)]
            return k, [self._num(i, at.value, j) for j in range(n.value)]
        return k, self._num(i, t.value)

    def _tensor(self, i) -> TensorInfo:
        name = C.create_string_buffer(65536)
        nd, ty, off = C.c_uint32(), C.c_uint32(), C.c_uint64()
        dims = (C.c_uint64 * 4)()
        check(lib().llamd_gguf_tensor(self._h, i, name, len(name), C.byref(nd), dims, C.byref(ty),
                                      C.byref(off)), "gguf tensor")
        return TensorInfo(name.value.decode("utf-8", errors="replace"),
                          [int(dims[d]) for d in range(nd.value)], ty.value, off.value)

    # -- the reference's accessors -------------------------------------------
    def get(self, key: str):
        return self.metadata.get(key)

    def architecture(self):
        v = self.metadata.get("general.architecture")
        return v if isinstance(v, str) else None

    def tensor(self, name: str):
        for t in self.tensors:
            if t.name == name:
                return t
        return None

    def file_size(self) -> int:
        return self._size

    def tensor_data(self, t: TensorInfo) -> np.ndarray:
        """The tensor's bytes, borrowed from the mapping (no copy; read-only;
        valid until close())."""
        i = lib().llamd_gguf_find_tensor(self._h, t.name.encode())
        if i < 0:
            raise HipError(f"gguf: tensor {t.name} is absent")
        n = C.c_uint64()
        p = check_ptr(lib().llamd_gguf_tensor_data(self._h, i, C.byref(n)), "gguf tensor_data")
        a = np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p))
        a.flags.writeable = False
        return a

    # -- device ----------------------------------------------------------------
    def upload_q6k(self, name: str):
        """A Q6_K tensor on the device (2D: one matrix; 3D: n_expert matrices)."""
        from . import rocm
        t = self.tensor(name)
        if t is None:
            raise HipError(f"gguf: tensor {name} is absent")
        h = check_ptr(lib().llamd_gguf_upload_q6k(self._h, name.encode()), "gguf upload")
        ne = t.dims[2] if len(t.dims) == 3 else 1
        return rocm.DeviceWeights(h, t.dims[1], t.dims[0] // 256, ne)

    def moe_layer(self, layer: int):
        """blk.<layer>'s MoE FFN as a rocm.MoeLayer."""
        from . import rocm
        h = check_ptr(lib().llamd_gguf_moe_create(self._h, layer), "gguf moe layer")
        r = self.tensor(f"blk.{layer}.ffn_gate_inp.weight")
        g = self.tensor(f"blk.{layer}.ffn_gate_exps.weight")
        n_used = self.get(f"{self.architecture()}.expert_used_count")
        return rocm.MoeLayer.from_handle(h, r.dims[0], g.dims[1], r.dims[1], n_used)

    def close(self):
        if self._h:
            lib().llamd_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
