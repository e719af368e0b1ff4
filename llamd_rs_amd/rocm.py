"""Python mirror of the reference's llamd-rocm safe wrappers, over the C ABI.

Names, argument meaning and error behaviour follow
crates/llamd-rocm/src/lib.rs so that tests read like the reference's own
(crates/llamd-testing/tests/grouped_expert.rs, rocm_oracle.rs, planar.rs):

  available(), device_count(), device_info(i)          lib.rs:167-257
  DeviceWeights.upload(w, rows, blocks)                lib.rs:277-308
      .matvec(act)                                     lib.rs:319-375
      .matvec_grouped(act, ids, rows)                  lib.rs:434-511
      .bench_kernel_only(act, iters)                   lib.rs:378-431
  quantize_q8k_on_device(x)                            lib.rs:569-623
  matvec_q6k(w, act, rows)                             lib.rs:914-
plus the pieces of llamd-models / llamd-runtime this backend puts on the
device: route (moe.rs:73-113), MoeLayer (layer.rs:230-260 + the router), and
LmHead (the output matvec + argmax).

Validation happens before any device call; a bad argument raises ValueError
(the Rust wrappers' Error::Shape / Error::Other) and a failing C call raises
HipError. There is no CPU fallback anywhere in this module.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np

from ._lib import HipError, HipUnavailable, check, check_ptr, lib

QK_K = 256
Q6K_BLOCK_BYTES = 210


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


@dataclass
class BlockQ8K:
    """Q8_K activations as arrays: d [nb] f32, qs [nb,256] i8, bsums [nb,16] i16
    (crates/llamd-quant/src/dot.rs:52-62)."""
    d: np.ndarray
    qs: np.ndarray
    bsums: np.ndarray

    @property
    def nblocks(self) -> int:
        return self.d.shape[0]


def device_count() -> int:
    return int(lib().llamd_rocm_device_count())


def available() -> bool:
    try:
        return device_count() > 0
    except (HipUnavailable, OSError):
        return False


@dataclass
class DeviceInfo:
    name: str
    arch: str
    total_mem: int
    compute_units: int
    wave_size: int


def device_info(index: int = 0) -> DeviceInfo:
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(64)
    mem = C.c_size_t()
    cus = C.c_int()
    wave = C.c_int()
    check(lib().llamd_rocm_device_info(index, name, 256, arch, 64, C.byref(mem), C.byref(cus),
                                       C.byref(wave)), "device_info")
    return DeviceInfo(name.value.decode(), arch.value.decode(), mem.value, cus.value, wave.value)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def quantize_q8k_on_device(x) -> BlockQ8K:
    x = _f32(x)
    if x.size % QK_K:
        raise ValueError("Q8_K quantizes whole 256-element blocks")
    nb = x.size // QK_K
    qs = np.empty((nb, QK_K), np.int8)
    d = np.empty(nb, np.float32)
    bs = np.empty((nb, 16), np.int16)
    check(lib().llamd_rocm_quantize_q8k(_ptr(x), nb, _ptr(qs), _ptr(d), _ptr(bs)), "quantize_q8k")
    return BlockQ8K(d, qs, bs)


def swiglu_q8k_on_device(gate, up) -> tuple[np.ndarray, BlockQ8K]:
    """act = silu(gate) * up (CpuBackend::silu/mul) and its Q8_K, fused."""
    g, u = _f32(gate), _f32(up)
    if g.shape != u.shape or g.size % QK_K:
        raise ValueError("gate/up must match and be whole 256-element blocks")
    nb = g.size // QK_K
    act = np.empty(g.size, np.float32)
    qs = np.empty((nb, QK_K), np.int8)
    d = np.empty(nb, np.float32)
    bs = np.empty((nb, 16), np.int16)
    check(lib().llamd_hip_swiglu_q8k(_ptr(g), _ptr(u), nb, _ptr(act), _ptr(qs), _ptr(d), _ptr(bs)),
          "swiglu_q8k")
    return act, BlockQ8K(d, qs, bs)


def _act_arrays(act: BlockQ8K | list[BlockQ8K]):
    if isinstance(act, BlockQ8K):
        return np.ascontiguousarray(act.qs, np.int8), np.ascontiguousarray(act.d, np.float32), 1
    qs = np.ascontiguousarray(np.concatenate([a.qs for a in act]), np.int8)
    d = np.ascontiguousarray(np.concatenate([a.d for a in act]), np.float32)
    return qs, d, len(act)


class DeviceWeights:
    """A Q6_K matrix resident on the device, in the tiled layout.

    Owns its allocation; released exactly once (close() or garbage collection),
    like the Rust handle's Drop (crates/llamd-rocm/src/lib.rs:896-907)."""

    def __init__(self, ptr, rows: int, blocks: int, n_expert: int = 1):
        self._ptr = ptr
        self._rows = rows
        self._blocks = blocks
        self._n_expert = n_expert

    @classmethod
    def upload(cls, w, rows: int, blocks: int) -> "DeviceWeights":
        w = np.ascontiguousarray(np.frombuffer(bytes(w), np.uint8) if isinstance(w, (bytes, bytearray))
                                 else w, dtype=np.uint8)
        if rows <= 0 or blocks <= 0:
            raise ValueError("rows and blocks must be positive")
        need = rows * blocks * Q6K_BLOCK_BYTES
        if w.size < need:
            raise ValueError(f"need {need} bytes for {rows}x{blocks} Q6_K blocks, have {w.size}")
        p = check_ptr(lib().llamd_rocm_upload_q6k(_ptr(w), rows, blocks), "upload_q6k")
        return cls(p, rows, blocks)

    @classmethod
    def upload_experts(cls, w, n_expert: int, rows: int, blocks: int) -> "DeviceWeights":
        w = np.ascontiguousarray(w, dtype=np.uint8)
        need = n_expert * rows * blocks * Q6K_BLOCK_BYTES
        if w.size < need:
            raise ValueError(f"need {need} bytes, have {w.size}")
        p = check_ptr(lib().llamd_rocm_upload_q6k_experts(_ptr(w), n_expert, rows, blocks),
                      "upload_q6k_experts")
        return cls(p, rows, blocks, n_expert)

    @property
    def ptr(self):
        return self._ptr

    def rows(self) -> int:
        return self._rows

    def blocks(self) -> int:
        return self._blocks

    def _check_act(self, act: BlockQ8K):
        if act.nblocks < self._blocks:
            raise ValueError(f"activation has {act.nblocks} blocks, weights need {self._blocks}")

    def matvec(self, act: BlockQ8K) -> np.ndarray:
        self._check_act(act)
        qs, d, _ = _act_arrays(act)
        rows = self._rows
        out = np.empty(rows, np.float32)
        check(lib().llamd_rocm_matvec_q6k_resident(self._ptr, _ptr(qs), _ptr(d), _ptr(out),
                                                   self._blocks, rows), "matvec")
        return out

    def matvec_grouped(self, act: BlockQ8K, ids, rows: int) -> np.ndarray:
        """out[e*rows + r] = row r of expert ids[e] against one shared activation."""
        self._check_act(act)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if ids.size == 0 or rows <= 0:
            raise ValueError("no experts / zero rows")
        qs, d, _ = _act_arrays(act)
        out = np.empty(rows * ids.size, np.float32)
        check(lib().llamd_rocm_matvec_grouped(self._ptr, _ptr(ids), _ptr(qs), _ptr(d), _ptr(out),
                                              self._blocks, rows, ids.size), "matvec_grouped")
        return out

    def matvec_grouped_pa(self, acts: list[BlockQ8K], ids, rows: int) -> np.ndarray:
        """Like matvec_grouped, slot e with its own activation acts[e]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if len(acts) != ids.size or ids.size == 0:
            raise ValueError("one activation per routed expert")
        for a in acts:
            self._check_act(a)
        qs, d, _ = _act_arrays(acts)
        out = np.empty(rows * ids.size, np.float32)
        check(lib().llamd_hip_matvec_grouped_pa(self._ptr, _ptr(ids), _ptr(qs), _ptr(d), _ptr(out),
                                                self._blocks, rows, ids.size), "matvec_grouped_pa")
        return out

    def matvec_batched(self, acts: list[BlockQ8K]) -> np.ndarray:
        """out[s, r] for every activation s; weights read once per 16."""
        for a in acts:
            self._check_act(a)
        qs, d, n = _act_arrays(acts)
        out = np.empty((n, self._rows), np.float32)
        check(lib().llamd_hip_matvec_q6k_batched(self._ptr, _ptr(qs), _ptr(d), _ptr(out),
                                                 self._blocks, self._rows, n), "matvec_batched")
        return out

    def dequantize(self) -> np.ndarray:
        if self._n_expert != 1:
            raise ValueError("dequantize one matrix at a time")
        out = np.empty((self._rows, self._blocks * QK_K), np.float32)
        check(lib().llamd_hip_dequant_q6k(self._ptr, self._rows, self._blocks, _ptr(out)),
              "dequant_q6k")
        return out

    def bench_kernel_only(self, act: BlockQ8K, iters: int) -> float:
        qs, d, _ = _act_arrays(act)
        ms = C.c_float()
        check(lib().llamd_rocm_matvec_bench(self._ptr, _ptr(qs), _ptr(d), self._blocks, self._rows,
                                            iters, C.byref(ms)), "matvec_bench")
        return ms.value

    def close(self):
        if self._ptr:
            lib().llamd_rocm_release(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Q8_0Weights:
    """A Q8_0 matrix resident on the device (planar layout)."""

    def __init__(self, w, rows: int, k: int):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        if k % 32 or w.size < rows * k // 32 * 34:
            raise ValueError("Q8_0 needs whole 32-element blocks")
        self._ptr = check_ptr(lib().llamd_hip_upload_q8_0(_ptr(w), rows, k), "upload_q8_0")
        self.rows, self.k = rows, k

    def matvec(self, x) -> np.ndarray:
        x = _f32(x)
        if x.size != self.k:
            raise ValueError(f"expected {self.k} activations, got {x.size}")
        out = np.empty(self.rows, np.float32)
        check(lib().llamd_hip_matvec_q8_0(self._ptr, _ptr(x), _ptr(out), self.rows, self.k),
              "matvec_q8_0")
        return out

    def dequantize(self) -> np.ndarray:
        out = np.empty((self.rows, self.k), np.float32)
        check(lib().llamd_hip_dequant_q8_0(self._ptr, self.rows, self.k, _ptr(out)), "dequant_q8_0")
        return out

    def close(self):
        if self._ptr:
            lib().llamd_rocm_release(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matvec_q6k(w, act: BlockQ8K, rows: int) -> np.ndarray:
    """Upload, multiply, release (crates/llamd-rocm/src/lib.rs:914-)."""
    blocks = act.nblocks
    dw = DeviceWeights.upload(w, rows, blocks)
    try:
        return dw.matvec(act)
    finally:
        dw.close()


@dataclass
class Routing:
    experts: np.ndarray   # int32 [n_used], best first
    weights: np.ndarray   # f32 [n_used], renormalised


def route(logits, n_used: int) -> Routing:
    """crates/llamd-models/src/moe.rs:73-113 on the device."""
    lg = _f32(logits)
    if n_used == 0 or n_used > lg.size:
        raise ValueError(f"{n_used} experts requested of {lg.size}")
    ids = np.empty(n_used, np.int32)
    w = np.empty(n_used, np.float32)
    check(lib().llamd_hip_route(_ptr(lg), lg.size, n_used, _ptr(ids), _ptr(w)), "route")
    return Routing(ids, w)


def argmax(x) -> np.ndarray:
    """Row-wise argmax, lowest index on ties."""
    x = np.atleast_2d(_f32(x))
    ids = np.empty(x.shape[0], np.int32)
    check(lib().llamd_hip_argmax(_ptr(x), x.shape[1], x.shape[0], _ptr(ids)), "argmax")
    return ids


class MoeLayer:
    """One MoE FFN (router -> route -> experts -> combine) resident on the device.

    router: f32 [n_expert, n_embd]; gate/up: ggml Q6_K bytes of
    [n_expert][n_ff][n_embd]; down: [n_expert][n_embd][n_ff]."""

    EXACT = 1

    def __init__(self, router, gate, up, down, n_embd: int, n_ff: int, n_expert: int, n_used: int):
        router = _f32(router)
        gate, up, down = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
        if router.size != n_expert * n_embd:
            raise ValueError("router must be [n_expert, n_embd]")
        per = n_ff * n_embd // QK_K * Q6K_BLOCK_BYTES
        if gate.size < n_expert * per or up.size < n_expert * per or down.size < n_expert * per:
            raise ValueError("expert tensors are short")
        self.n_embd, self.n_ff, self.n_expert, self.n_used = n_embd, n_ff, n_expert, n_used
        self._h = check_ptr(lib().llamd_hip_moe_create(_ptr(router), _ptr(gate), _ptr(up), _ptr(down),
                                                       n_embd, n_ff, n_expert, n_used), "moe_create")

    @classmethod
    def from_handle(cls, h, n_embd: int, n_ff: int, n_expert: int, n_used: int) -> "MoeLayer":
        """Wrap a layer the library built elsewhere (e.g. llamd_gguf_moe_create)."""
        m = cls.__new__(cls)
        m.n_embd, m.n_ff, m.n_expert, m.n_used = n_embd, n_ff, n_expert, n_used
        m._h = check_ptr(h, "moe layer")
        return m

    @property
    def handle(self):
        return self._h

    def forward(self, x, res=None, exact: bool = True):
        """Returns (out, Routing, logits). out = res + moe_ffn(x) (res optional).
        Every call is bit-exact; `exact` is accepted for older callers."""
        x = _f32(x)
        if x.size != self.n_embd:
            raise ValueError("x must be [n_embd]")
        r = None if res is None else _f32(res)
        out = np.empty(self.n_embd, np.float32)
        ids = np.empty(self.n_used, np.int32)
        w = np.empty(self.n_used, np.float32)
        lg = np.empty(self.n_expert, np.float32)
        check(lib().llamd_hip_moe_forward_host(self._h, _ptr(x), _ptr(r), _ptr(out), _ptr(ids),
                                               _ptr(w), _ptr(lg), self.EXACT if exact else 0),
              "moe_forward")
        return out, Routing(ids, w), lg

    def forward_batch(self, x, res=None):
        """nseq sequences at once, each routed by its own logits; returns
        (out [nseq, n_embd], ids [nseq, n_used], weights [nseq, n_used],
        logits [nseq, n_expert]). Bit-identical to forward() per row."""
        x = _f32(x).reshape(-1, self.n_embd)
        nseq = x.shape[0]
        r = None if res is None else _f32(res).reshape(nseq, self.n_embd)
        out = np.empty((nseq, self.n_embd), np.float32)
        ids = np.empty((nseq, self.n_used), np.int32)
        w = np.empty((nseq, self.n_used), np.float32)
        lg = np.empty((nseq, self.n_expert), np.float32)
        check(lib().llamd_hip_moe_forward_batch_host(self._h, _ptr(x), _ptr(r), _ptr(out), _ptr(ids),
                                                     _ptr(w), _ptr(lg), nseq), "moe_forward_batch")
        return out, ids, w, lg

    def prefill(self, x, ids, weights, reduction: bool = False) -> np.ndarray:
        """moe_ffn for n_tok tokens with the given routing [n_tok, n_used].
        reduction=True: the REDUCTION-tolerance GEMMs (LLAMD_HIP_REDUCTION);
        otherwise bit-identical to the CPU path."""
        x = _f32(x).reshape(-1, self.n_embd)
        n_tok = x.shape[0]
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(n_tok, self.n_used)
        w = _f32(weights).reshape(n_tok, self.n_used)
        out = np.empty((n_tok, self.n_embd), np.float32)
        check(lib().llamd_hip_moe_prefill_host_ex(self._h, _ptr(x), _ptr(ids), _ptr(w), _ptr(out), n_tok,
                                                  1 if reduction else 0), "moe_prefill")
        return out

    def stats(self) -> tuple[int, int]:
        a, b = C.c_int(), C.c_int()
        check(lib().llamd_hip_moe_stats(self._h, C.byref(a), C.byref(b)), "moe_stats")
        return a.value, b.value

    def counters(self) -> tuple[np.ndarray, np.ndarray]:
        """([calls, exact calls, certified calls, wait timed out], the last
        call's logit estimates T [n_expert] and bounds E [n_expert])."""
        c = np.zeros(4, np.int32)
        est = np.zeros(2 * self.n_expert, np.float64)
        check(lib().llamd_hip_moe_counters(self._h, c.ctypes.data_as(C.POINTER(C.c_int)), _ptr(est)),
              "moe_counters")
        return c, est.reshape(2, self.n_expert)

    def close(self):
        if self._h:
            lib().llamd_hip_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """Raw device memory on the library's allocator (for device-pointer calls)."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = check_ptr(lib().llamd_fwd_alloc(nbytes), "alloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than buffer")
        check(lib().llamd_fwd_upload(self.ptr, _ptr(a), a.nbytes), "upload")

    def download(self, a: np.ndarray) -> np.ndarray:
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than buffer")
        check(lib().llamd_fwd_download(_ptr(a), self.ptr, a.nbytes), "download")
        return a

    def close(self):
        if self.ptr:
            lib().llamd_fwd_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LmHead:
    """Q6_K output projection + argmax over the vocabulary."""

    def __init__(self, weights: DeviceWeights, max_seq: int = 16):
        self.w = weights
        self.rows, self.blocks, self.max_seq = weights.rows(), weights.blocks(), max_seq
        self._h = check_ptr(lib().llamd_hip_lmhead_create(weights.ptr, self.rows, self.blocks, max_seq),
                            "lmhead_create")
        self._x = DeviceBuffer(max_seq * self.blocks * QK_K * 4)
        self._logits = DeviceBuffer(max_seq * self.rows * 4)
        self._ids = DeviceBuffer(max_seq * 4)

    @property
    def handle(self):
        return self._h

    def forward(self, x, reduction: bool = False) -> tuple[np.ndarray, np.ndarray]:
        """logits [nseq, rows] and arg-max ids [nseq]. reduction=True
        (LLAMD_HIP_REDUCTION, nseq > 1): logits within REDUCTION, ids still
        the exact logits' arg-max."""
        x = np.atleast_2d(_f32(x))
        nseq = x.shape[0]
        if x.shape[1] != self.blocks * QK_K or nseq > self.max_seq:
            raise ValueError("x must be [nseq <= max_seq, k]")
        self._x.upload(x)
        check(lib().llamd_hip_lmhead_forward_ex(self._h, self._x.ptr, nseq, self._logits.ptr, self._ids.ptr,
                                                1 if reduction else 0), "lmhead_forward")
        logits = self._logits.download(np.empty((nseq, self.rows), np.float32))
        ids = self._ids.download(np.empty(nseq, np.int32))
        return logits, ids

    def close(self):
        if self._h:
            lib().llamd_hip_lmhead_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = [
    "BlockQ8K", "DeviceInfo", "DeviceWeights", "Q8_0Weights", "MoeLayer", "LmHead", "Routing",
    "DeviceBuffer", "available", "device_count", "device_info", "quantize_q8k_on_device",
    "swiglu_q8k_on_device", "matvec_q6k", "route", "argmax", "HipError", "HipUnavailable",
]


class _PinnedPool:
    """Page-locked host buffers of one size (hipHostMalloc), handed out as
    numpy arrays and taken back when an array is collected. A device-to-host
    copy into page-locked memory is one DMA, without the bounce buffer a
    pageable destination goes through (608 KB of logits: ~48 us -> ~12 us)."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self._free = []
        self._closed = False
        hip = C.CDLL("libamdhip64.so.7")   # already loaded by the library
        self._malloc = hip.hipHostMalloc
        self._malloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t, C.c_uint]
        self._malloc.restype = C.c_int
        self._hfree = hip.hipHostFree
        self._hfree.argtypes = [C.c_void_p]
        self._hfree.restype = C.c_int

    def _put(self, ptr):
        if self._closed:
            self._hfree(ptr)
        else:
            self._free.append(ptr)

    def array(self, n: int, dtype) -> np.ndarray:
        if self._free:
            ptr = self._free.pop()
        else:
            p = C.c_void_p()
            if self._malloc(C.byref(p), self.nbytes, 0) != 0 or not p.value:
                raise HipError("hipHostMalloc failed")
            ptr = p.value
        arr = np.frombuffer((C.c_char * self.nbytes).from_address(ptr), dtype=dtype, count=n)
        fin = weakref.finalize(arr, self._put, ptr)
        fin.atexit = False  # at interpreter exit the process's pages go with it
        return arr

    def close(self):
        self._closed = True
        while self._free:
            self._hfree(self._free.pop())


class DeviceModel:
    """A resident Qwen3-MoE decode loop from a GGUF (DeviceModel::load /
    forward, crates/llamd-runtime/src/device.rs:262-722): weights uploaded
    once, KV cache for max_kv positions, one synchronisation per token."""

    def __init__(self, gguf, max_kv: int):
        self._h = check_ptr(lib().llamd_hip_model_create(gguf._h, max_kv), "model_create")
        a, b, c, d = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        check(lib().llamd_hip_model_info(self._h, C.byref(a), C.byref(b), C.byref(c), C.byref(d)),
              "model_info")
        self.n_layer, self.n_embd, self.n_vocab, self.max_kv = a.value, b.value, c.value, d.value
        self._pinned = _PinnedPool(self.n_vocab * 4)

    def forward(self, token: int, pos: int):
        """(logits [n_vocab], next token = argmax) for `token` at `pos`. The
        logits live in page-locked host memory (returned to a pool when the
        array is collected)."""
        logits = self._pinned.array(self.n_vocab, np.float32)
        nxt = np.zeros(1, np.int32)
        check(lib().llamd_hip_model_forward(self._h, int(token), int(pos), _ptr(logits), _ptr(nxt)),
              "model_forward")
        return logits, int(nxt[0])

    def close(self):
        if self._h:
            lib().llamd_hip_model_destroy(self._h)
            self._h = None
        if getattr(self, "_pinned", None) is not None:
            self._pinned.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
