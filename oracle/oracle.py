"""ctypes wrapper of the CPU oracle (oracle/libllamd_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and only as the checker / CPU baseline -- never
by llamd_rs_amd. See llamd_oracle.h for what each function restates.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libllamd_oracle.so"
QK_K = 256

EXACT = 0.0
F32_ULP = 1.2e-7
REDUCTION = 1e-5
QUANTIZED_MATMUL = 1e-3
QUANTIZED_LAYER = 5e-3
ATTENTION = 1e-5
LAYER = 1e-4
LOGITS = 2e-3

_L = None


def _lib():
    global _L
    if _L is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        vp, sz, u32, f = C.c_void_p, C.c_size_t, C.c_uint32, C.c_float
        sig = {
            "orc_f16_to_f32": (f, [C.c_uint16]),
            "orc_bytes_for": (C.c_longlong, [u32, sz]),
            "orc_dequantize": (C.c_int, [u32, vp, sz, sz, vp]),
            "orc_nearest_int": (C.c_int32, [f]),
            "orc_quantize_q8_k": (C.c_int, [vp, sz, vp, vp, vp]),
            "orc_dot_q6k_q8k": (f, [vp, vp, vp, sz]),
            "orc_matvec_q6k_act": (None, [vp, sz, sz, vp, vp, vp]),
            "orc_matvec_q6k_act_mt": (C.c_int, [vp, sz, sz, vp, vp, vp, C.c_int]),
            "orc_matvec_q6k": (C.c_int, [vp, sz, sz, vp, vp]),
            "orc_matvec_f32": (None, [vp, sz, sz, vp, vp]),
            "orc_matvec_q8_0": (C.c_int, [vp, sz, sz, vp, vp]),
            "orc_route": (C.c_int, [vp, sz, sz, vp, vp, vp, vp]),
            "orc_silu": (None, [vp, vp, sz]),
            "orc_rms_norm": (None, [vp, C.c_int, C.c_int, C.c_float, vp]),
            "orc_mul": (None, [vp, vp, vp, sz]),
            "orc_softmax": (None, [vp, vp, sz]),
            "orc_matvec_expert_q6k": (C.c_int, [vp, sz, sz, sz, sz, vp, vp]),
            "orc_moe_ffn": (C.c_int, [vp, sz, sz, sz, vp, vp, vp, vp, vp, sz, vp]),
            "orc_moe_layer": (C.c_int, [vp, vp, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp, vp, vp]),
            "orc_argmax": (u32, [vp, sz]),
            "orc_moe_ffn_tokens": (C.c_int, [vp, sz, sz, sz, sz, vp, vp, vp, vp, vp, sz, vp]),
            "orc_close": (C.c_int, [f, f, f]),
            "orc_rope": (None, [vp, C.c_int, C.c_int, u32, f]),
            "orc_attend": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp]),
        }
        for n, (r, a) in sig.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = r, a
        _L = L
    return _L


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def _u8(a):
    return np.ascontiguousarray(a, np.uint8)


def f16_to_f32(h: int) -> float:
    return _lib().orc_f16_to_f32(h)


def bytes_for(ty: int, n: int) -> int:
    return _lib().orc_bytes_for(ty, n)


def dequantize(ty: int, src, n: int) -> np.ndarray:
    src = _u8(src)
    out = np.empty(n, np.float32)
    if _lib().orc_dequantize(ty, _p(src), src.size, n, _p(out)):
        raise ValueError("malformed quantized data")
    return out


def nearest_int(v: float) -> int:
    return _lib().orc_nearest_int(v)


class Q8K:
    def __init__(self, d, qs, bsums):
        self.d, self.qs, self.bsums = d, qs, bsums


def quantize_q8_k(x) -> Q8K:
    x = _f32(x).ravel()
    nb = x.size // QK_K
    d = np.empty(nb, np.float32)
    qs = np.empty((nb, QK_K), np.int8)
    bs = np.empty((nb, 16), np.int16)
    if _lib().orc_quantize_q8_k(_p(x), x.size, _p(d), _p(qs), _p(bs)):
        raise ValueError("Q8_K quantizes whole 256-element blocks")
    return Q8K(d, qs, bs)


def dot_q6k_q8k(w, a: Q8K, n: int) -> float:
    w = _u8(w)
    return _lib().orc_dot_q6k_q8k(_p(w), _p(_f32(a.d)), _p(np.ascontiguousarray(a.qs, np.int8)), n)


def matvec_q6k_act(w, rows: int, k: int, a: Q8K) -> np.ndarray:
    w = _u8(w)
    y = np.empty(rows, np.float32)
    _lib().orc_matvec_q6k_act(_p(w), rows, k, _p(_f32(a.d)), _p(np.ascontiguousarray(a.qs, np.int8)),
                              _p(y))
    return y


def matvec_q6k_act_mt(w, rows: int, k: int, a: Q8K, nthreads: int) -> tuple[np.ndarray, int]:
    """matvec_q6k_act over nthreads host threads (same bits): (y, threads used)."""
    w = _u8(w)
    y = np.empty(rows, np.float32)
    used = _lib().orc_matvec_q6k_act_mt(_p(w), rows, k, _p(_f32(a.d)),
                                        _p(np.ascontiguousarray(a.qs, np.int8)), _p(y), nthreads)
    return y, int(used)


def matvec_q6k(w, rows: int, k: int, x) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    y = np.empty(rows, np.float32)
    if _lib().orc_matvec_q6k(_p(w), rows, k, _p(x), _p(y)):
        raise ValueError("bad shape")
    return y


def matvec_f32(w, rows: int, k: int, x) -> np.ndarray:
    w, x = _f32(w), _f32(x)
    y = np.empty(rows, np.float32)
    _lib().orc_matvec_f32(_p(w), rows, k, _p(x), _p(y))
    return y


def matvec_q8_0(w, rows: int, k: int, x) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    y = np.empty(rows, np.float32)
    if _lib().orc_matvec_q8_0(_p(w), rows, k, _p(x), _p(y)):
        raise ValueError("bad shape")
    return y


class Routing:
    def __init__(self, experts, weights_raw, weight_sum, weights):
        self.experts, self.weights_raw = experts, weights_raw
        self.weight_sum, self.weights = weight_sum, weights


def route(logits, n_used: int) -> Routing:
    lg = _f32(logits)
    e = np.empty(max(n_used, 1), np.uint32)
    raw = np.empty(max(n_used, 1), np.float32)
    w = np.empty(max(n_used, 1), np.float32)
    s = C.c_float()
    if _lib().orc_route(_p(lg), lg.size, n_used, _p(e), _p(raw), C.byref(s), _p(w)):
        raise ValueError(f"{n_used} experts requested of {lg.size}")
    return Routing(e, raw, s.value, w)


def silu(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    _lib().orc_silu(_p(x), _p(y), x.size)
    return y


def rms_norm(x, rows: int, n: int, eps: float) -> np.ndarray:
    """CpuBackend::rms_norm (llamd-cpu/src/lib.rs:55-75) over `rows` rows of n."""
    x = _f32(x)
    if x.size != rows * n:
        raise ValueError("x must be [rows, n]")
    out = np.empty(rows * n, np.float32)
    _lib().orc_rms_norm(_p(x), rows, n, eps, _p(out))
    return out


def mul(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    y = np.empty_like(a)
    _lib().orc_mul(_p(a), _p(b), _p(y), a.size)
    return y


def softmax(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    _lib().orc_softmax(_p(x), _p(y), x.size)
    return y


def matvec_expert_q6k(w, n_expert, rows, k, expert, x) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    y = np.empty(rows, np.float32)
    if _lib().orc_matvec_expert_q6k(_p(w), n_expert, rows, k, expert, _p(x), _p(y)):
        raise ValueError("bad expert")
    return y


def moe_ffn(x, n_embd, n_ff, n_expert, gate, up, down, experts, weights) -> np.ndarray:
    x = _f32(x)
    e = np.ascontiguousarray(experts, np.uint32)
    w = _f32(weights)
    out = np.empty(n_embd, np.float32)
    if _lib().orc_moe_ffn(_p(x), n_embd, n_ff, n_expert, _p(_u8(gate)), _p(_u8(up)), _p(_u8(down)),
                          _p(e), _p(w), e.size, _p(out)):
        raise ValueError("moe_ffn failed")
    return out


def moe_layer(x, x_res, n_embd, n_ff, n_expert, n_used, router, gate, up, down):
    """Returns (out, logits, ids, weights)."""
    x, xr = _f32(x), _f32(x_res)
    out = np.empty(n_embd, np.float32)
    lg = np.empty(n_expert, np.float32)
    ids = np.empty(n_used, np.uint32)
    w = np.empty(n_used, np.float32)
    if _lib().orc_moe_layer(_p(x), _p(xr), n_embd, n_ff, n_expert, n_used, _p(_f32(router)),
                            _p(_u8(gate)), _p(_u8(up)), _p(_u8(down)), _p(out), _p(lg), _p(ids), _p(w)):
        raise ValueError("moe_layer failed")
    return out, lg, ids, w


def argmax(v) -> int:
    v = _f32(v)
    return int(_lib().orc_argmax(_p(v), v.size))


def moe_ffn_tokens(x, n_embd, n_ff, n_expert, gate, up, down, ids, weights) -> np.ndarray:
    x = _f32(x).reshape(-1, n_embd)
    n_tok = x.shape[0]
    ids = np.ascontiguousarray(ids, np.uint32).reshape(n_tok, -1)
    w = _f32(weights).reshape(n_tok, -1)
    out = np.empty((n_tok, n_embd), np.float32)
    if _lib().orc_moe_ffn_tokens(_p(x), n_tok, n_embd, n_ff, n_expert, _p(_u8(gate)), _p(_u8(up)),
                                 _p(_u8(down)), _p(ids), _p(w), ids.shape[1], _p(out)):
        raise ValueError("moe_ffn_tokens failed")
    return out


def close(a: float, b: float, tol: float) -> bool:
    return bool(_lib().orc_close(a, b, tol))


def max_deviation(a, b):
    """tolerance.rs:135-151: (index, worst relative deviation)."""
    a, b = _f32(a), _f32(b)
    worst = (0, 0.0)
    both_nan = np.isnan(a) & np.isnan(b)
    scale = np.maximum(np.maximum(np.abs(a), np.abs(b)), 1.0)
    d = np.abs(a - b) / scale
    d[both_nan] = 0.0
    if d.size:
        i = int(np.argmax(d))
        if d[i] > 0:
            worst = (i, float(d[i]))
    return worst


def rope(x, heads: int, hd: int, pos: int, base: float) -> np.ndarray:
    """CpuBackend::rope (llamd-cpu/src/lib.rs:158-209), NeoX pairs (i, i + hd/2)."""
    y = np.array(_f32(x), np.float32, copy=True)
    if y.size != heads * hd or hd % 2:
        raise ValueError("x must be [heads, hd] with hd even")
    _lib().orc_rope(_p(y), heads, hd, pos, base)
    return y


def attend(q, k, v, n_kv: int, n_head: int, n_head_kv: int, hd: int) -> np.ndarray:
    """attend (llamd-runtime/src/attention.rs:73-125); k, v [n_kv][n_head_kv*hd]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(n_head * hd, np.float32)
    if (q.size != n_head * hd or k.size != n_kv * n_head_kv * hd or v.size != k.size or
            _lib().orc_attend(_p(q), _p(k), _p(v), n_kv, n_head, n_head_kv, hd, _p(out))):
        raise ValueError("attend: shape or grouping violation")
    return out
