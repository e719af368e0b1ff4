"""Seeded synthetic workloads (llamd_rs_amd/csrc/host/synth.cpp) as numpy.

SplitMix64 -> Box-Muller N(0, sigma) f32; this project's Q6_K / Q8_0 weight
quantizers (the reference has none); Zipf(s) expert routing for prefill.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def normal(seed: int, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().llamd_synth_normal(seed, sigma, _p(out), n)
    return out


def quantize_q6k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, k = (x.shape if x.ndim == 2 else (1, x.size))
    out = np.empty(rows * k // 256 * 210, np.uint8)
    check(lib().llamd_synth_quantize_q6k(_p(x), rows, k, _p(out)), "quantize_q6k")
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, k = (x.shape if x.ndim == 2 else (1, x.size))
    out = np.empty(rows * k // 32 * 34, np.uint8)
    check(lib().llamd_synth_quantize_q8_0(_p(x), rows, k, _p(out)), "quantize_q8_0")
    return out


def q6k_matrix(seed: int, sigma: float, rows: int, k: int) -> np.ndarray:
    """rows x k weights ~ N(0, sigma) quantized to Q6_K, streamed (no f32 copy)."""
    out = np.empty(rows * (k // 256) * 210, np.uint8)
    check(lib().llamd_synth_q6k_matrix(seed, sigma, rows, k, _p(out)), "q6k_matrix")
    return out


def q8_0_matrix(seed: int, sigma: float, rows: int, k: int) -> np.ndarray:
    out = np.empty(rows * (k // 32) * 34, np.uint8)
    check(lib().llamd_synth_q8_0_matrix(seed, sigma, rows, k, _p(out)), "q8_0_matrix")
    return out


def zipf_routing(seed: int, s: float, n_tok: int, n_expert: int, n_used: int):
    ids = np.empty((n_tok, n_used), np.uint32)
    w = np.empty((n_tok, n_used), np.float32)
    check(lib().llamd_synth_zipf_routing(seed, s, n_tok, n_expert, n_used, _p(ids), _p(w)),
          "zipf_routing")
    return ids, w


def f32_to_f16_bits(v: float) -> int:
    return int(lib().llamd_synth_f32_to_f16(v))
