"""Input generators of the reference's own tests, restated in numpy.

These reproduce the seeded synthetic inputs of crates/llamd-testing/tests so
that our parity tests run on the same kind of data the reference's GPU tests
did (there are no golden files in the reference: every fixture is generated
in-test from these integer PRNGs).
"""
from __future__ import annotations

import numpy as np

QK_K = 256
B = 210
D_OFF = QK_K // 2 + QK_K // 4 + QK_K // 16  # 208


def _lcg_states(seed_state: int, n: int, a: int, c: int, bits: int) -> np.ndarray:
    """States s_1..s_n of s <- a*s + c (mod 2^bits), vectorised by composing
    the affine maps: s_i = a^i s_0 + c (1 + a + ... + a^(i-1))."""
    mask = np.uint64((1 << bits) - 1) if bits < 64 else np.uint64(0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        pw = np.cumprod(np.full(n, a, dtype=np.uint64), dtype=np.uint64)          # a^i
        geo = np.cumsum(np.concatenate([[np.uint64(1)], pw[:-1]]), dtype=np.uint64)  # sum_{j<i} a^j
        s = pw * np.uint64(seed_state) + np.uint64(c) * geo
    return s & mask


def sample(n: int, seed: int) -> np.ndarray:
    """rocm_oracle.rs:18-26: uniform [-1, 1) from a 32-bit LCG."""
    s0 = (seed * 2654435761 + 1) & 0xFFFFFFFF
    s = _lcg_states(s0, n, 1664525, 1013904223, 32)
    return (((s >> np.uint64(8)).astype(np.float32) / np.float32(1 << 24)) * np.float32(2.0)
            - np.float32(1.0)).astype(np.float32)


def weights(rows: int, blocks: int, seed: int) -> np.ndarray:
    """rocm_oracle.rs:29-44 / planar.rs:19-32: pseudo-Q6_K bytes from a 32-bit
    LCG with a sane f16 super-scale 0.008 + (blk % 17) * 0.002 per block."""
    n = rows * blocks * B
    st0 = (seed * 2246822519 + 7) & 0xFFFFFFFF
    s = _lcg_states(st0, n, 1664525, 1013904223, 32)
    w = ((s >> np.uint64(16)) & np.uint64(0xFF)).astype(np.uint8)
    nblk = rows * blocks
    blk = np.arange(nblk)
    d = (np.float32(0.008) + (blk % 17).astype(np.float32) * np.float32(0.002)).astype(np.float32)
    dh = d.astype(np.float16).view(np.uint16)
    w = w.reshape(nblk, B)
    w[:, D_OFF] = (dh & 0xFF).astype(np.uint8)
    w[:, D_OFF + 1] = (dh >> 8).astype(np.uint8)
    return w.reshape(-1)


def synth(rows: int, blocks: int, seed: int) -> np.ndarray:
    """grouped_expert.rs:37-56: PCG-multiplier bytes xor the byte index, with
    every block's f16 d set to 0x2c00 (~0.0156)."""
    n = rows * blocks * B
    s = _lcg_states(seed | 1, n, 6364136223846793005, 1442695040888963407, 64)
    v = ((s >> np.uint64(33)) & np.uint64(0xFF)).astype(np.uint8) ^ (np.arange(n) & 0xFF).astype(np.uint8)
    v = v.reshape(rows * blocks, B)
    v[:, D_OFF] = 0x00
    v[:, D_OFF + 1] = 0x2C
    return v.reshape(-1)


def sin_ramp(k: int, step: float, phase: float = 0.0, amp: float = 1.0) -> np.ndarray:
    """((i as f32) * step + phase).sin() * amp, in f32 like the reference's tests."""
    i = np.arange(k, dtype=np.float32)
    return (np.sin(i * np.float32(step) + np.float32(phase)) * np.float32(amp)).astype(np.float32)


def cos_ramp(k: int, step: float) -> np.ndarray:
    i = np.arange(k, dtype=np.float32)
    return np.cos(i * np.float32(step)).astype(np.float32)


def q8k_cases() -> np.ndarray:
    """The five blocks of grouped_expert.rs:235-240 / planar.rs:239-244:
    mixed, negative peak, all zero, exact +-0.5 ties, upper clamp."""
    i = np.arange(QK_K, dtype=np.float32)
    mixed = np.sin(i * np.float32(0.11)) * np.float32(3.0)
    negpk = -np.abs(np.cos(i * np.float32(0.07))) * np.float32(2.0)
    zero = np.zeros(QK_K, np.float32)
    ties = np.where(np.arange(QK_K) % 2 == 0, np.float32(0.5), np.float32(-0.5))
    clamp = np.where(np.arange(QK_K) == 0, np.float32(-8.0), np.float32(8.0))
    return np.concatenate([mixed, negpk, zero, ties, clamp]).astype(np.float32)


def rms(v: np.ndarray) -> float:
    v = v.astype(np.float64)
    return float(np.sqrt(np.mean(v * v)))


def q6k_block(codes: np.ndarray, scale: int, d: float) -> np.ndarray:
    """dot.rs:258-282: one Q6_K block from 256 6-bit codes and one scale."""
    blk = np.zeros(B, np.uint8)
    for half in range(2):
        ql, qh, o = half * 64, QK_K // 2 + half * 32, half * 128
        for l in range(32):
            c0, c1, c2, c3 = (int(codes[o + l]), int(codes[o + l + 32]), int(codes[o + l + 64]),
                              int(codes[o + l + 96]))
            blk[ql + l] = (c0 & 0xF) | ((c2 & 0xF) << 4)
            blk[ql + l + 32] = (c1 & 0xF) | ((c3 & 0xF) << 4)
            blk[qh + l] = (c0 >> 4) | ((c1 >> 4) << 2) | ((c2 >> 4) << 4) | ((c3 >> 4) << 6)
    blk[QK_K // 2 + QK_K // 4: D_OFF] = np.uint8(scale & 0xFF)
    dh = np.array([d], np.float32).astype(np.float16).view(np.uint16)[0]
    blk[D_OFF] = dh & 0xFF
    blk[D_OFF + 1] = dh >> 8
    return blk


def par_map(fn, items, workers: int | None = None) -> list:
    """fn over items on a thread pool. The oracle's ctypes calls release the
    GIL, so full-size oracle checks spread over the host's cores (at most 16:
    a GPU box's CPU share)."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    items = list(items)
    workers = workers or max(1, min(16, os.cpu_count() or 1, len(items)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        return list(ex.map(fn, items))
