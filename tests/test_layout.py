"""Host-side weight layouts: the tiled Q6_K and planar Q8_0 re-layouts are
permutations (crates/llamd-quant/src/dot.rs:425-461 holds the reference's own
repack to the same standard)."""
import ctypes as C

import numpy as np

import helpers as H
from llamd_rs_amd._lib import lib


def p(a):
    return a.ctypes.data_as(C.c_void_p)


def test_tiled_roundtrip_is_identity():
    L = lib()
    for rows, blocks in [(1, 1), (7, 5), (16, 8), (33, 3), (48, 2)]:
        w = H.weights(rows, blocks, rows * 7 + blocks)
        n = L.llamd_hip_q6k_tiled_bytes(rows, blocks)
        assert n == ((rows + 15) // 16) * blocks * 3360
        t = np.empty(n, np.uint8)
        assert L.llamd_hip_q6k_tile(p(w), rows, blocks, p(t)) == 0
        back = np.empty_like(w)
        assert L.llamd_hip_q6k_untile(p(t), rows, blocks, p(back)) == 0
        assert np.array_equal(back, w), (rows, blocks)


def test_tiled_is_a_bit_permutation_when_full():
    """16-row tiles have no padding: the multiset of bit values per field
    class is preserved (same 6-bit code histogram, same scale and d bytes)."""
    L = lib()
    rows, blocks = 32, 4
    w = H.synth(rows, blocks, 99)
    t = np.empty(L.llamd_hip_q6k_tiled_bytes(rows, blocks), np.uint8)
    L.llamd_hip_q6k_tile(p(w), rows, blocks, p(t))
    assert t.size == w.size
    wb = w.reshape(-1, 210)
    seg = t.reshape(-1, 3360)
    # scales and d: same bytes, different places
    assert sorted(wb[:, 192:208].ravel()) == sorted(seg[:, 3072:3328].ravel())
    assert sorted(wb[:, 208:210].ravel()) == sorted(seg[:, 3328:3360].ravel())
    # total popcount of the code bits is preserved
    pc = lambda a: int(np.unpackbits(a).sum())
    assert pc(wb[:, :192]) == pc(seg[:, :3072])


def test_tiled_segment_map_by_hand():
    """Spot-check the documented byte map: lane L = n + 16 s, class c word."""
    L = lib()
    codes = np.arange(256, dtype=np.uint8) % 64
    blk = H.q6k_block(codes, 0, 1.0)
    blk[192:208] = np.arange(16, dtype=np.uint8) + 100
    rows = np.tile(blk, 16)
    t = np.empty(3360, np.uint8)
    L.llamd_hip_q6k_tile(p(rows), 16, 1, p(t))
    n, s, c = 3, 2, 5
    lane = n + 16 * s
    word = t[(c // 4) * 1024 + 16 * lane + 4 * (c % 4): (c // 4) * 1024 + 16 * lane + 4 * (c % 4) + 4]
    for j in range(4):
        e_lo, e_hi = 8 * (8 * s + j) + c, 8 * (8 * s + j + 4) + c
        assert word[j] == (codes[e_lo] & 0xF) | ((codes[e_hi] & 0xF) << 4)
    assert list(t[3072 + 4 * lane: 3072 + 4 * lane + 4]) == [100 + 4 * s + v for v in range(4)]


def test_q8_0_planar():
    L = lib()
    rows, k = 5, 96
    w = np.random.default_rng(0).integers(0, 256, rows * k // 32 * 34).astype(np.uint8)
    n = L.llamd_hip_q8_0_planar_bytes(rows, k)
    out = np.empty(n, np.uint8)
    assert L.llamd_hip_q8_0_planarize(p(w), rows, k, p(out)) == 0
    blk = w.reshape(rows, k // 32, 34)
    assert np.array_equal(out[:rows * k].reshape(rows, k // 32, 32), blk[:, :, 2:])
    assert np.array_equal(out[rows * k:].reshape(rows, k // 32, 2), blk[:, :, :2])
