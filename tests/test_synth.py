"""This project's synthetic-weight quantizers (llamd_rs_amd/csrc/host/synth.cpp).

The reference has no Q6_K or Q8_0 weight quantizer (crates/llamd-quant only
dequantizes), so there is nothing to match bit for bit: parity of the
quantizers themselves is unpinned. What the block formats and the method
fix is checked instead, reading the blocks back with the oracle's pinned
dequantizers:
- format invariants (scale ranges, the all-zero block, f16 d finite);
- the value of largest magnitude in a Q6_K block maps to code 0 (w = -32)
  with group scale -128 and returns to within f16's rounding of d;
- a per-element round-trip bound derived from the method (below);
- the seeded generators are deterministic.
"""
import numpy as np
import pytest

from llamd_rs_amd import synth
from oracle import oracle as O

QK_K = 256


def _inputs():
    yield synth.normal(11, 0.02, 64 * QK_K)
    yield synth.normal(12, 1.0, 64 * QK_K) * np.repeat(np.geomspace(1e-3, 1e3, 64), QK_K).astype(np.float32)
    x = synth.normal(13, 1.0, 8 * QK_K)
    x[QK_K:2 * QK_K] = 0.0                      # an all-zero block
    x[2 * QK_K + 16:2 * QK_K + 32] = 0.0        # an all-zero group
    x[3 * QK_K:4 * QK_K] = 5.0                  # a constant block
    yield x


@pytest.mark.parametrize("x", list(_inputs()))
def test_q6k_round_trip(x):
    """Per 16-weight group the method takes the signed scale s_g = m/-32 (m
    the group's value of largest magnitude); per block d = f16(sm/-128) (sm
    the largest |s_g|, with its sign), sc_g = min(127, nearest(-128 s_g/sm))
    and codes clamp(nearest(x/(d sc_g)), -32, 31) + 32. So |x| <= 32 |s_g|,
    |s_g| <= (|sc_g| + 1/2) |d| (1 + 2^-11), and with de = d sc_g the error
    is |x - de q| <= |de| / 2 below the clamp. Values of the other sign than
    m reach code 31 at most (the clamp is asymmetric): there the error is
    |x| - 31 |de| <= |de| + 16 |d| + 32 (|sc_g| + 1/2) |d| 2^-11."""
    q = synth.quantize_q6k(x)
    y = O.dequantize(14, q, x.size)
    blk = q.reshape(-1, 210)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float32).ravel()
    sc = blk[:, 192:208].view(np.int8).astype(np.float32)
    assert np.all(np.isfinite(d))
    de = np.abs(np.repeat(d[:, None] * sc, 16, axis=1)).ravel()
    dd = np.repeat(np.abs(d), QK_K)
    bound = de + 16 * dd + 32 * (de + dd / 2) * 2.0 ** -11
    err = np.abs(x.astype(np.float64) - y)
    assert np.all(err <= bound * (1 + 2.0 ** -20) + 1e-30)
    for b in range(blk.shape[0]):
        xb = x[b * QK_K:(b + 1) * QK_K]
        if not np.any(xb):
            assert d[b] == 0 and np.all(y[b * QK_K:(b + 1) * QK_K] == 0)
            continue
        i = int(np.argmax(np.abs(xb)))
        g = i // 16
        assert sc[b, g] == -128
        # y = 4096 d with d = f16(m / 4096): off by f16's rounding of d at most
        # (2^-11 relative, 2^-25 absolute when d is an f16 subnormal)
        assert abs(float(y[b * QK_K + i]) - float(xb[i])) <= 4096 * max(
            abs(float(xb[i])) / 4096 * 2.0 ** -11, 2.0 ** -25) * (1 + 2.0 ** -20)


@pytest.mark.parametrize("x", list(_inputs()))
def test_q8_0_round_trip(x):
    """d = amax/127 stored as f16, q = round(x/d) with |q| <= 127: the error
    is at most d/2 plus 127 times the f16 rounding of d (2^-11 relative, or
    2^-25 absolute for a subnormal f16)."""
    q = synth.quantize_q8_0(x)
    y = O.dequantize(8, q, x.size)
    blk = q.reshape(-1, 34)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(np.isfinite(d)) and np.all(d >= 0)
    qs = blk[:, 2:].view(np.int8)
    assert qs.min() >= -127
    amax = np.abs(x.reshape(-1, 32)).max(axis=1).astype(np.float64)
    assert np.all(np.abs(d - amax / 127) <= amax / 127 * 2.0 ** -11 + 2.0 ** -25)
    bound = np.repeat(d / 2 + 127 * (d * 2.0 ** -11 + 2.0 ** -25) * (1 + 2.0 ** -10), 32)
    assert np.all(np.abs(x.astype(np.float64) - y) <= bound + 1e-30)


def test_generators_are_seeded():
    assert np.array_equal(synth.q6k_matrix(5, 0.02, 32, 512), synth.q6k_matrix(5, 0.02, 32, 512))
    assert not np.array_equal(synth.q6k_matrix(5, 0.02, 32, 512), synth.q6k_matrix(6, 0.02, 32, 512))
    a = synth.normal(9, 1.0, 100000)
    assert abs(float(a.mean())) < 0.02 and abs(float(a.std()) - 1.0) < 0.02
    ids, w = synth.zipf_routing(3, 1.1, 64, 128, 8)
    assert all(len(set(r)) == 8 for r in ids.tolist())      # 8 distinct experts per token
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
