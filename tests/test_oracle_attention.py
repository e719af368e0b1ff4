"""The oracle's RoPE and attention, pinned by the reference's own tests
(crates/llamd-cpu/src/lib.rs:313-357, crates/llamd-runtime/src/attention.rs
tests) and by float64 restatements of the same formulas."""
import math

import numpy as np
import pytest

from oracle import oracle as O

ATTENTION = 1e-5   # llamd-core tolerance.rs
F32_ULP = 1.2e-7


def close(a, b, tol):
    return abs(a - b) / max(abs(a), abs(b), 1.0) <= tol


def test_rope_at_position_zero_is_the_identity():
    x = np.array([1, 2, 3, 4], np.float32)
    out = O.rope(x, 1, 4, 0, 10000.0)
    assert all(close(a, c, F32_ULP) for a, c in zip(x, out))


def test_rope_pairs_across_the_half_boundary():
    out = O.rope(np.array([1, 0, 0, 0], np.float32), 1, 4, 1, 10000.0)
    assert close(out[0], math.cos(1.0), ATTENTION)
    assert close(out[2], math.sin(1.0), ATTENTION)     # partner of 0 is 2, not 1
    assert close(out[1], 0.0, ATTENTION)


def test_rope_preserves_the_norm_of_each_pair():
    x = np.array([0.3, -1.2, 0.7, 2.0, -0.5, 1.1, 0.9, -0.2], np.float32)
    out = O.rope(x, 1, 8, 37, 10_000_000.0)
    for i in range(4):
        assert close(math.hypot(x[i], x[i + 4]), math.hypot(out[i], out[i + 4]), ATTENTION)


def test_rope_matches_a_float64_rotation():
    rng = np.random.default_rng(1)
    heads, hd = 4, 128
    x = rng.standard_normal(heads * hd).astype(np.float32)
    for pos in (1, 17, 4095):
        out = O.rope(x, heads, hd, pos, 1_000_000.0).reshape(heads, hd)
        xs = x.astype(np.float64).reshape(heads, hd)
        i = np.arange(hd // 2)
        theta = pos / np.power(1_000_000.0, 2.0 * i / hd)
        a, b = xs[:, : hd // 2], xs[:, hd // 2:]
        want = np.concatenate([a * np.cos(theta) - b * np.sin(theta),
                               a * np.sin(theta) + b * np.cos(theta)], axis=1)
        # f32 theta carries ~pos * 2^-24 radians of rounding
        tol = 4e-6 * (1 + pos * 1e-3)
        assert np.max(np.abs(out - want)) < tol * np.max(np.abs(xs)) * 4, pos


def test_attention_single_position_returns_v():
    v = np.array([7, 8, 9, 10], np.float32)
    out = O.attend(np.full(4, 0.5, np.float32), np.full(4, 0.25, np.float32), v, 1, 1, 1, 4)
    assert all(close(o, e, ATTENTION) for o, e in zip(out, v))


def test_attention_is_a_convex_combination():
    q = np.array([1, 0], np.float32)
    k = np.array([1, 0, 0, 1, 0.5, 0.5], np.float32)
    v = np.array([10, 10, 20, 20, 30, 30], np.float32)
    out = O.attend(q, k, v, 3, 1, 1, 2)
    assert 10 < out[0] < 20


def test_grouped_query_heads_share_kv_heads_by_integer_division():
    k = np.array([1, 0, 1, 0], np.float32)
    v = np.array([100, 100, 200, 200], np.float32)
    q = np.array([1, 0] * 4, np.float32)
    out = O.attend(q, k, v, 1, 4, 2, 2)
    assert [close(out[i], w, ATTENTION) for i, w in ((0, 100), (2, 100), (4, 200), (6, 200))] == [True] * 4


def test_the_scale_is_one_over_sqrt_head_dim():
    q = np.array([2, 0, 0, 0], np.float32)
    k = np.array([2, 0, 0, 0, 0, 2, 0, 0], np.float32)
    v = np.array([1, 0, 0, 0, 0, 0, 0, 0], np.float32)
    out = O.attend(q, k, v, 2, 1, 1, 4)
    want = math.exp(2.0) / (math.exp(2.0) + 1.0)
    assert close(out[0], want, ATTENTION)


def test_large_logits_do_not_overflow():
    out = O.attend(np.full(4, 100, np.float32), np.array([100] * 4 + [-100] * 4, np.float32),
                   np.array([1] * 4 + [2] * 4, np.float32), 2, 1, 1, 4)
    assert np.all(np.isfinite(out)) and close(out[0], 1.0, ATTENTION)


def test_shape_and_grouping_violations_are_refused():
    with pytest.raises(ValueError):
        O.attend(np.zeros(6, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 1, 3, 2, 2)
    with pytest.raises(ValueError):
        O.attend(np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 0, 1, 1, 4)


def test_attention_matches_a_float64_restatement():
    rng = np.random.default_rng(2)
    n_head, n_kv_head, hd, n_kv = 8, 2, 64, 37
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_kv * n_kv_head * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * n_kv_head * hd).astype(np.float32)
    out = O.attend(q, k, v, n_kv, n_head, n_kv_head, hd).reshape(n_head, hd)
    K = k.astype(np.float64).reshape(n_kv, n_kv_head, hd)
    V = v.astype(np.float64).reshape(n_kv, n_kv_head, hd)
    for h in range(n_head):
        kvh = h // (n_head // n_kv_head)
        lg = K[:, kvh] @ q[h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
        p = np.exp(lg - lg.max())
        p /= p.sum()
        want = p @ V[:, kvh]
        assert np.max(np.abs(out[h] - want)) < 1e-4, h
