"""The oracle's routing, SwiGLU, MoE FFN and argmax, pinned.

Routing restates every unit test of crates/llamd-models/src/moe.rs:115-247;
the rest is checked against float64 restatements and closed forms.
"""
import numpy as np
import pytest

import helpers as H
from oracle import oracle as O


def test_selects_the_highest_scoring_experts_in_order():      # moe.rs:120-125
    assert list(O.route([0.1, 5.0, 0.2, 3.0, 0.3], 2).experts) == [1, 3]


def test_weights_sum_to_one_after_renormalisation():           # moe.rs:127-136
    r = O.route([1, 2, 3, 4, 5, 6, 7, 8], 3)
    assert O.close(float(np.sum(r.weights, dtype=np.float32)), 1.0, O.ATTENTION)
    assert r.weights[0] > r.weights[1] > r.weights[2]


def test_weights_are_renormalised_not_re_softmaxed():          # moe.rs:138-166
    r = O.route([10.0, 9.0, 0.0, 0.0], 2)
    assert O.close(float(r.weights[0]), 0.7310586, O.ATTENTION)
    assert O.close(float(r.weights[1]), 0.2689414, O.ATTENTION)
    p = np.array([0.7310586, 0.2689414], np.float32)
    e = np.exp(p - p[0])
    assert abs(float(r.weights[0]) - float(e[0] / e.sum())) > 0.1


def test_softmax_order_is_irrelevant_but_renormalisation_is_not():  # moe.rs:168-197
    logits = np.array([3.0, 1.0, 4.0, 1.0, 5.0], np.float32)
    r = O.route(logits, 2)
    ch = np.array([logits[4], logits[2]])
    e = np.exp(ch - ch.max())
    for a, b in zip(r.weights, e / e.sum()):
        assert O.close(float(a), float(b), O.ATTENTION)
    ea = np.exp(logits - logits.max())
    assert (ea[4] + ea[2]) / ea.sum() < 0.95


def test_ties_break_toward_the_lower_index():                  # moe.rs:199-212
    for _ in range(8):
        assert list(O.route([1.0, 1.0, 1.0, 1.0], 2).experts) == [0, 1]


def test_the_real_shape_routes_eight_of_128():                 # moe.rs:214-227
    lg = (np.sin(np.arange(128, dtype=np.float32) * np.float32(0.37)) * np.float32(3.0)).astype(np.float32)
    r = O.route(lg, 8)
    assert len(set(r.experts.tolist())) == 8
    assert O.close(float(np.sum(r.weights, dtype=np.float32)), 1.0, O.ATTENTION)


def test_a_degenerate_router_does_not_divide_by_zero():        # moe.rs:229-240
    r = O.route([0.0, -800.0, -800.0, -800.0], 3)
    assert np.all(np.isfinite(r.weights))
    # p = [1, 0, 0, 0]: zero probabilities tie and go in index order
    assert list(r.experts) == [0, 1, 2]


def test_impossible_requests_are_refused():                    # moe.rs:242-246
    with pytest.raises(ValueError):
        O.route([1.0, 2.0], 0)
    with pytest.raises(ValueError):
        O.route([1.0, 2.0], 3)


def test_route_matches_float64_softmax_topk():
    """Random logits: ids = argsort of logits (no ties), weights = renormalised
    softmax of the chosen ones, to f32 rounding."""
    rng = np.random.default_rng(0)
    for _ in range(50):
        lg = rng.standard_normal(128).astype(np.float32)
        r = O.route(lg, 8)
        order = np.argsort(-lg.astype(np.float64), kind="stable")[:8]
        assert list(r.experts) == list(order)
        ch = lg[order].astype(np.float64)
        w = np.exp(ch - ch.max())
        w /= w.sum()
        assert np.allclose(r.weights, w, rtol=1e-5, atol=1e-7)


def test_silu_and_mul_closed_form():
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    y = O.silu(x)
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.allclose(y, want, rtol=3e-7, atol=1e-30)
    assert np.array_equal(O.mul(x, x), (x * x).astype(np.float32))


def test_softmax_sums_to_one():                                 # llamd-cpu lib.rs:262
    y = O.softmax(np.array([1.0, 2.0, 3.0], np.float32))
    assert abs(float(y.sum()) - 1.0) < 1e-6 and y[2] > y[1] > y[0]


def test_argmax_lowest_index_and_nan():                         # device_forward.rs:23-37
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.argmax([np.nan, 5.0, 1.0]) == 0
    assert O.argmax([1.0, np.nan, 5.0]) == 2
    assert O.argmax([-np.inf, -np.inf]) == 0
    v = np.random.default_rng(2).standard_normal(10000).astype(np.float32)
    assert O.argmax(v) == int(np.argmax(v))


def test_moe_ffn_matches_float64_restatement():
    """moe_ffn against an independent float64 computation from dequantized
    weights and Q8_K-dequantized activations (the only approximations being
    f32 rounding and the Q8_K of the SwiGLU activation)."""
    rng = np.random.default_rng(4)
    n_embd, n_ff, n_exp = 512, 256, 4
    gate = H.weights(n_exp * n_ff, n_embd // 256, 1)
    up = H.weights(n_exp * n_ff, n_embd // 256, 2)
    down = H.weights(n_exp * n_embd, n_ff // 256, 3)
    x = rng.standard_normal(n_embd).astype(np.float32)
    ids, wts = np.array([2, 0], np.uint32), np.array([0.7, 0.3], np.float32)
    out = O.moe_ffn(x, n_embd, n_ff, n_exp, gate, up, down, ids, wts)

    def deq(w, rows, k, e):
        per = rows * k // 256 * 210
        return O.dequantize(14, w[e * per:(e + 1) * per], rows * k).reshape(rows, k).astype(np.float64)

    a = O.quantize_q8_k(x)
    xq = (a.qs.astype(np.float64) * a.d[:, None]).ravel()
    want = np.zeros(n_embd)
    for e, wt in zip(ids, wts):
        g = deq(gate, n_ff, n_embd, e) @ xq
        u = deq(up, n_ff, n_embd, e) @ xq
        with np.errstate(over="ignore"):
            act = g / (1 + np.exp(-g)) * u
        aq = O.quantize_q8_k(act.astype(np.float32))
        actq = (aq.qs.astype(np.float64) * aq.d[:, None]).ravel()
        want += wt * (deq(down, n_embd, n_ff, e) @ actq)
    scale = max(H.rms(want), 1.0)
    # the activation re-quantization can flip a rounding; bound it loosely
    assert np.max(np.abs(out - want)) <= 1e-3 * scale


def test_moe_layer_and_tokens_compose():
    rng = np.random.default_rng(6)
    n_embd, n_ff, n_exp, n_used = 256, 256, 8, 3
    router = (rng.standard_normal((n_exp, n_embd)) * 0.05).astype(np.float32)
    gate = H.weights(n_exp * n_ff, 1, 11)
    up = H.weights(n_exp * n_ff, 1, 12)
    down = H.weights(n_exp * n_embd, 1, 13)
    x = rng.standard_normal(n_embd).astype(np.float32)
    res = rng.standard_normal(n_embd).astype(np.float32)
    out, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_exp, n_used, router, gate, up, down)
    assert np.array_equal(lg, O.matvec_f32(router, n_exp, n_embd, x))
    r = O.route(lg, n_used)
    assert np.array_equal(ids, r.experts) and np.array_equal(w, r.weights)
    ffn = O.moe_ffn(x, n_embd, n_ff, n_exp, gate, up, down, ids, w)
    assert np.array_equal(out, (res + ffn).astype(np.float32))
    toks = O.moe_ffn_tokens(np.stack([x, x]), n_embd, n_ff, n_exp, gate, up, down,
                            np.stack([ids, ids]), np.stack([w, w]))
    assert np.array_equal(toks[0], ffn) and np.array_equal(toks[1], ffn)


def test_tolerance_semantics():                                 # tolerance.rs:153-197
    assert O.close(1.0, 1.0, O.EXACT)
    assert not O.close(1.0, 1.0 + O.F32_ULP, O.EXACT)
    assert not O.close(0.0, -0.0, O.EXACT)
    assert O.close(float("nan"), float("nan"), O.LOGITS)
    assert not O.close(float("nan"), 0.0, O.LOGITS)
    assert O.close(1e-9, 2e-9, O.ATTENTION)
    assert not O.close(1.0, 1.1, O.ATTENTION)
    assert O.EXACT < O.F32_ULP < O.REDUCTION <= O.ATTENTION < O.LAYER < O.LOGITS
    assert O.LAYER < O.QUANTIZED_MATMUL < O.QUANTIZED_LAYER
