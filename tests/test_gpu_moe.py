"""Routing, the MoE decode layer, prefill grouping and the LM head on the
MI355X against the CPU oracle. Router logits, expert ids, routing weights,
decode-layer outputs and argmax ids: EXACT (bit-identical)."""
import math

import numpy as np
import pytest

import helpers as H
from llamd_rs_amd._lib import lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu
QK_K = 256


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


CASES = [([0.1, 5.0, 0.2, 3.0, 0.3], 2), ([1, 2, 3, 4, 5, 6, 7, 8], 3), ([10.0, 9.0, 0.0, 0.0], 2),
         ([3.0, 1.0, 4.0, 1.0, 5.0], 2), ([1.0, 1.0, 1.0, 1.0], 2), ([0.0, -800.0, -800.0, -800.0], 3),
         ([0.0, -800.0, -900.0, -850.0], 3)]


@pytest.mark.parametrize("logits,n_used", CASES)
def test_route_known_answers(gpu, logits, n_used):               # moe.rs:115-247
    want = O.route(logits, n_used)
    got = gpu.route(logits, n_used)
    assert list(got.experts) == list(want.experts)
    assert bits_equal(got.weights, want.weights)


def test_route_random_and_tied_logits(gpu):
    rng = np.random.default_rng(0)
    for t in range(200):
        lg = rng.standard_normal(128).astype(np.float32) * 2
        if t % 3 == 0:
            lg[rng.integers(0, 128, 20)] = lg[5]          # exact ties
        if t % 5 == 0:
            lg[7] = np.nextafter(lg[9], np.float32(10))   # one-ulp neighbours
        want = O.route(lg, 8)
        got = gpu.route(lg, 8)
        assert list(got.experts) == list(want.experts), t
        assert bits_equal(got.weights, want.weights), t


def test_route_refuses_impossible_requests(gpu):
    with pytest.raises(ValueError):
        gpu.route([1.0, 2.0], 0)
    with pytest.raises(ValueError):
        gpu.route([1.0, 2.0], 3)


def test_argmax_lowest_index(gpu):
    v = np.zeros((3, 10000), np.float32)
    v[0, [17, 5000, 9999]] = 3.0
    v[1] = np.random.default_rng(1).standard_normal(10000)
    v[2, :] = -np.inf
    ids = gpu.argmax(v)
    assert list(ids) == [O.argmax(v[0]), O.argmax(v[1]), O.argmax(v[2])] == [17, int(np.argmax(v[1])), 0]


def make_layer(n_embd, n_ff, n_expert, seed):
    from llamd_rs_amd import synth
    router = synth.normal(seed, 0.02, n_expert * n_embd).reshape(n_expert, n_embd)
    gate = synth.q6k_matrix(seed + 1, 0.02, n_expert * n_ff, n_embd)
    up = synth.q6k_matrix(seed + 2, 0.02, n_expert * n_ff, n_embd)
    down = synth.q6k_matrix(seed + 3, 0.02, n_expert * n_embd, n_ff)
    return router, gate, up, down


@pytest.fixture(scope="module")
def qwen_layer(gpu):
    """hidden 2048, 128 experts of Q6_K gate/up [768 x 2048] and
    down [2048 x 768], f32 router [128 x 2048], top-8."""
    n_embd, n_ff, n_expert, n_used = 2048, 768, 128, 8
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 500)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    yield layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    layer.close()


def test_moe_layer_bit_identical(gpu, qwen_layer):
    """configs[2] decode layer: logits, expert ids, routing weights and the
    layer output all equal the CPU path's bits on every call."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    calls0, _ = layer.stats()
    for t in range(8):
        x = synth.normal(1000 + t, 1.0, n_embd)
        res = synth.normal(2000 + t, 1.0, n_embd)
        want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
        out, r, lg_used = layer.forward(x, res)
        assert bits_equal(lg_used, lg), t
        assert list(r.experts) == list(ids), t
        assert bits_equal(r.weights, w), t
        assert bits_equal(out, want), t
    calls, exact_calls = layer.stats()
    assert calls - calls0 == 8 and exact_calls == calls


def test_moe_layer_sweep_certified_path(gpu, qwen_layer):
    """48 more calls over input scales from 1e-3 to 1e3: every call's logits,
    ids, weights and output are the CPU path's bits, and the calls that
    started gate/up on the certified estimate (the composite-key top-k and
    its outward-rounded bounds) are counted."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    c0, _ = layer.counters()
    for t in range(48):
        scale = np.float32(10.0 ** (t % 7 - 3))
        x = synth.normal(5000 + t, 1.0, n_embd) * scale
        res = synth.normal(6000 + t, 1.0, n_embd)
        want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
        out, r, lg_used = layer.forward(x, res)
        assert bits_equal(lg_used, lg), t
        assert list(r.experts) == list(ids), t
        assert bits_equal(r.weights, w), t
        assert bits_equal(out, want), t
    c1, est = layer.counters()
    assert c1[0] - c0[0] == 48
    # the estimate certifies unless the chosen logits spread over 80 or more
    # (probabilities that could underflow to a tie): scales 1e2 and 1e3 do
    assert c1[2] - c0[2] >= 30, (c1, c0)
    assert c1[3] == 0                       # no wait gave up


def test_moe_layer_without_residual(gpu, qwen_layer):
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    x = synth.normal(3000, 1.0, n_embd)
    zero = np.zeros(n_embd, np.float32)
    want, lg, ids, w = O.moe_layer(x, zero, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
    out, r, _ = layer.forward(x, None)
    # res = 0 adds +0.0 to each sum: the same bits except that -0.0 becomes +0.0
    assert np.array_equal(out, want)


def test_moe_layer_near_tied_router_stays_exact(gpu):
    """A router whose top experts are separated by far less than the float
    error of the parallel sum: the ids must still be the CPU's."""
    n_embd, n_ff, n_expert, n_used = 256, 256, 16, 4
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 900)
    router = router.copy()
    for e in (3, 8, 12):
        router[e] = router[5]
    router[9] = router[5] * np.float32(1 + 2 ** -22)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    rng = np.random.default_rng(3)
    for t in range(10):
        x = rng.standard_normal(n_embd).astype(np.float32)
        x = x * np.sign(router[5] @ x)      # make the tied group win
        want, lg, ids, w = O.moe_layer(x, np.zeros(n_embd, np.float32), n_embd, n_ff, n_expert,
                                       n_used, router, gate, up, down)
        out, r, _ = layer.forward(x, np.zeros(n_embd, np.float32))
        assert list(r.experts) == list(ids), (t, r.experts, ids)
        assert bits_equal(r.weights, w), t
        assert bits_equal(out, want), t
    layer.close()


@pytest.mark.parametrize("twin", [1, 0])
def test_prefill_grouped_equals_token_major(gpu, twin):
    """R14: expert-grouped prefill == per-token moe_ffn, EXACT, including a
    1-token case and experts of 1 to 13 16-token chunks (twin = 1: two chunks
    of one expert per wave, with a lone chunk where the count is odd; twin =
    0: one chunk per wave)."""
    from llamd_rs_amd import synth
    n_embd, n_ff, n_expert, n_used = 512, 256, 16, 4
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 700)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    prev = lib().llamd_hip_tune(b"batched_twin", twin)
    try:
        for n_tok in (1, 5, 37, 80, 200):
            x = synth.normal(10 + n_tok, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
            ids, w = synth.zipf_routing(20 + n_tok, 1.1, n_tok, n_expert, n_used)
            got = layer.prefill(x, ids.astype(np.int32), w)
            want = O.moe_ffn_tokens(x, n_embd, n_ff, n_expert, gate, up, down, ids, w)
            assert bits_equal(got, want), n_tok
            check_reduction_prefill(layer.prefill(x, ids.astype(np.int32), w, reduction=True), want)
            chunks = -(-np.bincount(ids.ravel(), minlength=n_expert) // 16)
            if n_tok == 80:
                assert chunks.max() >= 3 and (chunks % 2 == 1).any() and (chunks == 2).any()
            if n_tok == 200:
                assert chunks.max() > 8
    finally:
        lib().llamd_hip_tune(b"batched_twin", prev)
    layer.close()


def test_prefill_grouping_past_one_id_batch(gpu):
    """The grouping kernel takes the expert ids in batches of 8 per thread of
    its 1024 (8192 pairs); the last batch stays in registers for the scatter
    and the others are loaded again. 1040 tokens x top-8 = 8320 pairs cross
    that line: every token is checked bit for bit against the CPU."""
    from llamd_rs_amd import synth
    n_embd, n_ff, n_expert, n_used, n_tok = 512, 256, 16, 8, 1040
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 910)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    x = synth.normal(911, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
    ids, w = synth.zipf_routing(912, 1.1, n_tok, n_expert, n_used)
    assert ids.size > 8192
    got = layer.prefill(x, ids.astype(np.int32), w)
    parts = H.par_map(lambda s: O.moe_ffn_tokens(x[s:s + 16], n_embd, n_ff, n_expert, gate, up,
                                                 down, ids[s:s + 16], w[s:s + 16]),
                      range(0, n_tok, 16))
    want = np.concatenate(parts)
    bad = [t for t in range(n_tok) if not bits_equal(got[t], want[t])]
    assert not bad, bad[:10]
    layer.close()


@pytest.mark.parametrize("twin", [1, 0])
def test_prefill_chunk_boundary_groups(gpu, twin):
    """Groups at the 16-token chunk boundaries: one expert taking every token
    (4 full chunks), one with exactly 16 pairs, one with 17 (a chunk and a
    lone token), one with 15, the rest spread thin; EXACT against
    token-major moe_ffn with and without twins."""
    n_embd, n_ff, n_expert, n_used, n_tok = 512, 256, 16, 4, 64
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 760)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    t = np.arange(n_tok)
    ids = np.stack([np.zeros(n_tok, int), np.where(t < 16, 1, 5), np.where(t < 17, 2, 6),
                    np.where(t < 15, 3, 7 + t % 9)], axis=1).astype(np.int32)
    counts = np.bincount(ids.ravel(), minlength=n_expert)
    assert (counts[0], counts[1], counts[2], counts[3]) == (64, 16, 17, 15)
    rng = np.random.default_rng(761)
    w = rng.random((n_tok, n_used)).astype(np.float32) + 0.1
    w /= w.sum(axis=1, keepdims=True)
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    prev = lib().llamd_hip_tune(b"batched_twin", twin)
    try:
        got = layer.prefill(x, ids, w)
        want = O.moe_ffn_tokens(x, n_embd, n_ff, n_expert, gate, up, down, ids, w)
        assert bits_equal(got, want)
        check_reduction_prefill(layer.prefill(x, ids, w, reduction=True), want)
    finally:
        lib().llamd_hip_tune(b"batched_twin", prev)
    layer.close()


def test_prefill_config_shape_sample(gpu, qwen_layer):
    """configs[3] shapes (hidden 2048, 128 experts, top-8, Zipf 1.1) on 48 tokens."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    n_tok = 48
    x = synth.normal(77, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
    ids, w = synth.zipf_routing(78, 1.1, n_tok, n_expert, n_used)
    got = layer.prefill(x, ids.astype(np.int32), w)
    want = O.moe_ffn_tokens(x, n_embd, n_ff, n_expert, gate, up, down, ids, w)
    assert bits_equal(got, want)


@pytest.fixture(scope="module")
def lm_head(gpu):
    from llamd_rs_amd import synth
    rows, k = 151936, 2048
    w = synth.q6k_matrix(4242, 0.02, rows, k)
    dw = gpu.DeviceWeights.upload(w, rows, k // QK_K)
    head = gpu.LmHead(dw, max_seq=16)
    yield head, w, rows, k
    head.close()
    dw.close()


def test_lm_head_b1_logits_and_argmax_exact(gpu, lm_head):
    from llamd_rs_amd import synth
    head, w, rows, k = lm_head
    x = synth.normal(31, 1.0, k)
    logits, ids = head.forward(x)
    want = O.matvec_q6k(w, rows, k, x)
    assert bits_equal(logits[0], want)
    assert ids[0] == O.argmax(want)


def test_lm_head_b16_argmax_exact(gpu, lm_head):
    """configs[4] at b = 16: all 16 sequences' 151936 logits and argmax ids
    against the CPU's matvec_quant and argmax."""
    from llamd_rs_amd import synth
    head, w, rows, k = lm_head
    x = synth.normal(32, 1.0, 16 * k).reshape(16, k)
    logits, ids = head.forward(x)
    want = H.par_map(lambda s: O.matvec_q6k(w, rows, k, x[s]), range(16))
    for s in range(16):
        assert bits_equal(logits[s], want[s]), s
        assert ids[s] == O.argmax(want[s]), s
    # LLAMD_HIP_REDUCTION: logits within REDUCTION, ids still bit-exact
    fl, fids = head.forward(x, reduction=True)
    for s in range(16):
        check_reduction_logits(fl[s], want[s])
        assert fids[s] == O.argmax(want[s]), s


def check_reduction_logits(got, want):
    """Logits of the LLAMD_HIP_REDUCTION LM head: NaN where the CPU's are,
    every other logit within tolerance::REDUCTION x the rms of the logits (the
    reference's bound for reductions over random weights, grouped_expert.rs:
    147-175), the certified tiles' rows bit-identical."""
    assert (np.isnan(got) == np.isnan(want)).all()
    ok = ~np.isnan(want)
    g, w = got[ok].astype(np.float64), want[ok].astype(np.float64)
    rms = np.sqrt((w ** 2).mean())
    assert np.abs(g - w).max() <= O.REDUCTION * rms, (np.abs(g - w).max(), rms)
    assert (got[ok] == want[ok]).any()  # at least the recomputed tiles are exact


def test_lm_head_b16_reduction_near_ties(gpu):
    """LLAMD_HIP_REDUCTION at b = 16 where the two largest logits differ by
    about one activation step: a copy of the winning row, in a lower and in a
    higher tile, with one 6-bit code moved by +1 or -1 at a weight whose Q8_K
    quant is +-1. The ids must be the CPU's arg-max in every case, whichever
    way the float rounding of the fast logits leans."""
    rows, k, nseq = 64 * 16, 256, 16
    x = H.sample(nseq * k, 77).reshape(nseq, k)
    w0 = H.weights(rows, 1, 78).reshape(rows, 210).copy()
    qs = O.quantize_q8_k(x[0]).qs.reshape(-1)
    m = int(np.argmax(O.matvec_q6k(w0.reshape(-1), rows, k, x[0])))
    # a weight e with quant +-1; its sub-block scale in row m set to 1, so one
    # code step moves the logit by f16(d) * a.d only (while m stays the arg-max)
    for e in np.flatnonzero(np.abs(qs) == 1):
        w1 = w0.copy()
        w1[m, 192 + e // 16] = 1
        if O.argmax(O.matvec_q6k(w1.reshape(-1), rows, k, x[0])) == m:
            break
    w0 = w1
    for dst in (m % 16 + 16 * ((m // 16 + 7) % 64), m % 16 + 16 * ((m // 16 + 57) % 64)):
        for step in (1, -1):
            w = w0.copy()
            w[dst] = w[m]
            # weight e = 128 half + 32 j + l: a nibble of ql[64 half + l + 32 (j & 1)],
            # the high one for j >= 2 (lib.rs:181-226)
            half, r = divmod(e, 128)
            j, l = divmod(r, 32)
            byte = 64 * half + l + 32 * (j & 1)
            shift = 4 * (j >> 1)
            nib = (int(w[dst, byte]) >> shift) & 0xF
            if not 0 <= nib + step <= 15:
                continue
            w[dst, byte] = (int(w[dst, byte]) & ~(0xF << shift) | ((nib + step) << shift)) & 0xFF
            dw = gpu.DeviceWeights.upload(w.reshape(-1), rows, 1)
            head = gpu.LmHead(dw, max_seq=nseq)
            fl, ids = head.forward(x, reduction=True)
            want = O.matvec_q6k(w.reshape(-1), rows, k, x[0])
            assert 0 < abs(float(want[dst]) - float(want[m])) < 1e-3
            assert ids[0] == O.argmax(want), (dst, step, ids[0], O.argmax(want))
            check_reduction_logits(fl[0], want)
            head.close()
            dw.close()


@pytest.mark.parametrize("nseq", [1, 16])
def test_lm_head_argmax_ties_and_nan(gpu, nseq):          # device_forward.rs:23-37
    """The per-tile arg-max candidates of the matvec epilogue, reduced: a
    duplicated winning row loses to its lower-index copy across tiles, a NaN
    logit never wins, and a NaN at index 0 makes the answer 0."""
    _lm_head_ties_and_nan(gpu, nseq)


def test_lm_head_b1_argmax_across_tiles_and_calls(gpu):
    """b = 1 over 130 tiles: copies of the winner in a tile 64 apart and in
    the next tile resolve to the lowest row; all-negative logits pick the
    least negative; repeated calls on one head (later maxima smaller) each
    give the oracle's id."""
    rows, k = 130 * 16, 256
    x = H.sample(k, 23)
    w = H.weights(rows, 1, 29).reshape(rows, 210).copy()
    logits = O.matvec_q6k(w.reshape(-1), rows, k, x)
    m = int(np.argmax(logits))
    t = m // 16
    for dst_tile in (t + 64 if t + 64 < 130 else t - 64, (t + 1) % 130):
        w[dst_tile * 16 + 5] = w[m]
    neg = w.copy()
    pos = O.matvec_q6k(w.reshape(-1), rows, k, x) > 0
    neg[pos, 209] ^= 0x80                        # d's sign flipped: every logit <= 0 at x
    for case, wc in (("copies", w), ("negative", neg)):
        dw = gpu.DeviceWeights.upload(wc.reshape(-1), rows, 1)
        head = gpu.LmHead(dw, max_seq=1)
        for xs in (x, x * 0.25, -x):             # later calls with smaller maxima
            got_logits, ids = head.forward(xs.reshape(1, k))
            want = O.matvec_q6k(wc.reshape(-1), rows, k, xs)
            assert bits_equal(got_logits[0], want), case
            assert ids[0] == O.argmax(want), (case, ids[0], O.argmax(want))
        head.close()
        dw.close()


def _lm_head_ties_and_nan(gpu, nseq):
    rows, k = 64, 256
    x = H.sample(nseq * k, 5).reshape(nseq, k)
    w = H.weights(rows, 1, 17).reshape(rows, 210).copy()
    logits = np.stack([O.matvec_q6k(w.reshape(-1), rows, k, x[s]) for s in range(nseq)])
    m = int(np.argmax(logits[0]))
    w[37] = w[m]                        # a copy in a later tile
    w[3 if m > 3 else 60] = w[m]        # and one in another tile
    w[50, 208:210] = (0x00, 0x7E)       # f16 NaN scale: logit 50 is NaN
    for case in ("ties", "nan0"):
        if case == "nan0":
            w[0, 208:210] = (0x00, 0x7E)
        dw = gpu.DeviceWeights.upload(w.reshape(-1), rows, 1)
        head = gpu.LmHead(dw, max_seq=16)
        got_logits, ids = head.forward(x)
        fl, fids = head.forward(x, reduction=True)
        for s in range(nseq):
            want = O.matvec_q6k(w.reshape(-1), rows, k, x[s])
            assert bits_equal(got_logits[s], want), (case, s)
            assert ids[s] == O.argmax(want), (case, s, ids[s], O.argmax(want))
            if nseq > 1:  # the certified arg-max, through its NaN fallback
                check_reduction_logits(fl[s], want)
                assert fids[s] == ids[s], (case, s)
        if case == "ties":
            assert ids[0] == min(m, 3 if m > 3 else 60)
        else:
            assert list(ids) == [0] * nseq
        head.close()
        dw.close()


def test_prefill_full_config_512_tokens(gpu, qwen_layer):
    """configs[3] at full size: 512 tokens, top-8 of 128, Zipf 1.1 (about 4096
    pairs, the most popular experts far above 16 tokens). Every one of the 512
    tokens is checked bit for bit against the CPU's moe_ffn, for both prefill
    kernels (two chunks of one expert per wave, and one)."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    n_tok = 512
    x = synth.normal(700, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
    ids, w = synth.zipf_routing(701, 1.1, n_tok, n_expert, n_used)
    got = layer.prefill(x, ids.astype(np.int32), w)
    counts = np.bincount(ids.ravel(), minlength=n_expert)
    assert counts.max() > 64
    parts = H.par_map(lambda s: O.moe_ffn_tokens(x[s:s + 16], n_embd, n_ff, n_expert, gate, up,
                                                 down, ids[s:s + 16], w[s:s + 16]),
                      range(0, n_tok, 16))
    want = np.concatenate(parts)
    bad = [t for t in range(n_tok) if not bits_equal(got[t], want[t])]
    assert not bad, bad[:10]
    for alt in (0,):  # the one-chunk wave kernel gives the same bits
        prev = lib().llamd_hip_tune(b"batched_twin", alt)
        try:
            other = layer.prefill(x, ids.astype(np.int32), w)
        finally:
            lib().llamd_hip_tune(b"batched_twin", prev)
        assert bits_equal(other, want), alt
    check_reduction_prefill(layer.prefill(x, ids.astype(np.int32), w, reduction=True), want)


def check_reduction_prefill(fast, want):
    """LLAMD_HIP_REDUCTION against the CPU's moe_ffn, by the survey's parity
    plan for the MoE output: a token whose SwiGLU Q8_K bytes are the CPU's is
    within REDUCTION x the rms of its output (the reference's reduction bound,
    grouped_expert.rs:147-175). A gate/up value that lands within rounding of
    a .5 quantization boundary can move one activation quant by 1; such a
    token is held to QUANTIZED_MATMUL under tolerance::close (tolerance.rs),
    and these tokens must stay rare."""
    rms = np.sqrt((want.astype(np.float64) ** 2).mean(axis=1))
    dev = np.abs(fast.astype(np.float64) - want).max(axis=1)
    rel = np.abs(fast.astype(np.float64) - want) / np.maximum(
        np.maximum(np.abs(fast), np.abs(want)), 1.0)
    over = np.flatnonzero(dev > O.REDUCTION * rms)
    print(f"REDUCTION prefill: {len(over)} of {len(want)} tokens beyond REDUCTION x rms "
          f"(worst close-deviation {rel.max():.2e}); median |dev|/rms {np.median(dev / rms):.2e}")
    assert rel.max() <= O.QUANTIZED_MATMUL
    assert len(over) <= max(2, len(want) // 20), over


def _host_bound(router, x):
    """Exact prefix-sum bound of the f32 sequential fold, on the host."""
    p = (router.astype(np.float32) * x.astype(np.float32)[None, :]).astype(np.float64)
    T = np.array([math.fsum(r) for r in p])
    pre = np.cumsum(p, axis=1)
    return T, 2.0 ** -24 * np.abs(pre).sum(axis=1), np.abs(p).sum(axis=1)


def test_decode_logit_estimates_bound_the_sequential_fold(gpu, qwen_layer):
    """The decode kernel starts gate/up on a top-k set certified from
    estimates T, E of the logits (|logit - T| <= E, Higham's recursive
    summation bound over the prefix sums). The published estimates must bound
    the reference's fold on every expert and match the host's bound."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    for t in range(6):
        x = synth.normal(4000 + t, 1.0 + 3 * t, n_embd)
        out, r, lg = layer.forward(x)
        _, est = layer.counters()
        T, E = est
        Th, Eh, pabs = _host_bound(router, x)
        assert np.all(np.abs(T - Th) <= 1e-12 * pabs), t
        assert np.all(np.abs(lg.astype(np.float64) - T) <= E), t
        assert np.all(E >= Eh) and np.all(E <= Eh * 1.01 + 2.0 ** -39 * pabs), t


def test_decode_certified_and_fallback_paths_both_exact(gpu):
    """Well-separated logits take the certified path, logits tied at the
    k-th place take the wait-for-exact path; both give the CPU's bits."""
    n_embd, n_ff, n_expert, n_used = 256, 256, 16, 4
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 910)
    router = router.copy()
    for e in (5, 7, 9, 11):
        router[e] = router[2]               # five experts tied exactly ...
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    rng = np.random.default_rng(5)
    try:
        c0, _ = layer.counters()
        n_cert = 0
        for t in range(12):
            x = rng.standard_normal(n_embd).astype(np.float32)
            if t % 2:
                x = x * np.sign(router[2] @ x) * 4  # ... on top: the tie straddles k = 4
            want, lg, ids, w = O.moe_layer(x, np.zeros(n_embd, np.float32), n_embd, n_ff, n_expert,
                                           n_used, router, gate, up, down)
            out, r, lgd = layer.forward(x)
            assert bits_equal(lgd, lg) and list(r.experts) == list(ids), t
            assert bits_equal(r.weights, w) and np.array_equal(out, want), t
        c1, _ = layer.counters()
        certified = c1[2] - c0[2]
        assert c1[3] == 0                       # no wait ever timed out
        assert c1[0] - c0[0] == 12 and c1[1] == c1[0]
        assert 0 < certified < 12, certified    # both paths were taken
    finally:
        layer.close()


def test_decode_past_the_fused_kernel_bit_identical(gpu):
    """A layer whose n_ff (2304: 9 blocks) exceeds the two-launch decode
    kernel's LDS takes one launch per step of the reference's chain (router;
    routing + gate/up; SwiGLU + Q8_K; down + combine): the same bits as the
    CPU's layer on every call."""
    from llamd_rs_amd import synth
    n_embd, n_ff, n_expert, n_used = 512, 2304, 16, 4
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 900)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    try:
        for t in range(3):
            x = synth.normal(5000 + t, 1.0, n_embd)
            res = synth.normal(5100 + t, 1.0, n_embd)
            want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
            out, r, lgd = layer.forward(x, res)
            assert bits_equal(lgd, lg) and list(r.experts) == list(ids), t
            assert bits_equal(r.weights, w) and bits_equal(out, want), t
    finally:
        layer.close()


@pytest.mark.parametrize("path", ["decode", "grouped"])
@pytest.mark.parametrize("nseq", [1, 2, 5, 16, 24])
def test_batched_decode_equals_per_sequence_decode(gpu, qwen_layer, nseq, path):
    """forward_batch: every sequence routed by its own exact logits -- through
    the decode kernels (router fold beside gate/up, per sequence) or through
    the expert-grouped kernels; each row bit-identical to the CPU's layer."""
    from llamd_rs_amd import synth
    from llamd_rs_amd._lib import lib
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    x = synth.normal(900 + nseq, 1.0, nseq * n_embd).reshape(nseq, n_embd)
    res = synth.normal(950 + nseq, 1.0, nseq * n_embd).reshape(nseq, n_embd)
    prev = lib().llamd_hip_tune(b"batch_decode_max", 64 if path == "decode" else 0)
    try:
        out, ids, w, lg = layer.forward_batch(x, res)
    finally:
        lib().llamd_hip_tune(b"batch_decode_max", prev)
    for s in range(nseq):
        want, lgc, idc, wc = O.moe_layer(x[s], res[s], n_embd, n_ff, n_expert, n_used, router, gate,
                                         up, down)
        assert bits_equal(lg[s], lgc), s
        assert list(ids[s]) == list(idc), s
        assert bits_equal(w[s], wc), s
        assert bits_equal(out[s], want), s


@pytest.mark.parametrize("path", ["decode", "grouped"])
def test_batched_decode_shared_experts_and_ties(gpu, path):
    """A batch whose sequences share experts (same x twice), tie at the k-th
    place (identical router rows) and run without a residual."""
    from llamd_rs_amd import synth
    n_embd, n_ff, n_expert, n_used = 256, 256, 16, 4
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 930)
    router = router.copy()
    for e in (5, 7, 9, 11):
        router[e] = router[2]
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    try:
        x = synth.normal(931, 1.0, 6 * n_embd).reshape(6, n_embd)
        x[3] = x[0]
        x[4] = x[4] * np.sign(router[2] @ x[4]) * 4
        from llamd_rs_amd._lib import lib
        prev = lib().llamd_hip_tune(b"batch_decode_max", 64 if path == "decode" else 0)
        try:
            c0, _ = layer.counters()
            out, ids, w, lg = layer.forward_batch(x)
            c1, _ = layer.counters()
        finally:
            lib().llamd_hip_tune(b"batch_decode_max", prev)
        if path == "decode":
            assert c1[0] - c0[0] == 6 and c1[3] == 0
            assert 0 < c1[2] - c0[2] < 6        # sequence 4 is not certified
        for s in range(6):
            want, lgc, idc, wc = O.moe_layer(x[s], np.zeros(n_embd, np.float32), n_embd, n_ff,
                                             n_expert, n_used, router, gate, up, down)
            assert list(ids[s]) == list(idc) and bits_equal(w[s], wc), s
            assert np.array_equal(out[s], want), s   # no residual: +0.0 vs -0.0 aside
        assert bits_equal(out[3], out[0])
    finally:
        layer.close()


def test_decode_waits_that_give_up_still_route_exactly(gpu, qwen_layer):
    """Workgroups of the decode launch wait on lower-indexed ones (the router
    folds). HIP does not promise dispatch order, so a wait that gives up must
    not route on an empty slot: the waiting wave computes the logit itself.
    moe_polls = 0 makes every wait give up at once (every kernel still exits
    normally); logits, ids, weights and outputs stay the CPU's bits, for one
    sequence and for the batched decode kernels."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    prev = lib().llamd_hip_tune(b"moe_polls", 0)
    try:
        for t in range(3):
            x = synth.normal(6000 + t, 1.0, n_embd)
            res = synth.normal(6100 + t, 1.0, n_embd)
            want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
            out, r, lgd = layer.forward(x, res)
            assert bits_equal(lgd, lg) and list(r.experts) == list(ids), t
            assert bits_equal(r.weights, w) and bits_equal(out, want), t
        c, _ = layer.counters()
        assert c[3] == 1          # the give-up path ran
        nseq = 3
        xb = synth.normal(6200, 1.0, nseq * n_embd).reshape(nseq, n_embd)
        prev_b = lib().llamd_hip_tune(b"batch_decode_max", 64)
        try:
            out, idb, wb, lgb = layer.forward_batch(xb)
        finally:
            lib().llamd_hip_tune(b"batch_decode_max", prev_b)
        for s in range(nseq):
            want, lgc, idc, wc = O.moe_layer(xb[s], np.zeros(n_embd, np.float32), n_embd, n_ff,
                                             n_expert, n_used, router, gate, up, down)
            assert bits_equal(lgb[s], lgc) and list(idb[s]) == list(idc), s
            assert bits_equal(wb[s], wc) and np.array_equal(out[s], want), s
    finally:
        lib().llamd_hip_tune(b"moe_polls", prev)
    assert lib().llamd_hip_tune(b"moe_polls", prev) == prev


@pytest.mark.parametrize("polls", [2, 6, 20])
def test_decode_some_waits_give_up(gpu, qwen_layer, polls):
    """A small bound on every wait makes some workgroups give up (and route
    on the exact logits, computing those not yet published) while others,
    placed later, still find the estimates and use the certified set: the
    slots hold the set in expert-index order either way, so every act row
    belongs to one expert and the results stay the CPU's bits."""
    from llamd_rs_amd import synth
    layer, (router, gate, up, down, n_embd, n_ff, n_expert, n_used) = qwen_layer
    prev = lib().llamd_hip_tune(b"moe_polls", polls)
    try:
        for t in range(6):
            x = synth.normal(6300 + 10 * polls + t, 1.0, n_embd)
            res = synth.normal(6400 + t, 1.0, n_embd)
            want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
            out, r, lgd = layer.forward(x, res)
            assert bits_equal(lgd, lg) and list(r.experts) == list(ids), t
            assert bits_equal(r.weights, w) and bits_equal(out, want), t
    finally:
        lib().llamd_hip_tune(b"moe_polls", prev)


def test_lm_head_b1_repeats_and_all_nan(gpu):
    """The b = 1 call (quantize, matvec with per-tile candidates, arg-max):
    calls in a row on changing inputs each get their own logits and answer,
    and a vocabulary of NaN logits gives 0 as the reference's scan does."""
    rows, k = 4000, 512
    w = H.weights(rows, 2, 23)
    dw = gpu.DeviceWeights.upload(w, rows, 2)
    head = gpu.LmHead(dw, max_seq=1)
    try:
        for seed in range(6):
            x = H.sample(k, 40 + seed) * (1 + seed)
            logits, ids = head.forward(x)
            want = O.matvec_q6k(w, rows, k, x)
            assert bits_equal(logits[0], want), seed
            assert ids[0] == O.argmax(want), (seed, ids[0], O.argmax(want))
    finally:
        head.close()
        dw.close()
    wn = H.weights(rows, 2, 24).reshape(rows * 2, 210).copy()
    wn[:, 208:210] = (0x00, 0x7E)  # every f16 scale NaN: every logit NaN
    dw = gpu.DeviceWeights.upload(wn.reshape(-1), rows, 2)
    head = gpu.LmHead(dw, max_seq=1)
    try:
        logits, ids = head.forward(H.sample(k, 3))
        assert np.isnan(logits[0]).all() and ids[0] == 0
        logits, ids = head.forward(H.sample(k, 4))
        assert ids[0] == 0
    finally:
        head.close()
        dw.close()


@pytest.mark.parametrize("rows,blocks", [(4000, 8), (1000, 5), (333, 3), (2000, 16), (50, 13), (700, 17)])
def test_lm_head_b1_block_counts(gpu, rows, blocks):
    """The b = 1 LM head at block counts that split unevenly over the matvec's
    four waves per tile and at row counts that leave a partial last tile:
    the CPU's logits and id bit for bit, over calls in a row."""
    k = blocks * QK_K
    w = H.weights(rows, blocks, 500 + blocks)
    dw = gpu.DeviceWeights.upload(w, rows, blocks)
    head = gpu.LmHead(dw, max_seq=1)
    try:
        for j in range(3):
            x = H.sample(k, 600 + j) * (1 + j)
            want = O.matvec_q6k(w, rows, k, x)
            logits, ids = head.forward(x)
            assert bits_equal(logits[0], want), j
            assert ids[0] == O.argmax(want), (j, ids[0])
    finally:
        head.close()
        dw.close()
