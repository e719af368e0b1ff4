"""The CPU oracle's quantization arithmetic, pinned.

Each reference unit test of crates/llamd-quant (lib.rs:228-324, dot.rs:198-347)
is restated here against the C restatement, plus checks the reference does
not make but the mathematics fixes: every f16 code, every Q6_K element
position, and a float64 bound on the dot product.
"""
import numpy as np
import pytest

import helpers as H
from oracle import oracle as O

QK_K = 256


def test_q6k_block_size_matches_ggml():           # lib.rs:234-240
    assert O.bytes_for(14, QK_K) == 210
    assert 2 + QK_K // 16 + 3 * QK_K // 4 == 210


def test_q8_0_block_size_matches_ggml():          # lib.rs:242-247
    assert O.bytes_for(8, 32) == 34


def test_unknown_type_is_refused():               # lib.rs:249-259
    assert O.bytes_for(12, 256) == -1
    assert O.bytes_for(0, 3) == 12 and O.bytes_for(1, 3) == 6


def test_q8_0_dequantizes_by_hand():              # lib.rs:261-275
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([2.0], np.float16).view(np.uint8)
    blk[2] = 1
    blk[3] = 0xFF
    out = O.dequantize(8, blk, 32)
    assert out[0] == 2.0 and out[1] == -2.0 and np.all(out[2:] == 0.0)


def test_q6k_centres_on_minus_32():               # lib.rs:277-291
    blk = np.zeros(210, np.uint8)
    blk[192] = 1
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    assert O.dequantize(14, blk, QK_K)[0] == -32.0


def test_q6k_reads_high_bits_from_qh():           # lib.rs:293-307
    blk = np.zeros(210, np.uint8)
    blk[0] = 0x05
    blk[128] = 0b11
    blk[192] = 1
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    assert O.dequantize(14, blk, QK_K)[0] == 21.0


def test_short_and_partial_input_refused():       # lib.rs:309-323
    with pytest.raises(ValueError):
        O.dequantize(14, np.zeros(10, np.uint8), QK_K)
    assert O.bytes_for(14, 100) == -1
    assert O.bytes_for(14, 512) == 420


def test_f16_every_code_matches_ieee():
    """half 2.7.1's to_f32 is exact IEEE; numpy's float16 is the independent
    implementation. All 65536 codes, NaNs compared as NaN."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(c)) for c in codes], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_q6k_every_position_probe():
    """One nonzero code at a time: element e must come out as d*sc[e/16]*(code-32)
    exactly at position e and -32*d*sc elsewhere. Catches any index or shift
    mistake in the unpacking (a transposed half, wrong qh pair, wrong scale)."""
    rng = np.random.default_rng(1)
    for e in range(QK_K):
        codes = np.full(QK_K, 32, np.uint8)  # weight 0 everywhere
        code = int(rng.integers(0, 64))
        codes[e] = code
        blk = H.q6k_block(codes, 0, 1.0)
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        blk[192:208] = sc.view(np.uint8)
        blk[208:210] = np.array([0.5], np.float16).view(np.uint8)
        out = O.dequantize(14, blk, QK_K)
        want = np.zeros(QK_K, np.float32)
        want[e] = np.float32(0.5) * np.float32(sc[e // 16]) * np.float32(code - 32)
        assert np.array_equal(out, want), e


def test_rounding_is_half_to_even():              # dot.rs:209-221
    assert O.nearest_int(0.5) == 0
    assert O.nearest_int(1.5) == 2
    assert O.nearest_int(2.5) == 2
    assert O.nearest_int(-0.5) == 0
    assert O.nearest_int(-1.5) == -2
    assert O.nearest_int(-2.5) == -2


def test_the_peak_magnitude_maps_to_minus_127():  # dot.rs:223-237
    v = np.full(QK_K, 0.1, np.float32)
    v[7] = 5.0
    assert O.quantize_q8_k(v).qs[0, 7] == -127
    v[7] = -5.0
    assert O.quantize_q8_k(v).qs[0, 7] == -127


def test_an_all_zero_block_has_no_scale():        # dot.rs:239-245
    b = O.quantize_q8_k(np.zeros(QK_K, np.float32))
    assert b.d[0] == 0.0 and np.all(b.qs == 0)


def test_bsums_are_group_sums_of_sixteen():       # dot.rs:247-255
    v = np.sin(np.arange(QK_K, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    b = O.quantize_q8_k(v)
    assert np.array_equal(b.bsums[0], b.qs[0].reshape(16, 16).astype(np.int16).sum(1))


def test_q8k_reconstruction_and_convention():
    """Closed form: |x - d*q| <= |d|/2 except at the clamp, the first
    largest-magnitude element maps to -127, and d = max/-127 to 1 ulp."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal(QK_K * 64).astype(np.float32)
    x[QK_K * 3 + 5] = x[QK_K * 3 + 9] = 7.0     # tie: first index wins
    b = O.quantize_q8_k(x)
    for i in range(64):
        xb = x[i * QK_K:(i + 1) * QK_K]
        j = int(np.argmax(np.abs(xb)))
        assert b.qs[i, j] == -127
        rec = b.d[i] * b.qs[i].astype(np.float32)
        assert np.max(np.abs(rec - xb)) <= abs(b.d[i]) * 0.5 * (1 + 1e-5)
        assert np.isclose(b.d[i], xb[j] / -127.0, rtol=2e-7)
    assert b.qs[3, 5] == -127 and b.qs[3, 9] == -127


def test_q8k_known_device_cases():
    """grouped_expert.rs:235-240 cases against the closed form."""
    x = H.q8k_cases()
    b = O.quantize_q8_k(x)
    assert b.d[2] == 0.0 and np.all(b.qs[2] == 0)                 # all zero
    assert b.qs[1][np.argmax(np.abs(x[QK_K:2 * QK_K]))] == -127    # negative peak
    # ties: peak 0.5 (first, +0.5) -> iscale -254 -> +-0.5 * -254 = -+127
    assert np.all(b.qs[3][::2] == -127) and np.all(b.qs[3][1::2] == 127)
    # clamp: first element -8 is the peak -> iscale 127/8 -> +8 maps to +127
    assert b.qs[4][0] == -127 and np.all(b.qs[4][1:] == 127)


def test_dot_agrees_with_dequantize_then_multiply():   # dot.rs:284-322
    codes = np.array([32 + (i % 7) - 3 for i in range(QK_K)], np.uint8)
    w = H.q6k_block(codes, 2, 0.5)
    x = np.sin(np.arange(QK_K, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    a = O.quantize_q8_k(x)
    q = O.dot_q6k_q8k(w, a, QK_K)
    wf = O.dequantize(14, w, QK_K)
    exact = float(np.sum(wf.astype(np.float64) * x))
    scale = max(float(np.sum(np.abs(wf.astype(np.float64) * x))), 1e-6)
    assert abs(q - exact) / scale < 5e-3


def test_a_zero_weight_block_gives_zero():        # dot.rs:324-331
    w = H.q6k_block(np.full(QK_K, 32, np.uint8), 1, 1.0)
    a = O.quantize_q8_k(np.arange(QK_K, dtype=np.float32))
    assert O.dot_q6k_q8k(w, a, QK_K) == 0.0


def test_multiple_blocks_accumulate():            # dot.rs:333-346
    w1 = H.q6k_block(np.full(QK_K, 33, np.uint8), 1, 1.0)
    w = np.concatenate([w1, w1])
    a = O.quantize_q8_k(np.ones(2 * QK_K, np.float32))
    one = O.dot_q6k_q8k(w1, type(a)(a.d[:1], a.qs[:1], a.bsums[:1]), QK_K)
    two = O.dot_q6k_q8k(w, a, 2 * QK_K)
    assert abs(two - 2 * one) < 1e-3 * max(abs(one), 1.0)


def test_dot_single_element_brute_force():
    """One nonzero weight and one nonzero activation at every position e:
    the integer identity gives the exact answer d * a.d * sc * (q-32) * qa
    (a single product, so the ordered epilogue is exact too)."""
    rng = np.random.default_rng(3)
    for e in range(QK_K):
        codes = np.full(QK_K, 32, np.uint8)
        code = int(rng.integers(0, 64))
        codes[e] = code
        blk = H.q6k_block(codes, 0, 1.0)
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        blk[192:208] = sc.view(np.uint8)
        blk[208:210] = np.array([0.25], np.float16).view(np.uint8)
        qs = np.zeros((1, QK_K), np.int8)
        qa = int(rng.integers(-127, 128))
        qs[0, e] = qa
        a = O.Q8K(np.array([0.125], np.float32), qs, np.zeros((1, 16), np.int16))
        want = np.float32(0.25) * np.float32(0.125) * np.float32(int(sc[e // 16]) * (code - 32) * qa)
        assert O.dot_q6k_q8k(blk, a, QK_K) == want, e


def test_dot_matches_float64_within_epilogue_bound():
    """Random rows: the oracle equals sum_b d_b*a.d_b*aux(b) in exact arithmetic
    up to the f32 epilogue's rounding (a few ulp of the accumulated terms).
    A dropped class, a sign error or a wrong scale would be O(1)."""
    rng = np.random.default_rng(11)
    for trial in range(20):
        nb = int(rng.integers(1, 9))
        w = H.weights(1, nb, 100 + trial)
        x = rng.standard_normal(nb * QK_K).astype(np.float32)
        a = O.quantize_q8_k(x)
        got = O.dot_q6k_q8k(w, a, nb * QK_K)
        wf = O.dequantize(14, w, nb * QK_K).astype(np.float64)
        af = (a.qs.astype(np.float64) * a.d[:, None].astype(np.float64)).ravel()
        terms = wf * af
        exact = terms.sum()
        bound = 64 * 2.0 ** -24 * np.abs(terms).sum() + 1e-30
        assert abs(got - exact) <= bound, (trial, got, exact, bound)


def test_matvec_paths_compose():
    """R7 = quantize then per-row dots; R8 = dequantize then sequential sum."""
    rng = np.random.default_rng(5)
    rows, k = 9, 512
    w = H.weights(rows, k // QK_K, 42)
    x = rng.standard_normal(k).astype(np.float32)
    y = O.matvec_q6k(w, rows, k, x)
    a = O.quantize_q8_k(x)
    for r in range(rows):
        assert y[r] == O.dot_q6k_q8k(w[r * 420:(r + 1) * 420], a, k)
    wf = rng.standard_normal((rows, k)).astype(np.float32)
    yf = O.matvec_f32(wf, rows, k, x)
    for r in range(rows):
        s = np.float32(-0.0)
        for t in range(k):
            s = np.float32(s + np.float32(wf[r, t] * x[t]))
        assert yf[r] == s
