"""The float epilogue of dot_q6k_q8k in the reference's order, pinned by
inputs where any other order changes the last bit.

dot.rs:174-195: per block, the integer class sums aux32[c] (c = weight index
mod 8) are exact; then sums[c] += (f16(d) * y.d) * aux32[c] as f32, block
after block, and the result is sum over c = 0..7 of sums[c], in class order.
Three rows are built so that the integer part is known exactly and the float
part has one right answer:

  A  lane order: sums = [2^24, 1, 1, 1, 1, 1, 1, 1]. In order every + 1 is a
     tie at 2^24 and rounds to even: 2^24. Summed in reverse (7 first) the
     answer is 2^24 + 8; pairwise (s0 + s1) + (s2 + s3) + ... it is 2^24 + 6.
  B  block order: class 0 gets 2^24, then 1, then 1 from three blocks:
     ((0 + 2^24) + 1) + 1 = 2^24; adding the last two blocks first gives
     2^24 + 2.
  C  the (d * y.d) * aux association and no FMA: block 0 leaves
     sums[0] = 591; block 1 has d = f16 0x3E3C (1.55859375),
     y.d = f32 0x3FD2E081 (1.64747632...) and aux32[0] = 710. The rounded
     steps give 0x4516E19A; a fused multiply-add gives 0x4516E199, and
     d * (y.d * aux) gives 0x4516E198.

The expected values of A and B follow by hand from round-to-nearest-even
(written above); those of C are IEEE single steps worked with numpy's
float32 scalars, independent of the oracle's code. The same rows go through
the oracle (CPU) and the device matvec (GPU).
"""
import numpy as np
import pytest

QK_K = 256
F16_ONE, F16_FOUR = 0x3C00, 0x4400


def _set_code(blk, e, code):
    """The 6-bit code of weight e in a ggml Q6_K block (lib.rs:181-226)."""
    h, i = divmod(e, 128)
    q4, l = divmod(i, 32)
    lo = h * 64 + l + (q4 & 1) * 32
    sh = 4 * (q4 >> 1)
    blk[lo] = (int(blk[lo]) & ~(0xF << sh) & 0xFF) | ((code & 0xF) << sh)
    hi = 128 + h * 32 + l
    sh2 = 2 * q4
    blk[hi] = (int(blk[hi]) & ~(3 << sh2) & 0xFF) | (((code >> 4) & 3) << sh2)


def _block(d_bits, scale, terms):
    """One Q6_K block and its Q8_K activation block. terms: {element:
    (q8, w)} with w = code - 32; every other weight has w = 0 and q8 = 0.
    All 16 group scales are `scale`."""
    blk = np.zeros(210, np.uint8)
    qs = np.zeros(QK_K, np.int8)
    for e in range(QK_K):
        _set_code(blk, e, 32)
    for e, (q8, w) in terms.items():
        _set_code(blk, e, w + 32)
        qs[e] = q8
    blk[192:208] = np.int8(scale).view(np.uint8)
    blk[208:210] = np.array([d_bits], np.uint16).view(np.uint8)
    return blk, qs


def _decompose(target):
    """{element: (q8, w)} of class 0 with sum q8 * w = target, scale 1."""
    terms, m = {}, 0
    while target:
        q8 = int(np.clip(target // 31 if target > 0 else -((-target) // 31), -127, 127))
        if q8 == 0:
            q8 = 1 if target > 0 else -1
            w = target if abs(target) <= 31 else (31 if target > 0 else -31)
            w = int(np.clip(w, -32, 31))
        else:
            w = 31
        terms[8 * m] = (q8, w)
        target -= q8 * w
        m += 1
    assert m <= 32
    return terms


def cases():
    f32 = np.float32
    two22 = {8 * m: (-64, -32) for m in range(32)}  # 32 x 64 * (-64) * (-32) = 2^22
    ones = {c: (1, 1) for c in range(1, 8)}          # aux32[c] = 1, c = 1..7, group 0
    d_c = int(np.array([1.55859375], np.float16).view(np.uint16)[0])
    ad_c = np.array([0x3FD2E081], np.uint32).view(np.float32)[0]
    out = {
        "A": ([(F16_FOUR, 64, two22, f32(1.0)), (F16_ONE, 1, ones, f32(1.0))], 0x4B800000),
        "B": ([(F16_FOUR, 64, two22, f32(1.0)), (F16_ONE, 1, {0: (1, 1)}, f32(1.0)),
               (F16_ONE, 1, {0: (1, 1)}, f32(1.0))], 0x4B800000),
        "C": ([(F16_ONE, 1, _decompose(591), f32(1.0)), (d_c, 1, _decompose(710), ad_c)],
              0x4516E19A),
    }
    rows = {}
    for name, (blocks, want) in out.items():
        w = np.concatenate([_block(d, s, t)[0] for d, s, t, _ in blocks])
        qs = np.stack([_block(d, s, t)[1] for d, s, t, _ in blocks])
        ad = np.array([a for *_, a in blocks], np.float32)
        rows[name] = (w, qs, ad, want)
    return rows


def _alternatives():
    """The wrong orders named in the docstring, worked step by step."""
    f = np.float32
    s = [f(2.0 ** 24)] + [f(1.0)] * 7
    rev = f(0.0)
    for v in reversed(s):
        rev = f(rev + v)
    pair = f(0.0)
    for i in range(0, 8, 2):
        pair = f(pair + f(s[i] + s[i + 1]))
    blocks_late = f(f(2.0 ** 24) + f(f(1.0) + f(1.0)))
    d = f(np.float16(1.55859375))
    ad = np.array([0x3FD2E081], np.uint32).view(np.float32)[0]
    dd = f(d * ad)
    ref = f(f(591.0) + f(dd * f(710.0)))
    from fractions import Fraction
    fma = f(float(Fraction(float(dd)) * 710 + 591))  # one rounding (exact in double first)
    assoc = f(f(591.0) + f(d * f(ad * f(710.0))))
    return rev, pair, blocks_late, ref, fma, assoc


def test_wrong_orders_differ_from_the_expected_bits():
    rev, pair, blocks_late, ref, fma, assoc = _alternatives()
    bits = lambda v: int(np.array([v], np.float32).view(np.uint32)[0])
    assert bits(rev) == 0x4B800004 and bits(pair) == 0x4B800003   # 2^24 + 8, 2^24 + 6
    assert bits(blocks_late) == 0x4B800001                         # 2^24 + 2
    assert bits(ref) == 0x4516E19A
    assert len({bits(ref), bits(fma), bits(assoc)}) == 3


@pytest.mark.parametrize("name", ["A", "B", "C"])
def test_oracle_epilogue_order(name):
    from oracle import oracle as O
    w, qs, ad, want = cases()[name]
    a = O.Q8K(ad, qs, np.zeros((len(ad), 16), np.int16))
    got = O.dot_q6k_q8k(w, a, len(ad) * QK_K)
    assert int(np.array([got], np.float32).view(np.uint32)[0]) == want


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["A", "B", "C"])
def test_device_epilogue_order(gpu, name):
    """The batch-1 matvec (MFMA integer part, ordered float epilogue) and the
    batched one (16 tokens per MFMA) on the same rows."""
    w, qs, ad, want = cases()[name]
    nb = len(ad)
    act = gpu.BlockQ8K(ad, qs, np.zeros((nb, 16), np.int16))
    dw = gpu.DeviceWeights.upload(w, 1, nb)
    try:
        got = dw.matvec(act)
        assert int(got.view(np.uint32)[0]) == want
        got_b = dw.matvec_batched([act] * 3)
        assert all(int(v) == want for v in got_b.reshape(3, -1)[:, 0].view(np.uint32))
    finally:
        dw.close()
