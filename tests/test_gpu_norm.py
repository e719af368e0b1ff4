"""RMSNorm (+ weight, + Q8_K) on the MI355X against the oracle: EXACT
(bit-identical), including the in-order f32 sum that a parallel reduction
would not reproduce. The last test runs the attention block's front end:
rms_norm_quant then one llamd_fwd_matvec_x3 launch for Q, K and V."""
import zlib

import numpy as np
import pytest

import helpers as H
from oracle import oracle as O

pytestmark = pytest.mark.gpu
QK_K = 256


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _lib():
    from llamd_rs_amd._lib import lib
    return lib()


def _sync():
    L = _lib()
    assert L.llamd_fwd_sync() == 0 and L.llamd_fwd_last_error() == 0


def _inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    x[:8] = [4096.0, 1, 1, 1, 1, 1, 1, 1]   # the in-order sum drops the ones
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return x, w


@pytest.mark.parametrize("n,eps", [(2048, 1e-6), (4096, 1e-6), (768, 0.0), (100, 1e-5)])
def test_rms_norm_mul_exact(gpu, n, eps):                       # llamd-cpu lib.rs:55-75
    L = _lib()
    x, w = _inputs(n, n)
    dx, dw, do = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(n * 4)
    L.llamd_fwd_rms_norm_mul(dx.ptr, dw.ptr, do.ptr, n, eps)
    _sync()
    want = O.mul(O.rms_norm(x, 1, n, eps), w)
    assert bits_equal(do.download(np.empty(n, np.float32)), want)


def test_head_rms_norm_mul_exact(gpu):                           # layer.rs:62-79
    L = _lib()
    n_head, hd, eps = 32, 128, 1e-6
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(n_head * hd) * 5).astype(np.float32)
    x[hd:2 * hd] *= 1e-3                     # heads normalise separately
    w = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    dx, dw, do = (gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(w),
                  gpu.DeviceBuffer(x.nbytes))
    L.llamd_fwd_head_rms_norm_mul(dx.ptr, dw.ptr, do.ptr, n_head, hd, eps)
    _sync()
    want = O.mul(O.rms_norm(x, n_head, hd, eps), np.tile(w, n_head))
    assert bits_equal(do.download(np.empty(x.size, np.float32)), want)


@pytest.mark.parametrize("n", [2048, 256, 4096])
def test_rms_norm_quant_exact(gpu, n):                           # llamd_forward.hip:845-855
    L = _lib()
    eps = 1e-6
    x, w = _inputs(n, 11 + n)
    nb = n // QK_K
    dx, dw = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(w)
    do, dq, dd, di = (gpu.DeviceBuffer(n * 4), gpu.DeviceBuffer(n), gpu.DeviceBuffer(nb * 4),
                      gpu.DeviceBuffer(4))
    L.llamd_fwd_rms_norm_quant(dx.ptr, dw.ptr, do.ptr, dq.ptr, dd.ptr, di.ptr, n, eps)
    _sync()
    want = O.mul(O.rms_norm(x, 1, n, eps), w)
    assert bits_equal(do.download(np.empty(n, np.float32)), want)
    q = O.quantize_q8_k(want)
    assert np.array_equal(dq.download(np.empty(n, np.int8)), np.asarray(q.qs).ravel())
    assert bits_equal(dd.download(np.empty(nb, np.float32)), np.asarray(q.d).ravel())


def test_rms_norm_of_zeros_with_eps(gpu):
    L = _lib()
    n = 512
    x, w = np.zeros(n, np.float32), np.ones(n, np.float32)
    dx, dw, do = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(n * 4)
    L.llamd_fwd_rms_norm_mul(dx.ptr, dw.ptr, do.ptr, n, 1e-6)
    _sync()
    assert bits_equal(do.download(np.empty(n, np.float32)), O.mul(O.rms_norm(x, 1, n, 1e-6), w))


def test_attention_front_end_norm_then_qkv(gpu):                 # layer.rs:100-118
    """attn_norm -> Q8_K -> Q (4096 rows), K, V (512 rows) in one x3 launch:
    every projection bit-identical to the CPU path's matvec_quant."""
    L = _lib()
    n_embd, eps, blocks = 2048, 1e-6, 8
    x, w = _inputs(n_embd, 5)
    shapes = [(4096, 41), (512, 42), (512, 43)]
    ws = [H.weights(r, blocks, s) for r, s in shapes]
    dws = [gpu.DeviceWeights.upload(m, r, blocks) for m, (r, _) in zip(ws, shapes)]
    dx, dw = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(w)
    dq, dd = gpu.DeviceBuffer(n_embd), gpu.DeviceBuffer(blocks * 4)
    outs = [gpu.DeviceBuffer(r * 4) for r, _ in shapes]
    L.llamd_fwd_rms_norm_quant(dx.ptr, dw.ptr, None, dq.ptr, dd.ptr, None, n_embd, eps)
    L.llamd_fwd_matvec_x3(dws[0].ptr, dws[1].ptr, dws[2].ptr, dq.ptr, dd.ptr, outs[0].ptr,
                          outs[1].ptr, outs[2].ptr, blocks, 4096, 512, 512)
    _sync()
    attn_norm = O.mul(O.rms_norm(x, 1, n_embd, eps), w)
    for m, (r, _), o in zip(ws, shapes, outs):
        want = O.matvec_q6k(m, r, n_embd, attn_norm)             # model.rs:241-276
        assert bits_equal(o.download(np.empty(r, np.float32)), want)


def test_many_short_rows_exercise_sqrt_and_divide(gpu):
    """8192 rows of 3 (per-head layout): thousands of distinct sums, so the
    correctly rounded sqrt and divide are checked value by value."""
    L = _lib()
    n_head, hd = 8192, 3
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(n_head * hd) * np.exp(rng.uniform(-6, 6, n_head * hd))).astype(np.float32)
    w = np.ones(hd, np.float32)
    for eps in (0.0, 1e-6):
        dx, dw, do = (gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(w),
                      gpu.DeviceBuffer(x.nbytes))
        L.llamd_fwd_head_rms_norm_mul(dx.ptr, dw.ptr, do.ptr, n_head, hd, eps)
        _sync()
        got = do.download(np.empty(x.size, np.float32))
        want = O.mul(O.rms_norm(x, n_head, hd, eps), np.tile(w, n_head))
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, (eps, bad[:5], got[bad[:5]], want[bad[:5]])


def _rows(kind, rows, n, rng):
    g = rng.standard_normal((rows, n))
    if kind == "normal":
        x = g
    elif kind == "outliers":           # a few channels 100x, as in real hidden states
        x = g * np.where(rng.random((rows, n)) < 0.01, 100.0, 1.0)
    elif kind == "tiny_first":         # the first squares far below the rest
        x = g.copy()
        x[:, :2] = np.array([1e-7, 1e-5])[:n]
    elif kind == "halves":             # squares k/4: increments that tie at coarse grids
        x = rng.integers(-40, 40, (rows, n)) / 2.0
    elif kind == "sparse":
        x = np.where(rng.random((rows, n)) < 0.7, 0.0, g)
    elif kind == "huge_range":         # too many uncertain steps: the serial fallback
        x = g * 10.0 ** rng.integers(-15, 15, (rows, n))
    elif kind == "subnormal_squares":
        x = g * 1e-22
    elif kind == "overflow":           # the sum overflows to inf part way
        x = g * 1e18
    elif kind == "constant":
        x = np.full((rows, n), 0.3)
    elif kind == "specials":           # inf and NaN in some rows
        x = g.copy()
        x[1, n // 2] = np.inf
        x[2, 0] = np.nan
        x[3, n - 1] = -np.inf
    return x.astype(np.float32)


KINDS = ["normal", "outliers", "tiny_first", "halves", "sparse", "huge_range",
         "subnormal_squares", "overflow", "constant", "specials"]


@pytest.mark.parametrize("n", [2048, 768, 8192, 129, 1])
@pytest.mark.parametrize("kind", KINDS)
def test_row_sum_of_squares_in_order(gpu, kind, n):              # llamd-cpu lib.rs:55-66
    """The workgroup's certified-increment replay of the in-order sum
    against the oracle's one-by-one f32 fold, row by row (bit-identical
    output rows; a sum off by one ulp moves the scale in about half the
    rows). Covers certain/uncertain mixes, ties, zeros, subnormal squares,
    overflow, inf/NaN and the serial fallback."""
    L = _lib()
    rows = 16 if n == 8192 else 64
    x = _rows(kind, rows, n, np.random.default_rng(zlib.crc32(f"{kind}/{n}".encode())))
    w = np.ones(n, np.float32)
    for eps in (0.0, 1e-6):
        dx, dw, do = (gpu.DeviceBuffer.from_array(x.ravel()), gpu.DeviceBuffer.from_array(w),
                      gpu.DeviceBuffer(x.nbytes))
        L.llamd_fwd_head_rms_norm_mul(dx.ptr, dw.ptr, do.ptr, rows, n, eps)
        _sync()
        got = do.download(np.empty(x.size, np.float32))
        want = O.mul(O.rms_norm(x.ravel(), rows, n, eps), np.tile(w, rows))
        differ = (got.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(got) & np.isnan(want))
        bad = np.flatnonzero(differ)
        assert bad.size == 0, (kind, n, eps, bad[:5] // n)
