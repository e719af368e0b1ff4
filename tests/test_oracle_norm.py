"""The oracle's rms_norm (CpuBackend::rms_norm, llamd-cpu/src/lib.rs:55-75),
pinned by the reference's own tests and by properties that a plausible
mistake (a pairwise or f64 sum, a missing eps, rsqrt instead of 1/sqrt, a
global instead of per-row norm) would break."""
import numpy as np

from oracle import oracle as O

F32_ULP = 1.2e-7     # llamd-core tolerance
ATTENTION = 1e-5


def f32_seq_rms(x, eps):
    """The reference's arithmetic, one f32 operation at a time."""
    x = np.asarray(x, np.float32)
    s = np.float32(0.0)
    for v in x:
        s = np.float32(s + np.float32(v * v))
    scale = np.float32(np.float32(1.0) / np.sqrt(np.float32(np.float32(s / np.float32(x.size)) + np.float32(eps))))
    return (x * scale).astype(np.float32)


def test_rms_norm_matches_hand_computation():                    # lib.rs:237-244
    out = O.rms_norm([3.0, 4.0], 1, 2, 0.0)
    rms = np.sqrt(np.float32(12.5))
    assert O.close(out[0], 3.0 / rms, F32_ULP) and O.close(out[1], 4.0 / rms, F32_ULP)


def test_rms_norm_is_per_row_not_global():                       # lib.rs:247-259
    out = O.rms_norm([3.0, 4.0, 300.0, 400.0], 2, 2, 0.0)
    assert O.close(out[0], out[2], ATTENTION) and O.close(out[1], out[3], ATTENTION)


def test_rms_norm_sums_sequentially_in_f32():
    # 4096^2 = 2^24: adding 1.0 to it rounds back to 2^24 (ties to even), so
    # the in-order f32 sum drops the seven ones; pairwise or f64 sums keep them
    x = np.array([4096.0] + [1.0] * 7, np.float32)
    got = O.rms_norm(x, 1, 8, 0.0)
    want = f32_seq_rms(x, 0.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    exact = x / np.sqrt(np.mean(x.astype(np.float64) ** 2))
    assert not np.array_equal(got, exact.astype(np.float32))


def test_rms_norm_matches_the_stepwise_f32_restatement():
    rng = np.random.default_rng(7)
    for n, eps in ((2048, 1e-6), (128, 1e-6), (768, 0.0), (5, 1e-3)):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        got = O.rms_norm(x, 1, n, eps)
        assert np.array_equal(got.view(np.uint32), f32_seq_rms(x, eps).view(np.uint32)), n


def test_rms_norm_eps_and_float64_bound():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(4 * 512) * 0.01).astype(np.float32)
    for eps in (0.0, 1e-6, 1e-2):
        got = O.rms_norm(x, 4, 512, eps).reshape(4, 512)
        xr = x.reshape(4, 512).astype(np.float64)
        want = xr / np.sqrt((xr ** 2).mean(axis=1, keepdims=True) + eps)
        assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 1e-5, eps
