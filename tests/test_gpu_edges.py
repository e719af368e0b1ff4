"""Edge cases on the device path: refused arguments (checked before any
device work, as the reference's safe wrappers do, crates/llamd-rocm/src/lib.rs:434-470),
all-zero activations (Q8_K d = 0), out-of-range expert ids on the device-pointer
prefill, and the largest routing the kernels take (256 experts, 16 used)."""
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


def make_layer(n_embd, n_ff, n_expert, seed):
    from llamd_rs_amd import synth
    router = synth.normal(seed, 0.02, n_expert * n_embd).reshape(n_expert, n_embd)
    gate = synth.q6k_matrix(seed + 1, 0.02, n_expert * n_ff, n_embd)
    up = synth.q6k_matrix(seed + 2, 0.02, n_expert * n_ff, n_embd)
    down = synth.q6k_matrix(seed + 3, 0.02, n_expert * n_embd, n_ff)
    return router, gate, up, down


def test_refused_arguments_return_errors(gpu):
    from llamd_rs_amd._lib import lib, last_error
    L = lib()
    w = gpu.DeviceWeights.upload(H.weights(32, 1, 3), 32, 1)
    q = np.zeros(QK_K, np.int8)
    d = np.zeros(1, np.float32)
    y = np.zeros(64, np.float32)
    p = lambda a: a.ctypes.data
    try:
        # wrong block count, zero rows, more rows than uploaded
        assert L.llamd_rocm_matvec_q6k_resident(w.ptr, p(q), p(d), p(y), 2, 32) == -1
        assert L.llamd_rocm_matvec_q6k_resident(w.ptr, p(q), p(d), p(y), 1, 0) == -1
        assert L.llamd_rocm_matvec_q6k_resident(w.ptr, p(q), p(d), p(y), 1, 33) == -1
        # device memory too small to hold the rows as ggml Q6_K (19 rows of
        # one block fit in 4096 bytes), and memory the library never handed out
        junk = gpu.DeviceBuffer(4096)
        assert L.llamd_rocm_matvec_q6k_resident(junk.ptr, p(q), p(d), p(y), 1, 32) == -1
        assert "19 rows" in last_error()
        junk.close()
        host = np.zeros(32 * 210, np.uint8)
        assert L.llamd_rocm_matvec_q6k_resident(p(host), p(q), p(d), p(y), 1, 32) == -1
        assert "neither a tiled upload" in last_error()
        # null buffers, empty input
        assert L.llamd_rocm_matvec_q6k_resident(w.ptr, None, p(d), p(y), 1, 32) == -1
        assert L.llamd_rocm_quantize_q8k(None, 1, p(q), p(d), None) == -1
        assert L.llamd_rocm_quantize_q8k(p(np.zeros(QK_K, np.float32)), 0, p(q), p(d), None) == -1
        # routing: no experts requested, more than there are
        lg = np.zeros(8, np.float32)
        ids = np.zeros(16, np.int32)
        wt = np.zeros(16, np.float32)
        assert L.llamd_hip_route(p(lg), 8, 0, p(ids), p(wt)) == -1
        assert L.llamd_hip_route(p(lg), 8, 9, p(ids), p(wt)) == -1
        assert last_error()
        # the library still works after the refusals
        got = w.matvec(gpu.quantize_q8k_on_device(H.sample(QK_K, 4)))
        assert bits_equal(got, O.matvec_q6k(H.weights(32, 1, 3), 32, QK_K, H.sample(QK_K, 4)))
    finally:
        w.close()


def test_moe_layer_refuses_bad_calls(gpu):
    from llamd_rs_amd._lib import lib
    L = lib()
    n_embd, n_ff, n_expert, n_used = 256, 256, 8, 2
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 60)
    p = lambda a: a.ctypes.data
    # shapes the kernels cannot take are refused at create
    assert not L.llamd_hip_moe_create(p(router), p(gate), p(up), p(down), n_embd, n_ff, n_expert, 17)
    assert not L.llamd_hip_moe_create(p(router), p(gate), p(up), p(down), n_embd, n_ff, n_expert, 0)
    assert not L.llamd_hip_moe_create(p(router), p(gate), p(up), p(down), 300, n_ff, n_expert, n_used)
    assert not L.llamd_hip_moe_create(p(router), p(gate), p(up), p(down), 4096, n_ff, n_expert, n_used)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    try:
        assert L.llamd_hip_moe_forward(layer.handle, None, None, None, 0) == -1
        assert L.llamd_hip_moe_prefill(layer.handle, None, None, None, None, 1) == -1
        x = np.zeros((1, n_embd), np.float32)
        with pytest.raises(gpu.HipError):
            layer.prefill(x, np.array([[0, n_expert]], np.int32), np.ones((1, n_used), np.float32))
        with pytest.raises(gpu.HipError):
            layer.prefill(x, np.array([[-1, 0]], np.int32), np.ones((1, n_used), np.float32))
        # still usable
        out, r, _ = layer.forward(np.ones(n_embd, np.float32))
        want, _, ids, _ = O.moe_layer(np.ones(n_embd, np.float32), np.zeros(n_embd, np.float32),
                                      n_embd, n_ff, n_expert, n_used, router, gate, up, down)
        assert list(r.experts) == list(ids) and np.array_equal(out, want)
    finally:
        layer.close()


def test_device_prefill_out_of_range_ids_add_nothing(gpu):
    """Device ids are not read by the host: a pair with an id outside
    [0, n_expert) is left out of every group and adds no term; the other pairs
    of its token are unchanged."""
    from llamd_rs_amd import synth
    from llamd_rs_amd._lib import lib
    n_embd, n_ff, n_expert, n_used = 256, 256, 8, 4
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 80)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    n_tok = 20
    x = synth.normal(81, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
    ids, w = synth.zipf_routing(82, 1.1, n_tok, n_expert, n_used)
    ids = ids.astype(np.int32)
    bad = ids.copy()
    bad[3, 1] = n_expert
    bad[7, 0] = -5
    bad[7, 3] = 1 << 30
    bufs = [gpu.DeviceBuffer.from_array(a) for a in (x, bad, w)]
    dout = gpu.DeviceBuffer(n_tok * n_embd * 4)
    try:
        assert lib().llamd_hip_moe_prefill(layer.handle, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr,
                                           dout.ptr, n_tok) == 0
        got = dout.download(np.empty((n_tok, n_embd), np.float32))
        # expected: the same pairs with weight 0 on a valid expert (0 * finite adds +-0)
        w0 = w.copy()
        fixed = bad.copy()
        for t, k in ((3, 1), (7, 0), (7, 3)):
            w0[t, k] = 0.0
            fixed[t, k] = 0
        want = O.moe_ffn_tokens(x, n_embd, n_ff, n_expert, gate, up, down, fixed, w0)
        assert np.array_equal(got, want)
        # the tokens with only valid ids are bit-identical to a clean call
        clean = layer.prefill(x, ids, w)
        others = [t for t in range(n_tok) if t not in (3, 7)]
        assert bits_equal(got[others], clean[others])
    finally:
        for b in bufs + [dout]:
            b.close()
        layer.close()


def test_zero_activation_gives_zero_outputs(gpu):
    """An all-zero activation quantizes to d = 0 and zero quants
    (crates/llamd-quant/src/dot.rs:102-106); every row is then the reference's
    sum of zero terms, for the single and the batched kernel."""
    rows, blocks = 48, 4
    w = H.weights(rows, blocks, 9)
    x = np.zeros(blocks * QK_K, np.float32)
    act = gpu.quantize_q8k_on_device(x)
    assert not np.any(act.d) and not np.any(act.qs)
    want = O.matvec_q6k(w, rows, blocks * QK_K, x)
    dw = gpu.DeviceWeights.upload(w, rows, blocks)
    try:
        assert bits_equal(dw.matvec(act), want)
        got_b = dw.matvec_batched([act, act, act])
        for s in range(3):
            assert bits_equal(got_b[s], want), s
    finally:
        dw.close()


def test_largest_routing_256_experts_16_used(gpu):
    rng = np.random.default_rng(4)
    for t in range(20):
        lg = (rng.standard_normal(256) * (1 + t)).astype(np.float32)
        lg[rng.integers(0, 256, 5)] = lg.max()          # ties at the top
        want = O.route(lg, 16)
        got = gpu.route(lg, 16)
        assert [int(e) for e in got.experts] == [int(e) for e in want.experts], t
        assert bits_equal(got.weights, want.weights), t


def test_moe_layer_256_experts_top16(gpu):
    """The largest decode layer the kernels take (256 experts, 16 used, 16
    waves in the down kernel), bit-identical to the CPU path."""
    from llamd_rs_amd import synth
    n_embd, n_ff, n_expert, n_used = 512, 256, 256, 16
    router, gate, up, down = make_layer(n_embd, n_ff, n_expert, 30)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    try:
        for t in range(3):
            x = synth.normal(40 + t, 1.0, n_embd)
            res = synth.normal(50 + t, 1.0, n_embd)
            want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate, up, down)
            out, r, lg_used = layer.forward(x, res)
            assert bits_equal(lg_used, lg), t
            assert [int(e) for e in r.experts] == [int(e) for e in ids], t
            assert bits_equal(r.weights, w), t
            assert bits_equal(out, want), t
        # and the grouped prefill on the same layer
        n_tok = 24
        xs = synth.normal(60, 1.0, n_tok * n_embd).reshape(n_tok, n_embd)
        pids, pw = synth.zipf_routing(61, 1.1, n_tok, n_expert, n_used)
        got = layer.prefill(xs, pids.astype(np.int32), pw)
        assert bits_equal(got, O.moe_ffn_tokens(xs, n_embd, n_ff, n_expert, gate, up, down, pids, pw))
    finally:
        layer.close()


def test_measurement_helpers(gpu):
    """The calibration entry points bench.py times with: the copy moves the
    bytes, the read-only and empty launches run and refuse bad arguments."""
    import ctypes as C
    from llamd_rs_amd._lib import lib
    L = lib()
    n = 1 << 20
    src = gpu.DeviceBuffer.from_array(np.arange(n // 4, dtype=np.int32))
    dst = gpu.DeviceBuffer(n)
    assert L.llamd_hip_copy_calibration(dst.ptr, src.ptr, n) == 0
    assert np.array_equal(dst.download(np.empty(n // 4, np.int32)), np.arange(n // 4, dtype=np.int32))
    assert L.llamd_hip_copy_calibration(dst.ptr, src.ptr, n - 4) == -1
    ptrs = (C.c_void_p * 3)(src.ptr, dst.ptr, src.ptr)
    assert L.llamd_hip_read_many(ptrs, n, 48, 3) == 0
    assert L.llamd_hip_read_many(None, 0, 48, 5) == 0       # empty kernels
    assert L.llamd_hip_read_many(ptrs, n - 8, 48, 3) == -1  # not a multiple of 16
    assert L.llamd_hip_read_many(ptrs, n, 0, 3) == -1       # no workgroups
    assert L.llamd_hip_read_many(None, n, 48, 3) == -1      # bytes but no sources
    assert L.llamd_fwd_sync() == 0
    src.close()
    dst.close()


def test_void_launchers_report_refusals(gpu):
    """The llamd_fwd_* launchers return nothing; one that refuses its
    arguments queues nothing, and the next llamd_fwd_last_error says -1
    once (the reference's wrappers check it after their synchronise)."""
    from llamd_rs_amd._lib import lib, last_error
    L = lib()
    x = gpu.DeviceBuffer(4 * 8192)
    out = gpu.DeviceBuffer(4 * 8192)
    wts = gpu.DeviceBuffer(4 * 64)
    assert L.llamd_fwd_sync() == 0 and L.llamd_fwd_last_error() == 0
    cases = [
        lambda: L.llamd_fwd_moe_combine(x.ptr, wts.ptr, out.ptr, 17, 256),     # n_used > 16
        lambda: L.llamd_fwd_moe_combine_add(x.ptr, wts.ptr, x.ptr, out.ptr, 0, 256),
        lambda: L.llamd_fwd_rms_norm_mul(x.ptr, x.ptr, out.ptr, 0, 1e-6),      # n = 0
        lambda: L.llamd_fwd_rms_norm_quant(x.ptr, x.ptr, out.ptr, out.ptr, out.ptr, out.ptr, 100, 1e-6),
    ]
    try:
        for i, call in enumerate(cases):
            call()
            assert L.llamd_fwd_sync() == 0, i
            assert L.llamd_fwd_last_error() == -1, i
            assert last_error(), i
            assert L.llamd_fwd_last_error() == 0, i   # reported once
    finally:
        x.close(); out.close(); wts.close()
