"""The device-pointer launchers of the forward path (llamd.hip:1313-1466,
llamd_forward.hip:701-916) on the MI355X: multi-matrix launches, the expert
combine, and graph capture/replay of the decode layer. Q6_K outputs and the
layer output are compared bit for bit (EXACT)."""
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


def _dev_act(gpu, act):
    return gpu.DeviceBuffer.from_array(np.asarray(act.qs, np.int8)), gpu.DeviceBuffer.from_array(
        np.asarray(act.d, np.float32))


def test_matvec_x3_one_launch_three_shapes(gpu):                  # llamd.hip:1400-1411
    """Q, K, V of a Qwen3 attention block: rows 4096 / 512 / 512, k 2048."""
    L = _lib()
    blocks = 8
    shapes = [(4096, 31), (512, 32), (512, 33)]
    ws = [H.weights(r, blocks, s) for r, s in shapes]
    act = O.quantize_q8_k(H.sin_ramp(blocks * QK_K, 0.013))
    dws = [gpu.DeviceWeights.upload(w, r, blocks) for w, (r, _) in zip(ws, shapes)]
    outs = [gpu.DeviceBuffer(r * 4) for r, _ in shapes]
    q, d = _dev_act(gpu, act)
    L.llamd_fwd_matvec_x3(dws[0].ptr, dws[1].ptr, dws[2].ptr, q.ptr, d.ptr, outs[0].ptr, outs[1].ptr,
                          outs[2].ptr, blocks, shapes[0][0], shapes[1][0], shapes[2][0])
    _sync()
    for w, (r, _), o in zip(ws, shapes, outs):
        got = o.download(np.empty(r, np.float32))
        assert bits_equal(got, O.matvec_q6k_act(w, r, blocks * QK_K, act))
    # the split-K spelling gives the same bits whatever nsub says
    L.llamd_fwd_matvec_x3_splitk(dws[0].ptr, dws[1].ptr, dws[2].ptr, q.ptr, d.ptr, outs[0].ptr,
                                 outs[1].ptr, outs[2].ptr, blocks, shapes[0][0], shapes[1][0],
                                 shapes[2][0], 2)
    _sync()
    got = outs[1].download(np.empty(512, np.float32))
    assert bits_equal(got, O.matvec_q6k_act(ws[1], 512, blocks * QK_K, act))


def test_matvec_x3_refuses_a_foreign_pointer(gpu):
    L = _lib()
    blocks = 1
    w = gpu.DeviceWeights.upload(H.weights(16, blocks, 5), 16, blocks)
    junk = gpu.DeviceBuffer(1024)  # 4 rows of ggml Q6_K: too few for 16
    o = gpu.DeviceBuffer(64)
    q, d = gpu.DeviceBuffer(256), gpu.DeviceBuffer(4)
    L.llamd_fwd_matvec_x3(w.ptr, junk.ptr, w.ptr, q.ptr, d.ptr, o.ptr, o.ptr, o.ptr, blocks, 16, 16, 16)
    from llamd_rs_amd._lib import last_error
    assert "4 rows" in last_error()
    # the refusal is reported once by llamd_fwd_last_error, then cleared
    assert L.llamd_fwd_last_error() == -1
    _sync()


def test_grouped_x2_equals_two_grouped_launches(gpu):            # llamd.hip:1413-1424
    L = _lib()
    rows, k, n_expert = 768, 2048, 6
    blocks = k // QK_K
    wa = H.synth(rows * n_expert, blocks, 0x11)
    wb = H.synth(rows * n_expert, blocks, 0x22)
    act = O.quantize_q8_k(H.cos_ramp(k, 0.011))
    ids = np.array([4, 0, 5, 5, 2], np.int32)
    da = gpu.DeviceWeights.upload_experts(wa, n_expert, rows, blocks)
    db = gpu.DeviceWeights.upload_experts(wb, n_expert, rows, blocks)
    di = gpu.DeviceBuffer.from_array(ids)
    q, d = _dev_act(gpu, act)
    oa, ob = gpu.DeviceBuffer(ids.size * rows * 4), gpu.DeviceBuffer(ids.size * rows * 4)
    L.llamd_fwd_matvec_grouped_x2(da.ptr, db.ptr, di.ptr, q.ptr, d.ptr, oa.ptr, ob.ptr, blocks, rows,
                                  ids.size)
    _sync()
    per = rows * blocks * 210
    for w, o in ((wa, oa), (wb, ob)):
        got = o.download(np.empty(ids.size * rows, np.float32))
        want = np.concatenate([O.matvec_q6k_act(w[e * per:(e + 1) * per], rows, k, act) for e in ids])
        assert bits_equal(got, want)


def test_moe_combine_without_residual(gpu):                       # llamd_forward.hip:813-817
    L = _lib()
    n_used, n_embd = 8, 2048
    rng = np.random.default_rng(5)
    down = rng.standard_normal((n_used, n_embd)).astype(np.float32)
    w = rng.random(n_used).astype(np.float32)
    dd, dw = gpu.DeviceBuffer.from_array(down), gpu.DeviceBuffer.from_array(w)
    o = gpu.DeviceBuffer(n_embd * 4)
    L.llamd_fwd_moe_combine(dd.ptr, dw.ptr, o.ptr, n_used, n_embd)
    _sync()
    want = np.zeros(n_embd, np.float32)             # layer.rs:245-258, expert order
    for e in range(n_used):
        want = want + w[e] * down[e]
    assert bits_equal(o.download(np.empty(n_embd, np.float32)), want)


def test_graph_replays_equal_eager_calls(gpu):                   # llamd_forward.hip:879-910
    """Capture four decode-layer calls, replay the graph three times with new
    inputs uploaded (and eager work run) between replays: every replay must
    give the eager bits for the inputs it saw."""
    from llamd_rs_amd import synth
    L = _lib()
    n_embd, n_ff, n_expert, n_used = 512, 256, 16, 4
    router = synth.normal(70, 0.02, n_expert * n_embd).reshape(n_expert, n_embd)
    gate = synth.q6k_matrix(71, 0.02, n_expert * n_ff, n_embd)
    up = synth.q6k_matrix(72, 0.02, n_expert * n_ff, n_embd)
    down = synth.q6k_matrix(73, 0.02, n_expert * n_embd, n_ff)
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    ntok = 4
    X = gpu.DeviceBuffer(ntok * n_embd * 4)
    R = gpu.DeviceBuffer(ntok * n_embd * 4)
    Y = gpu.DeviceBuffer(ntok * n_embd * 4)

    def calls():
        for t in range(ntok):
            off = t * n_embd * 4
            assert L.llamd_hip_moe_forward(layer.handle, X.ptr + off, R.ptr + off, Y.ptr + off, 0) == 0

    try:
        X.upload(np.zeros(ntok * n_embd, np.float32))
        R.upload(np.zeros(ntok * n_embd, np.float32))
        _sync()
        assert L.llamd_fwd_begin_capture() == 0
        calls()
        assert L.llamd_fwd_end_capture() == 0
        assert L.llamd_fwd_has_graph() == 1
        for rep in range(3):
            x = synth.normal(80 + rep, 1.0, ntok * n_embd)
            r = synth.normal(90 + rep, 1.0, ntok * n_embd)
            X.upload(x)
            R.upload(r)
            calls()                                    # eager
            _sync()
            eager = Y.download(np.empty(ntok * n_embd, np.float32))
            Y.upload(np.full(ntok * n_embd, np.nan, np.float32))
            _sync()
            assert L.llamd_fwd_graph_launch() == 0    # replay
            _sync()
            replay = Y.download(np.empty(ntok * n_embd, np.float32))
            assert bits_equal(replay, eager), rep
            want, _, _, _ = O.moe_layer(x[:n_embd], r[:n_embd], n_embd, n_ff, n_expert, n_used,
                                        router, gate, up, down)
            assert bits_equal(replay[:n_embd], want), rep
    finally:
        L.llamd_fwd_graph_destroy()
        layer.close()
    assert L.llamd_fwd_has_graph() == 0
