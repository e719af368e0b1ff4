"""The reference's own device layouts and the rest of its FFI, on the MI355X.

crates/llamd-rocm binds 91 functions. The weight-taking ones receive Q6_K in
the reference's layouts: ggml bytes uploaded verbatim (DevBuf::from_bytes,
crates/llamd-runtime/src/device.rs:231-233; DeviceWeights::upload,
crates/llamd-rocm/src/lib.rs:277-308) or the planar repack (PlanarWeights,
lib.rs:619-843; repack_q6k_planar, crates/llamd-quant/src/dot.rs:400-423).
Every Q6_K result here is compared bit for bit with the CPU oracle's
dot_q6k_q8k; every f32 piece with the oracle's restatement of the reference
CPU path (EXACT), except the F32 matvec (REDUCTION, as the header states).
"""
import ctypes as C

import numpy as np
import pytest

import helpers as H
from oracle import oracle as O

pytestmark = pytest.mark.gpu
QK_K = 256
Q6K = 14  # ggml type id


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def L():
    from llamd_rs_amd._lib import lib
    return lib()


def err():
    from llamd_rs_amd._lib import last_error
    return last_error()


def sync():
    assert L().llamd_fwd_sync() == 0
    assert L().llamd_fwd_last_error() == 0, err()


def planar(w: np.ndarray, rows: int, blocks: int):
    """repack_q6k_planar (dot.rs:400-423) and PlanarQ6K::layout (dot.rs:380-397)."""
    n = rows * blocks
    b = np.asarray(w, np.uint8).reshape(n, 210)
    out = np.concatenate([b[:, :128].ravel(), b[:, 128:192].ravel(), b[:, 192:208].ravel(),
                          b[:, 208:210].ravel()])
    off = (C.c_size_t * 4)(0, n * 128, n * 192, n * 208)
    return out, off


def acts(n_act, blocks, seed):
    """n_act Q8_K activations (the oracle's quantizer) as natural arrays."""
    xs = [H.sample(blocks * QK_K, seed + i) for i in range(n_act)]
    qa = [O.quantize_q8_k(x) for x in xs]
    q = np.concatenate([np.asarray(a.qs, np.int8).ravel() for a in qa])
    d = np.concatenate([np.asarray(a.d, np.float32) for a in qa])
    return qa, q, d


def dev(gpu, a):
    return gpu.DeviceBuffer.from_array(np.ascontiguousarray(a))


def down(buf, n, dtype=np.float32):
    return buf.download(np.empty(n, dtype))


# ---- Q6_K in ggml layout ---------------------------------------------------------

@pytest.mark.parametrize("rows,blocks", [(768, 8), (2048, 3), (100, 3), (17, 1)])
def test_raw_ggml_upload_matvec_and_dequant_exact(gpu, rows, blocks):
    """DeviceWeights::upload's llamd_rocm_upload pointer works unchanged."""
    w = H.weights(rows, blocks, rows + blocks)
    qa, q, d = acts(1, blocks, 5)
    p = L().llamd_rocm_upload(w.ctypes.data, w.nbytes)
    assert p, err()
    try:
        y = np.empty(rows, np.float32)
        assert L().llamd_rocm_matvec_q6k_resident(p, q.ctypes.data, d.ctypes.data, y.ctypes.data,
                                                  blocks, rows) == 0, err()
        assert bits_equal(y, O.matvec_q6k_act(w, rows, blocks * QK_K, qa[0]))
        # the tiled copy holds every byte: its dequantization is the reference's
        deq = np.empty(rows * blocks * QK_K, np.float32)
        assert L().llamd_hip_dequant_q6k(p, rows, blocks, deq.ctypes.data) == 0, err()
        assert bits_equal(deq, O.dequantize(Q6K, w, rows * blocks * QK_K))
    finally:
        L().llamd_rocm_release(p)


def test_fwd_launchers_on_raw_buffers(gpu):
    """llamd_fwd_matvec / _grouped / _grouped_pa / _x3 / _grouped_x2 / _splitk on
    DevBuf::from_bytes tensors (llamd.hip:1313-1466)."""
    rows, blocks, n_expert, n_used = 256, 8, 6, 3
    k = blocks * QK_K
    wa = H.synth(rows * n_expert, blocks, 0x31)
    wb = H.synth(rows * n_expert, blocks, 0x32)
    qa, q, d = acts(n_used, blocks, 40)
    ids = np.array([4, 0, 5], np.int32)
    A, B = dev(gpu, wa), dev(gpu, wb)
    Q, D, I = dev(gpu, q), dev(gpu, d), dev(gpu, ids)
    ya, yb = gpu.DeviceBuffer(rows * n_used * 4), gpu.DeviceBuffer(rows * n_used * 4)
    sl = lambda w, e: w[e * rows * blocks * 210:(e + 1) * rows * blocks * 210]
    want_a = [O.matvec_q6k_act(sl(wa, int(e)), rows, k, qa[0]) for e in ids]
    L().llamd_fwd_matvec(A.ptr, Q.ptr, D.ptr, ya.ptr, blocks, rows)
    sync()
    assert bits_equal(down(ya, rows), O.matvec_q6k_act(wa, rows, k, qa[0]))
    L().llamd_fwd_matvec_splitk(A.ptr, Q.ptr, D.ptr, ya.ptr, blocks, rows, 4)
    sync()
    assert bits_equal(down(ya, rows), O.matvec_q6k_act(wa, rows, k, qa[0]))
    L().llamd_fwd_matvec_grouped(A.ptr, I.ptr, Q.ptr, D.ptr, ya.ptr, blocks, rows, n_used)
    sync()
    assert bits_equal(down(ya, rows * n_used), np.concatenate(want_a))
    L().llamd_fwd_matvec_grouped_x2(A.ptr, B.ptr, I.ptr, Q.ptr, D.ptr, ya.ptr, yb.ptr, blocks, rows,
                                    n_used)
    sync()
    assert bits_equal(down(ya, rows * n_used), np.concatenate(want_a))
    assert bits_equal(down(yb, rows * n_used),
                      np.concatenate([O.matvec_q6k_act(sl(wb, int(e)), rows, k, qa[0]) for e in ids]))
    L().llamd_fwd_matvec_grouped_pa(A.ptr, I.ptr, Q.ptr, D.ptr, ya.ptr, blocks, rows, n_used)
    sync()
    assert bits_equal(down(ya, rows * n_used),
                      np.concatenate([O.matvec_q6k_act(sl(wa, int(e)), rows, k, qa[j])
                                      for j, e in enumerate(ids)]))
    # three matrices of one activation: rows 256 / 64 / 48 of different tensors
    o0, o1, o2 = (gpu.DeviceBuffer(rows * 4) for _ in range(3))
    L().llamd_fwd_matvec_x3(A.ptr, B.ptr, A.ptr, Q.ptr, D.ptr, o0.ptr, o1.ptr, o2.ptr, blocks, rows,
                            64, 48)
    sync()
    assert bits_equal(down(o1, 64), O.matvec_q6k_act(wb, 64, k, qa[0]))
    assert bits_equal(down(o2, 48), O.matvec_q6k_act(wa, 48, k, qa[0]))


def test_tiled_copy_follows_writes_and_frees(gpu):
    """A re-upload or memset of the bytes re-makes the copy; a freed and reused
    address never serves a stale copy."""
    rows, blocks = 64, 2
    k = blocks * QK_K
    qa, q, d = acts(1, blocks, 9)
    Q, D = dev(gpu, q), dev(gpu, d)
    y = gpu.DeviceBuffer(rows * 4)
    w1, w2 = H.weights(rows, blocks, 1), H.weights(rows, blocks, 2)
    W = dev(gpu, w1)
    L().llamd_fwd_matvec(W.ptr, Q.ptr, D.ptr, y.ptr, blocks, rows)
    sync()
    assert bits_equal(down(y, rows), O.matvec_q6k_act(w1, rows, k, qa[0]))
    W.upload(w2)
    L().llamd_fwd_matvec(W.ptr, Q.ptr, D.ptr, y.ptr, blocks, rows)
    sync()
    assert bits_equal(down(y, rows), O.matvec_q6k_act(w2, rows, k, qa[0]))
    assert L().llamd_fwd_memset(W.ptr, 0, w2.nbytes) == 0
    L().llamd_fwd_matvec(W.ptr, Q.ptr, D.ptr, y.ptr, blocks, rows)
    sync()
    zero = np.zeros_like(w2)
    assert bits_equal(down(y, rows), O.matvec_q6k_act(zero, rows, k, qa[0]))
    # free, then allocate the same size again (often the same address)
    addr = W.ptr
    W.close()
    W2 = dev(gpu, w1)
    L().llamd_fwd_matvec(W2.ptr, Q.ptr, D.ptr, y.ptr, blocks, rows)
    sync()
    assert bits_equal(down(y, rows), O.matvec_q6k_act(w1, rows, k, qa[0])), (addr, W2.ptr)


def test_memset_fills_every_byte(gpu):
    for n, off in [(1, 0), (17, 3), (4096, 0), (100003, 5)]:
        b = gpu.DeviceBuffer(n + off + 16)
        b.upload(np.full(n + off + 16, 0x11, np.uint8))
        addr = b.ptr + off
        assert L().llamd_fwd_memset(addr, 0x5A, n) == 0
        sync()
        got = down(b, n + off + 16, np.uint8)
        assert (got[off:off + n] == 0x5A).all() and (got[:off] == 0x11).all()
        assert (got[off + n:] == 0x11).all()


def test_foreign_and_short_weights_are_refused(gpu):
    rows, blocks = 32, 1
    qa, q, d = acts(1, blocks, 3)
    Q, D = dev(gpu, q), dev(gpu, d)
    y = gpu.DeviceBuffer(rows * 4)
    host = np.zeros(rows * 210, np.uint8)
    L().llamd_fwd_matvec(host.ctypes.data, Q.ptr, D.ptr, y.ptr, blocks, rows)
    assert "neither a tiled upload" in err()
    assert L().llamd_fwd_last_error() == -1
    short = gpu.DeviceBuffer(rows * 210 - 1)
    L().llamd_fwd_matvec(short.ptr, Q.ptr, D.ptr, y.ptr, blocks, rows)
    assert "31 rows" in err()
    assert L().llamd_fwd_last_error() == -1
    sync()


# ---- the planar repack -------------------------------------------------------------

def test_planar_entry_points_exact(gpu):
    rows, blocks, n_expert, n_used = 768, 8, 5, 4
    k = blocks * QK_K
    wa = H.synth(rows * n_expert, blocks, 0x41)
    wb = H.synth(rows * n_expert, blocks, 0x42)
    pa, fa = planar(wa, rows * n_expert, blocks)
    pb, fb = planar(wb, rows * n_expert, blocks)
    A, B = dev(gpu, pa), dev(gpu, pb)
    qa, q, d = acts(n_used, blocks, 70)
    ids = np.array([2, 4, 0, 2], np.int32)
    Q, D, I = dev(gpu, q), dev(gpu, d), dev(gpu, ids)
    sl = lambda w, e: w[e * rows * blocks * 210:(e + 1) * rows * blocks * 210]
    ya, yb = gpu.DeviceBuffer(rows * n_used * 4), gpu.DeviceBuffer(rows * n_used * 4)
    L().llamd_fwd_planar_matvec(A.ptr, fa, Q.ptr, D.ptr, ya.ptr, blocks, rows * n_expert)
    sync()
    assert bits_equal(down(ya, rows * n_used), O.matvec_q6k_act(wa, rows * n_used, k, qa[0]))
    L().llamd_fwd_planar_grouped(A.ptr, fa, I.ptr, Q.ptr, D.ptr, ya.ptr, blocks, rows, n_used)
    sync()
    want = np.concatenate([O.matvec_q6k_act(sl(wa, int(e)), rows, k, qa[0]) for e in ids])
    assert bits_equal(down(ya, rows * n_used), want)
    L().llamd_fwd_planar_grouped_x2(A.ptr, fa, B.ptr, fb, I.ptr, Q.ptr, D.ptr, ya.ptr, yb.ptr,
                                    blocks, rows, n_used)
    sync()
    assert bits_equal(down(ya, rows * n_used), want)
    assert bits_equal(down(yb, rows * n_used),
                      np.concatenate([O.matvec_q6k_act(sl(wb, int(e)), rows, k, qa[0]) for e in ids]))
    L().llamd_fwd_planar_grouped_pa(A.ptr, fa, I.ptr, Q.ptr, D.ptr, ya.ptr, blocks, rows, n_used)
    sync()
    assert bits_equal(down(ya, rows * n_used),
                      np.concatenate([O.matvec_q6k_act(sl(wa, int(e)), rows, k, qa[j])
                                      for j, e in enumerate(ids)]))
    o = [gpu.DeviceBuffer(rows * n_expert * 4) for _ in range(3)]
    L().llamd_fwd_planar_x3(A.ptr, fa, B.ptr, fb, A.ptr, fa, Q.ptr, D.ptr, o[0].ptr, o[1].ptr,
                            o[2].ptr, blocks, rows * n_expert, 512, 80)
    sync()
    assert bits_equal(down(o[0], rows * n_expert), O.matvec_q6k_act(wa, rows * n_expert, k, qa[0]))
    assert bits_equal(down(o[1], 512), O.matvec_q6k_act(wb, 512, k, qa[0]))
    assert bits_equal(down(o[2], 80), O.matvec_q6k_act(wa, 80, k, qa[0]))
    # host in, host out; and the bench entry point
    y = np.empty(rows, np.float32)
    assert L().llamd_rocm_planar_matvec(A.ptr, fa, q.ctypes.data, d.ctypes.data, y.ctypes.data,
                                        blocks, rows) == 0, err()
    assert bits_equal(y, O.matvec_q6k_act(wa, rows, k, qa[0]))
    ms = C.c_float(-1)
    assert L().llamd_rocm_planar_bench(A.ptr, fa, q.ctypes.data, d.ctypes.data, blocks, rows, 5,
                                       C.byref(ms)) == 0, err()
    assert ms.value > 0
    assert L().llamd_rocm_splitk_bench(A.ptr, q.ctypes.data, d.ctypes.data, blocks, rows, 2, 5,
                                       C.byref(ms)) == 0, err()  # the same bytes read as ggml


def test_planar_offsets_are_checked(gpu):
    rows, blocks = 16, 1
    pa, fa = planar(H.weights(rows, blocks, 8), rows, blocks)
    A = dev(gpu, pa)
    qa, q, d = acts(1, blocks, 1)
    Q, D = dev(gpu, q), dev(gpu, d)
    y = gpu.DeviceBuffer(rows * 4)
    bad = (C.c_size_t * 4)(0, 16 * 128, 16 * 192 + 1, 16 * 208)
    L().llamd_fwd_planar_matvec(A.ptr, bad, Q.ptr, D.ptr, y.ptr, blocks, rows)
    assert "planar offsets" in err()
    assert L().llamd_fwd_last_error() == -1
    sync()


def test_planar_first_use_inside_a_graph_capture(gpu):
    """device.rs captures the first token: the tiled copy is made during the
    capture (side stream), the graph then replays the matvec."""
    rows, blocks = 512, 8
    k = blocks * QK_K
    w = H.weights(rows, blocks, 77)
    pw, f = planar(w, rows, blocks)
    W = dev(gpu, pw)
    qa, q, d = acts(1, blocks, 12)
    Q, D = dev(gpu, q), dev(gpu, d)
    y = gpu.DeviceBuffer(rows * 4)
    want = O.matvec_q6k_act(w, rows, k, qa[0])
    assert L().llamd_fwd_begin_capture() == 0, err()
    L().llamd_fwd_planar_matvec(W.ptr, f, Q.ptr, D.ptr, y.ptr, blocks, rows)
    assert L().llamd_fwd_end_capture() == 0, err()
    try:
        for r in range(3):
            assert L().llamd_fwd_memset(y.ptr, 0xFF, rows * 4) == 0
            assert L().llamd_fwd_graph_launch() == 0, err()
            sync()
            assert bits_equal(down(y, rows), want), r
    finally:
        L().llamd_fwd_graph_destroy()


# ---- batched decode (llamd_batch.hip) ---------------------------------------------

@pytest.mark.parametrize("nseq", [1, 2, 5, 16])
def test_batched_matvecs_exact(gpu, nseq):
    rows, blocks = 576, 8
    k = blocks * QK_K
    w0, w1 = H.weights(rows, blocks, 91), H.weights(128, blocks, 92)
    qa, q, d = acts(nseq, blocks, 100)
    W0, W1, Q, D = dev(gpu, w0), dev(gpu, w1), dev(gpu, q), dev(gpu, d)
    y = gpu.DeviceBuffer(rows * nseq * 4)
    L().llamd_b_matvec(W0.ptr, Q.ptr, D.ptr, y.ptr, blocks, rows, nseq)
    sync()
    want0 = [O.matvec_q6k_act(w0, rows, k, a) for a in qa]
    assert bits_equal(down(y, rows * nseq), np.concatenate(want0))
    o = [gpu.DeviceBuffer(rows * nseq * 4) for _ in range(3)]
    L().llamd_b_matvec_x3(W0.ptr, W1.ptr, W0.ptr, Q.ptr, D.ptr, o[0].ptr, o[1].ptr, o[2].ptr, blocks,
                          rows, 128, 64, nseq)
    sync()
    assert bits_equal(down(o[0], rows * nseq), np.concatenate(want0))
    assert bits_equal(down(o[1], 128 * nseq),
                      np.concatenate([O.matvec_q6k_act(w1, 128, k, a) for a in qa]))
    assert bits_equal(down(o[2], 64 * nseq),
                      np.concatenate([O.matvec_q6k_act(w0, 64, k, a) for a in qa]))


@pytest.mark.parametrize("nseq", [1, 3, 8])
def test_batched_expert_matvecs_exact(gpu, nseq):
    rows, blocks, n_expert, n_used = 256, 8, 8, 4
    k = blocks * QK_K
    wa, wb = H.synth(rows * n_expert, blocks, 0x51), H.synth(rows * n_expert, blocks, 0x52)
    qa, q, d = acts(nseq, blocks, 200)
    rng = np.random.default_rng(nseq)
    ids = np.stack([rng.permutation(n_expert)[:n_used] for _ in range(nseq)]).astype(np.int32)
    A, B, Q, D, I = dev(gpu, wa), dev(gpu, wb), dev(gpu, q), dev(gpu, d), dev(gpu, ids)
    sl = lambda w, e: w[e * rows * blocks * 210:(e + 1) * rows * blocks * 210]
    ya, yb = gpu.DeviceBuffer(rows * n_used * nseq * 4), gpu.DeviceBuffer(rows * n_used * nseq * 4)
    L().llamd_b_grouped_x2(A.ptr, B.ptr, I.ptr, Q.ptr, D.ptr, ya.ptr, yb.ptr, blocks, rows, n_used,
                           nseq)
    sync()
    assert bits_equal(down(ya, rows * n_used * nseq), np.concatenate(
        [O.matvec_q6k_act(sl(wa, int(e)), rows, k, qa[s]) for s in range(nseq) for e in ids[s]]))
    assert bits_equal(down(yb, rows * n_used * nseq), np.concatenate(
        [O.matvec_q6k_act(sl(wb, int(e)), rows, k, qa[s]) for s in range(nseq) for e in ids[s]]))
    # down: one activation per (sequence, expert)
    pa, pq, pd = acts(nseq * n_used, blocks, 300)
    PQ, PD = dev(gpu, pq), dev(gpu, pd)
    L().llamd_b_grouped_pa(A.ptr, I.ptr, PQ.ptr, PD.ptr, ya.ptr, blocks, rows, n_used, nseq)
    sync()
    assert bits_equal(down(ya, rows * n_used * nseq), np.concatenate(
        [O.matvec_q6k_act(sl(wa, int(ids[s][j])), rows, k, pa[s * n_used + j])
         for s in range(nseq) for j in range(n_used)]))


def test_batched_f32_pieces_exact(gpu):
    nseq, n, n_expert, n_used = 3, 2048, 128, 8
    eps = 1e-6
    x = np.stack([H.sample(n, 10 + s) * 3 for s in range(nseq)]).astype(np.float32)
    wn = (1.0 + 0.1 * H.sample(n, 99)).astype(np.float32)
    X, WN = dev(gpu, x), dev(gpu, wn)
    out = gpu.DeviceBuffer(x.nbytes)
    L().llamd_b_rms_norm_mul(X.ptr, WN.ptr, out.ptr, n, nseq, C.c_float(eps))
    sync()
    want = np.concatenate([O.mul(O.rms_norm(x[s], 1, n, eps), wn) for s in range(nseq)])
    assert bits_equal(down(out, nseq * n), want)
    qs, dd, inv = gpu.DeviceBuffer(nseq * n), gpu.DeviceBuffer(nseq * n // 64), gpu.DeviceBuffer(64)
    L().llamd_b_rms_norm_quant(X.ptr, WN.ptr, out.ptr, qs.ptr, dd.ptr, inv.ptr, n, nseq,
                               C.c_float(eps))
    sync()
    assert bits_equal(down(out, nseq * n), want)
    qw = [O.quantize_q8_k(want[s * n:(s + 1) * n]) for s in range(nseq)]
    assert np.array_equal(down(qs, nseq * n, np.int8),
                          np.concatenate([np.asarray(a.qs, np.int8).ravel() for a in qw]))
    assert bits_equal(down(dd, nseq * n // 256), np.concatenate([a.d for a in qw]))
    L().llamd_b_quantize(X.ptr, qs.ptr, dd.ptr, nseq * n // 256)
    sync()
    qx = O.quantize_q8_k(x.ravel())
    assert np.array_equal(down(qs, nseq * n, np.int8), np.asarray(qx.qs, np.int8).ravel())
    # router: ids, weights and the softmax, per sequence
    lg = np.stack([H.sample(n_expert, 50 + s) * 4 for s in range(nseq)]).astype(np.float32)
    LG = dev(gpu, lg)
    ids, wts, probs = (gpu.DeviceBuffer(nseq * n_used * 4), gpu.DeviceBuffer(nseq * n_used * 4),
                       gpu.DeviceBuffer(nseq * n_expert * 4))
    L().llamd_b_router(LG.ptr, n_expert, n_used, ids.ptr, wts.ptr, probs.ptr, nseq)
    sync()
    got_ids = down(ids, nseq * n_used, np.int32).reshape(nseq, n_used)
    got_w = down(wts, nseq * n_used).reshape(nseq, n_used)
    got_p = down(probs, nseq * n_expert).reshape(nseq, n_expert)
    for s in range(nseq):
        r = O.route(lg[s], n_used)
        assert list(got_ids[s]) == list(r.experts) and bits_equal(got_w[s], r.weights)
        # route()'s probabilities (divided by the total, moe.rs:82-87)
        assert bits_equal(got_p[s][r.experts.astype(np.int64)], r.weights_raw)
        assert abs(float(got_p[s].astype(np.float64).sum()) - 1.0) < 1e-5
    # combine + residual, in routing order
    dn = np.stack([H.sample(n_used * n, 70 + s) for s in range(nseq)]).astype(np.float32)
    DN, RES = dev(gpu, dn), dev(gpu, x)
    L().llamd_b_moe_combine_add(DN.ptr, wts.ptr, RES.ptr, out.ptr, n_used, n, nseq)
    sync()
    want = np.empty((nseq, n), np.float32)
    for s in range(nseq):
        acc = np.zeros(n, np.float32)
        for e in range(n_used):
            acc = (acc + got_w[s, e] * dn[s, e * n:(e + 1) * n]).astype(np.float32)
        want[s] = x[s] + acc
    assert bits_equal(down(out, nseq * n), want)
    # add, silu * mul, argmax (ties and NaN at index 0 as the CPU path)
    L().llamd_b_add(X.ptr, RES.ptr, out.ptr, nseq * n)
    sync()
    assert bits_equal(down(out, nseq * n), (x + x).ravel())
    L().llamd_b_silu_mul(X.ptr, DN.ptr, out.ptr, nseq * n)
    sync()
    assert bits_equal(down(out, nseq * n), O.mul(O.silu(x.ravel()), dn.ravel()[:nseq * n]))
    v = np.stack([H.sample(151936, 7 + s) for s in range(nseq)]).astype(np.float32)
    v[1, 1000] = v[1, 5000] = 2.0
    v[2, 0] = np.nan
    V = dev(gpu, v)
    sv, si, am = gpu.DeviceBuffer(nseq * 64 * 4), gpu.DeviceBuffer(nseq * 64 * 4), gpu.DeviceBuffer(64)
    L().llamd_b_argmax(V.ptr, 151936, sv.ptr, si.ptr, am.ptr, 64, nseq)
    sync()
    assert list(down(am, nseq, np.int32)) == [O.argmax(v[s]) for s in range(nseq)] == \
        [O.argmax(v[0]), 1000, 0]
    # the router's F32 matvec: every sequence in one launch, each row the CPU
    # path's sequential fold bit for bit (model.rs:253-262)
    rw = H.sample(n_expert * n, 33).reshape(n_expert, n).astype(np.float32)
    RW = dev(gpu, rw)
    L().llamd_b_matvec_f32(RW.ptr, X.ptr, LG.ptr, n, n_expert, nseq)
    sync()
    got = down(LG, nseq * n_expert).reshape(nseq, n_expert)
    for s in range(nseq):
        assert bits_equal(got[s], O.matvec_f32(rw, n_expert, n, x[s])), s
    L().llamd_fwd_matvec_f32(RW.ptr, X.ptr, LG.ptr, n, n_expert)
    sync()
    assert bits_equal(down(LG, n_expert), O.matvec_f32(rw, n_expert, n, x[0]))
    # k outside the fold kernel's range (not a multiple of 256): FMA, within
    # REDUCTION x the rms of the outputs (grouped_expert.rs:147-175)
    k2 = 300
    X2 = dev(gpu, x.reshape(-1)[: nseq * k2])
    L().llamd_b_matvec_f32(RW.ptr, X2.ptr, LG.ptr, k2, n_expert, nseq)
    sync()
    got = down(LG, nseq * n_expert).reshape(nseq, n_expert)
    rw2 = rw.reshape(-1)[: n_expert * k2].reshape(n_expert, k2)
    for s in range(nseq):
        want = O.matvec_f32(rw2, n_expert, k2, x.reshape(-1)[s * k2:(s + 1) * k2])
        rms = float(np.sqrt((want.astype(np.float64) ** 2).mean()))
        assert np.abs(got[s].astype(np.float64) - want).max() <= O.REDUCTION * rms, s


# ---- the unsigned-activation form (llamd_udot.hip) ---------------------------------

def _bias(q):
    qb = (np.asarray(q, np.int8).ravel().view(np.uint8) ^ 0x80).astype(np.uint8)
    sb = qb.reshape(-1, 16).astype(np.int32).sum(axis=1).astype(np.int32)
    return qb, sb


def test_udot_quantizers_exact(gpu):
    nblocks = 24
    x = (H.sample(nblocks * QK_K, 4) * 5).astype(np.float32)
    qb, sb, d = np.empty(nblocks * QK_K, np.uint8), np.empty(nblocks * 16, np.int32), \
        np.empty(nblocks, np.float32)
    assert L().llamd_u_quantize_host(x.ctypes.data, nblocks, qb.ctypes.data, sb.ctypes.data,
                                     d.ctypes.data) == 0, err()
    a = O.quantize_q8_k(x)
    wqb, wsb = _bias(a.qs)
    assert np.array_equal(qb, wqb) and np.array_equal(sb, wsb) and bits_equal(d, a.d)
    # bias_sums of given signed quants
    Qs = dev(gpu, np.asarray(a.qs, np.int8).ravel())
    QB, SB = gpu.DeviceBuffer(qb.nbytes), gpu.DeviceBuffer(sb.nbytes)
    L().llamd_u_bias_sums(Qs.ptr, QB.ptr, SB.ptr, nblocks)
    sync()
    assert np.array_equal(down(QB, qb.size, np.uint8), wqb)
    assert np.array_equal(down(SB, sb.size, np.int32), wsb)
    # norm + quantize, two sequences
    n, nseq, eps = 2048, 2, 1e-6
    xs = x[:n * nseq]
    wn = (1.0 + 0.1 * H.sample(n, 6)).astype(np.float32)
    out = np.empty(n * nseq, np.float32)
    qb2, sb2, d2 = np.empty(n * nseq, np.uint8), np.empty(n * nseq // 16, np.int32), \
        np.empty(n * nseq // 256, np.float32)
    assert L().llamd_u_norm_quant_host(xs.ctypes.data, wn.ctypes.data, n, nseq, C.c_float(eps),
                                       out.ctypes.data, qb2.ctypes.data, sb2.ctypes.data,
                                       d2.ctypes.data) == 0, err()
    want = np.concatenate([O.mul(O.rms_norm(xs[s * n:(s + 1) * n], 1, n, eps), wn) for s in range(nseq)])
    assert bits_equal(out, want)
    aw = O.quantize_q8_k(want)
    wqb, wsb = _bias(aw.qs)
    assert np.array_equal(qb2, wqb) and np.array_equal(sb2, wsb) and bits_equal(d2, aw.d)
    L().llamd_u_set_tile(4)
    assert L().llamd_u_get_tile() == 4
    L().llamd_u_set_tile(3)
    assert L().llamd_u_get_tile() == 1


@pytest.mark.parametrize("nseq", [1, 4])
def test_udot_matvecs_exact(gpu, nseq):
    """The udot path's results are dot_q6k_q8k's bits (the reference's own
    udot kernels only reach REDUCTION)."""
    rows, blocks, n_expert, n_used = 512, 8, 4, 2
    k = blocks * QK_K
    wa, wb = H.synth(rows * n_expert, blocks, 0x61), H.synth(rows * n_expert, blocks, 0x62)
    pa, fa = planar(wa, rows * n_expert, blocks)
    pb, fb = planar(wb, rows * n_expert, blocks)
    A, B = dev(gpu, pa), dev(gpu, pb)
    qa, q, d = acts(nseq, blocks, 400)
    qb, sb = _bias(q)
    QB, SB, D = dev(gpu, qb), dev(gpu, sb), dev(gpu, d)
    y = gpu.DeviceBuffer(rows * n_expert * nseq * 4)
    L().llamd_u_matvec(A.ptr, fa, QB.ptr, SB.ptr, D.ptr, y.ptr, blocks, rows, nseq)
    sync()
    want = np.concatenate([O.matvec_q6k_act(wa, rows, k, a) for a in qa])
    assert bits_equal(down(y, rows * nseq), want)
    host = np.empty(rows * nseq, np.float32)
    assert L().llamd_u_matvec_host(A.ptr, fa, q.ctypes.data, d.ctypes.data, host.ctypes.data,
                                   blocks, rows, nseq) == 0, err()
    assert bits_equal(host, want)
    ms = C.c_float(-1)
    assert L().llamd_u_matvec_bench(A.ptr, fa, q.ctypes.data, d.ctypes.data, blocks, rows, nseq, 3,
                                    C.byref(ms)) == 0 and ms.value > 0, err()
    o = [gpu.DeviceBuffer(rows * nseq * 4) for _ in range(3)]
    L().llamd_u_x3(A.ptr, fa, B.ptr, fb, A.ptr, fa, QB.ptr, SB.ptr, D.ptr, o[0].ptr, o[1].ptr,
                   o[2].ptr, blocks, rows, 256, 32, nseq)
    sync()
    assert bits_equal(down(o[0], rows * nseq), want)
    assert bits_equal(down(o[1], 256 * nseq), np.concatenate([O.matvec_q6k_act(wb, 256, k, a) for a in qa]))
    assert bits_equal(down(o[2], 32 * nseq), np.concatenate([O.matvec_q6k_act(wa, 32, k, a) for a in qa]))
    ids = np.array([[3, 1], [0, 3], [2, 2], [1, 0]][:nseq], np.int32)
    I = dev(gpu, ids)
    sl = lambda w, e: w[e * rows * blocks * 210:(e + 1) * rows * blocks * 210]
    ya, yb = gpu.DeviceBuffer(rows * n_used * nseq * 4), gpu.DeviceBuffer(rows * n_used * nseq * 4)
    L().llamd_u_grouped_x2(A.ptr, fa, B.ptr, fb, I.ptr, QB.ptr, SB.ptr, D.ptr, ya.ptr, yb.ptr, blocks,
                           rows, n_used, nseq)
    sync()
    assert bits_equal(down(ya, rows * n_used * nseq), np.concatenate(
        [O.matvec_q6k_act(sl(wa, int(e)), rows, k, qa[s]) for s in range(nseq) for e in ids[s]]))
    assert bits_equal(down(yb, rows * n_used * nseq), np.concatenate(
        [O.matvec_q6k_act(sl(wb, int(e)), rows, k, qa[s]) for s in range(nseq) for e in ids[s]]))
    pa2, pq, pd = acts(nseq * n_used, blocks, 500)
    pqb, psb = _bias(pq)
    PQ, PS, PD = dev(gpu, pqb), dev(gpu, psb), dev(gpu, pd)
    L().llamd_u_grouped_pa(A.ptr, fa, I.ptr, PQ.ptr, PS.ptr, PD.ptr, ya.ptr, blocks, rows, n_used, nseq)
    sync()
    assert bits_equal(down(ya, rows * n_used * nseq), np.concatenate(
        [O.matvec_q6k_act(sl(wa, int(ids[s][j])), rows, k, pa2[s * n_used + j])
         for s in range(nseq) for j in range(n_used)]))


# ---- the f32 pieces of the decode step ----------------------------------------------

def test_embed_exact(gpu):
    vocab, blocks = 300, 8
    table = H.weights(vocab, blocks, 12)
    T = dev(gpu, table)
    n = blocks * QK_K
    deq = O.dequantize(Q6K, table, vocab * n).reshape(vocab, n)
    out = gpu.DeviceBuffer(3 * n * 4)
    L().llamd_fwd_embed(T.ptr, 257, out.ptr, blocks)
    sync()
    assert bits_equal(down(out, n), deq[257])
    meta = dev(gpu, np.array([299, 4, 17, 9, 0, 1], np.int32))
    L().llamd_fwd_embed_meta(T.ptr, meta.ptr, out.ptr, blocks)
    sync()
    assert bits_equal(down(out, n), deq[299])
    L().llamd_b_embed(T.ptr, meta.ptr, out.ptr, blocks, 3)
    sync()
    assert bits_equal(down(out, 3 * n), np.concatenate([deq[299], deq[17], deq[0]]))
    L().llamd_fwd_embed(T.ptr, vocab, out.ptr, blocks)  # outside the table
    assert "outside the table" in err() and L().llamd_fwd_last_error() == -1
    sync()


def _qk(x, w, heads, hd, eps):
    return O.mul(O.rms_norm(x, heads, hd, eps), np.tile(w, heads)) if w is not None else x


def test_rope_norm_and_cache_store_exact(gpu):
    n_head, n_head_kv, hd, base, eps = 32, 4, 128, 1.0e7, 1e-6
    kv_dim = n_head_kv * hd
    q = (H.sample(n_head * hd, 1) * 2).astype(np.float32)
    k = (H.sample(kv_dim, 2) * 2).astype(np.float32)
    v = H.sample(kv_dim, 3)
    qw, kw = (1 + 0.1 * H.sample(hd, 4)).astype(np.float32), (1 + 0.1 * H.sample(hd, 5)).astype(np.float32)
    Qd = dev(gpu, q)
    L().llamd_fwd_rope(Qd.ptr, 37, n_head, hd, C.c_float(base))
    sync()
    assert bits_equal(down(Qd, q.size), O.rope(q, n_head, hd, 37, base))
    pos = 1234
    meta = dev(gpu, np.array([5, pos], np.int32))
    Qd.upload(q)
    QW, KW = dev(gpu, qw), dev(gpu, kw)
    L().llamd_fwd_norm_rope(Qd.ptr, QW.ptr, n_head, hd, meta.ptr, C.c_float(base), C.c_float(eps))
    sync()
    assert bits_equal(down(Qd, q.size), O.rope(_qk(q, qw, n_head, hd, eps), n_head, hd, pos, base))
    max_kv = 2048
    KC, VC = gpu.DeviceBuffer(max_kv * kv_dim * 4), gpu.DeviceBuffer(max_kv * kv_dim * 4)
    Kd, Vd = dev(gpu, k), dev(gpu, v)
    L().llamd_fwd_k_norm_rope_store(Kd.ptr, KW.ptr, Vd.ptr, KC.ptr, VC.ptr, n_head_kv, hd, kv_dim,
                                    meta.ptr, C.c_float(base), C.c_float(eps))
    sync()
    kr = O.rope(_qk(k, kw, n_head_kv, hd, eps), n_head_kv, hd, pos, base)
    kc = down(KC, max_kv * kv_dim).reshape(max_kv, kv_dim)
    vc = down(VC, max_kv * kv_dim).reshape(max_kv, kv_dim)
    assert bits_equal(kc[pos], kr) and bits_equal(vc[pos], v) and bits_equal(down(Kd, kv_dim), kr)
    L().llamd_fwd_kv_store(KC.ptr, VC.ptr, Vd.ptr, Kd.ptr, 7, kv_dim)
    sync()
    kc = down(KC, max_kv * kv_dim).reshape(max_kv, kv_dim)
    assert bits_equal(kc[7], v)
    # two sequences at their own positions, each with its own cache slice
    nseq = 2
    meta2 = dev(gpu, np.array([1, 9, 2, 300], np.int32))
    q2 = np.concatenate([q, (q * 0.5).astype(np.float32)])
    k2 = np.concatenate([k, (k * 0.25).astype(np.float32)])
    v2 = np.concatenate([v, (v * 2).astype(np.float32)])
    Q2, K2, V2 = dev(gpu, q2), dev(gpu, k2), dev(gpu, v2)
    L().llamd_b_norm_rope(Q2.ptr, QW.ptr, n_head, hd, meta2.ptr, nseq, C.c_float(base), C.c_float(eps))
    KC2, VC2 = gpu.DeviceBuffer(nseq * max_kv * kv_dim * 4), gpu.DeviceBuffer(nseq * max_kv * kv_dim * 4)
    L().llamd_b_k_norm_rope_store(K2.ptr, KW.ptr, V2.ptr, KC2.ptr, VC2.ptr, n_head_kv, hd, kv_dim,
                                  max_kv, meta2.ptr, nseq, C.c_float(base), C.c_float(eps))
    sync()
    gq = down(Q2, q2.size).reshape(nseq, -1)
    kc2 = down(KC2, nseq * max_kv * kv_dim).reshape(nseq, max_kv, kv_dim)
    vc2 = down(VC2, nseq * max_kv * kv_dim).reshape(nseq, max_kv, kv_dim)
    for s, p in enumerate([9, 300]):
        qs = q2[s * q.size:(s + 1) * q.size]
        ks = k2[s * kv_dim:(s + 1) * kv_dim]
        assert bits_equal(gq[s], O.rope(_qk(qs, qw, n_head, hd, eps), n_head, hd, p, base))
        assert bits_equal(kc2[s, p], O.rope(_qk(ks, kw, n_head_kv, hd, eps), n_head_kv, hd, p, base))
        assert bits_equal(vc2[s, p], v2[s * kv_dim:(s + 1) * kv_dim])


def test_rope_past_the_table(gpu):
    """Positions at and past the 32768-row cos / sin table (Qwen3-30B-A3B
    allows 40960): the reference kernel computes theta for any position
    (llamd_forward.hip:419-440). Below the table the rotation is the CPU's bit
    for bit; past it theta = pos / powf(base, 2i/hd) is still the CPU's and
    only the device sincosf differs, so every value is within REDUCTION of
    CpuBackend::rope under close. The K store lands at its row when the cache
    holds it and is skipped (no write outside the cache) when it does not."""
    n_head, n_head_kv, hd, base, eps = 4, 2, 128, 1.0e6, 1e-6
    kv_dim = n_head_kv * hd
    q = (H.sample(n_head * hd, 41) * 2).astype(np.float32)
    Qd = dev(gpu, q)

    def near(got, want):
        rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.maximum(np.abs(got), np.abs(want)), 1.0)
        return rel.max() <= O.REDUCTION
    for pos in (32767, 32768, 40959, 1_000_000):
        Qd.upload(q)
        L().llamd_fwd_rope(Qd.ptr, pos, n_head, hd, C.c_float(base))
        sync()
        got, want = down(Qd, q.size), O.rope(q, n_head, hd, pos, base)
        assert near(got, want), pos
        if pos < 32768:
            assert bits_equal(got, want)
    qw = (1 + 0.1 * H.sample(hd, 42)).astype(np.float32)
    QW = dev(gpu, qw)
    meta = dev(gpu, np.array([1, 40000], np.int32))
    Qd.upload(q)
    L().llamd_fwd_norm_rope(Qd.ptr, QW.ptr, n_head, hd, meta.ptr, C.c_float(base), C.c_float(eps))
    sync()
    assert near(down(Qd, q.size), O.rope(_qk(q, qw, n_head, hd, eps), n_head, hd, 40000, base))
    # K store: a cache of 40001 rows holds position 40000; one of 39000 does not
    k = (H.sample(kv_dim, 43) * 2).astype(np.float32)
    v = H.sample(kv_dim, 44)
    kw = (1 + 0.1 * H.sample(hd, 45)).astype(np.float32)
    KW, Vd = dev(gpu, kw), dev(gpu, v)
    kr = O.rope(_qk(k, kw, n_head_kv, hd, eps), n_head_kv, hd, 40000, base)
    for rows in (40001, 39000):
        Kd = dev(gpu, k)
        KC, VC = gpu.DeviceBuffer(rows * kv_dim * 4), gpu.DeviceBuffer(rows * kv_dim * 4)
        KC.upload(np.zeros(rows * kv_dim, np.float32))
        VC.upload(np.zeros(rows * kv_dim, np.float32))
        L().llamd_fwd_k_norm_rope_store(Kd.ptr, KW.ptr, Vd.ptr, KC.ptr, VC.ptr, n_head_kv, hd, kv_dim,
                                        meta.ptr, C.c_float(base), C.c_float(eps))
        sync()
        assert near(down(Kd, kv_dim), kr)
        kc = down(KC, rows * kv_dim).reshape(rows, kv_dim)
        vc = down(VC, rows * kv_dim).reshape(rows, kv_dim)
        if rows > 40000:
            assert near(kc[40000], kr) and bits_equal(vc[40000], v)
        else:
            assert not kc.any() and not vc.any()


def test_attention_exact(gpu):
    n_head, n_head_kv, hd, n_kv, max_kv = 32, 4, 128, 211, 512
    kv_dim = n_head_kv * hd
    q = H.sample(n_head * hd, 21)
    kc = H.sample(max_kv * kv_dim, 22).reshape(max_kv, kv_dim)
    vc = H.sample(max_kv * kv_dim, 23).reshape(max_kv, kv_dim)
    Qd, KC, VC = dev(gpu, q), dev(gpu, kc), dev(gpu, vc)
    out, scores = gpu.DeviceBuffer(q.nbytes), gpu.DeviceBuffer(n_head * max_kv * 4)
    want = O.attend(q, kc[:n_kv], vc[:n_kv], n_kv, n_head, n_head_kv, hd)
    L().llamd_fwd_attention(Qd.ptr, KC.ptr, VC.ptr, out.ptr, scores.ptr, n_head, n_head_kv, hd, n_kv)
    sync()
    assert bits_equal(down(out, q.size), want)
    meta = dev(gpu, np.array([0, n_kv - 1], np.int32))
    L().llamd_fwd_attention_meta(Qd.ptr, KC.ptr, VC.ptr, out.ptr, scores.ptr, n_head, n_head_kv, hd,
                                 meta.ptr, max_kv)
    sync()
    assert bits_equal(down(out, q.size), want)
    # two sequences over their own cache slices
    q2 = np.concatenate([q, H.sample(q.size, 24)])
    kc2 = np.concatenate([kc, H.sample(max_kv * kv_dim, 25).reshape(max_kv, kv_dim)])
    vc2 = np.concatenate([vc, H.sample(max_kv * kv_dim, 26).reshape(max_kv, kv_dim)])
    Q2, K2, V2 = dev(gpu, q2), dev(gpu, kc2), dev(gpu, vc2)
    meta2 = dev(gpu, np.array([0, n_kv - 1, 0, 39], np.int32))
    out2 = gpu.DeviceBuffer(q2.nbytes)
    L().llamd_b_attention(Q2.ptr, K2.ptr, V2.ptr, out2.ptr, scores.ptr, n_head, n_head_kv, hd, max_kv,
                          meta2.ptr, 2)
    sync()
    got = down(out2, q2.size).reshape(2, -1)
    assert bits_equal(got[0], want)
    assert bits_equal(got[1], O.attend(q2[q.size:], kc2[max_kv:max_kv + 40], vc2[max_kv:max_kv + 40],
                                       40, n_head, n_head_kv, hd))
    L().llamd_fwd_attention(Qd.ptr, KC.ptr, VC.ptr, out.ptr, scores.ptr, n_head, n_head_kv, hd, 20000)
    assert "positions" in err() and L().llamd_fwd_last_error() == -1
    sync()


# ---- llamd-tensor Backend ops ------------------------------------------------------

def test_backend_ops_exact(gpu):
    rows, n = 5, 1000
    x = (H.sample(rows * n, 61) * 7).astype(np.float32)
    y = H.sample(rows * n, 62)
    X, Y = dev(gpu, x), dev(gpu, y)
    out = gpu.DeviceBuffer(x.nbytes)
    assert L().llamd_hip_be_rms_norm(X.ptr, out.ptr, rows, n, C.c_float(1e-6)) == 0, err()
    sync()
    assert bits_equal(down(out, x.size), O.rms_norm(x, rows, n, 1e-6))
    assert L().llamd_hip_be_softmax(X.ptr, out.ptr, rows, n) == 0
    sync()
    assert bits_equal(down(out, x.size), np.concatenate([O.softmax(x[r * n:(r + 1) * n])
                                                          for r in range(rows)]))
    assert L().llamd_hip_be_silu(X.ptr, out.ptr, x.size) == 0
    sync()
    assert bits_equal(down(out, x.size), O.silu(x))
    for fn, want in [(L().llamd_hip_be_add, x + y), (L().llamd_hip_be_mul, O.mul(x, y))]:
        assert fn(X.ptr, Y.ptr, out.ptr, x.size) == 0
        sync()
        assert bits_equal(down(out, x.size), want)
    assert L().llamd_hip_be_scale(X.ptr, C.c_float(0.3), out.ptr, x.size) == 0
    sync()
    assert bits_equal(down(out, x.size), (x * np.float32(0.3)).astype(np.float32))
    # matmul: w [m][k] x [n][k] -> [n][m], each sum in order
    m, nn, k = 70, 3, 333
    w = H.sample(m * k, 63)
    xm = H.sample(nn * k, 64)
    Wd, XM, OM = dev(gpu, w), dev(gpu, xm), gpu.DeviceBuffer(m * nn * 4)
    assert L().llamd_hip_be_matmul(Wd.ptr, XM.ptr, OM.ptr, m, nn, k) == 0
    sync()
    assert bits_equal(down(OM, m * nn), np.concatenate(
        [O.matvec_f32(w, m, k, xm[j * k:(j + 1) * k]) for j in range(nn)]))
    # rope with a position per row
    heads, hd = 4, 64
    xr = H.sample(3 * heads * hd, 65)
    XR = dev(gpu, xr)
    pos = np.array([0, 77, 4096], np.uint32)
    assert L().llamd_hip_be_rope(XR.ptr, 3, heads * hd, pos.ctypes.data, hd, C.c_float(1.0e6),
                                 C.c_float(1.0)) == 0, err()
    assert bits_equal(down(XR, xr.size), np.concatenate(
        [O.rope(xr[r * heads * hd:(r + 1) * heads * hd], heads, hd, int(pos[r]), 1.0e6)
         for r in range(3)]))
    ids = np.array([4, 0, 4, 2], np.uint32)
    G = gpu.DeviceBuffer(4 * n * 4)
    assert L().llamd_hip_be_get_rows(X.ptr, rows, n, ids.ctypes.data, 4, G.ptr) == 0
    sync()
    assert bits_equal(down(G, 4 * n), x.reshape(rows, n)[ids.astype(np.int64)])
    bad = np.array([rows], np.uint32)
    assert L().llamd_hip_be_get_rows(X.ptr, rows, n, bad.ctypes.data, 1, G.ptr) == -1
    assert "outside" in err()
    assert L().llamd_fwd_free_mem() > 0
    assert L().llamd_batch_max_seq() == 16


def test_host_calls_from_several_threads(gpu):
    """Host-in/host-out calls from 6 threads at once (ctypes drops the GIL, so
    they overlap in the library): raw ggml uploads, two threads sharing one
    pointer's first use (one tiled copy is made), every result the oracle's
    bits, on every repetition."""
    import threading
    shapes = [(768, 8), (2048, 3), (100, 3)]
    ws = [H.weights(r, b, 900 + r + b) for r, b in shapes]
    ptrs = [L().llamd_rocm_upload(w.ctypes.data, w.nbytes) for w in ws]
    assert all(ptrs), err()
    work = [0, 1, 2, 0, 1, 2]  # threads 3-5 share their pointer with 0-2
    wants, inputs = [], []
    for t, i in enumerate(work):
        rows, blocks = shapes[i]
        qa, q, d = acts(1, blocks, 70 + t)
        inputs.append((q, d))
        wants.append(O.matvec_q6k_act(ws[i], rows, blocks * QK_K, qa[0]))
    failures = []

    def run(t):
        i = work[t]
        rows, blocks = shapes[i]
        q, d = inputs[t]
        y = np.empty(rows, np.float32)
        for rep in range(20):
            rc = L().llamd_rocm_matvec_q6k_resident(ptrs[i], q.ctypes.data, d.ctypes.data,
                                                     y.ctypes.data, blocks, rows)
            if rc != 0 or not bits_equal(y, wants[t]):
                failures.append((t, rep, rc))
                return

    threads = [threading.Thread(target=run, args=(t,)) for t in range(len(work))]
    try:
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=60)
        assert not any(th.is_alive() for th in threads)
        assert not failures, failures
    finally:
        for p in ptrs:
            L().llamd_rocm_release(p)


def _fold_rows(k, rng):
    """Router rows that stress the in-order fold: random products, exact
    cancellation, zeros of both signs, a wide exponent range, values on a
    coarse grid (ties of round-to-nearest), subnormals, non-finite terms and
    a sum that overflows; with x = 1 each row's products are its values."""
    f32 = np.float32
    rows = []
    for t in range(6):
        rows.append((rng.normal(0, 0.02, k) * rng.normal(0, 1, k)).astype(f32))
    v = rng.normal(0, 1, k // 2).astype(f32)
    rows.append(np.concatenate([v, -v[::-1]]))
    v = rng.normal(0, 1, k).astype(f32)
    v[1::2] = -v[::2]
    rows.append(v)
    rows.append(np.zeros(k, f32))
    rows.append(-np.zeros(k, f32))
    v = -np.zeros(k, f32)
    v[k // 3] = 0.0
    rows.append(v)
    rows.append((rng.normal(0, 1, k) * 2.0 ** rng.integers(-60, 60, k)).astype(f32))
    rows.append((rng.integers(-1000, 1000, k) * 2.0 ** -10).astype(f32))
    v = np.full(k, f32(1.0))
    v[::3] = f32(2.0 ** -24)
    rows.append(v)
    rows.append((rng.normal(0, 1, k) * 1e-39).astype(f32))
    v = rng.normal(0, 1, k).astype(f32)
    v[:2] = f32(3e38)
    rows.append(v)
    v = rng.normal(0, 1, k).astype(f32)
    v[5] = np.nan
    rows.append(v)
    v = rng.normal(0, 1, k).astype(f32)
    v[k - 1] = np.inf
    rows.append(v)
    rows.append(rng.normal(1, 0.1, k).astype(f32))
    v = (rng.normal(0, 1, k) * 2.0 ** -20).astype(f32)
    v[0] = f32(1.0)
    v[k // 2] = f32(-1.0)
    rows.append(v)
    return np.stack(rows)


@pytest.mark.parametrize("k", [256, 768, 2048])
def test_router_fold_adversarial_rows(gpu, k):
    """The F32 router matvec's in-order fold (model.rs:253-262) on rows built
    to break a shortcut: every logit bit-identical to the CPU's sequential
    sum from -0.0, NaN and inf where the CPU has them."""
    rng = np.random.default_rng(k)
    rw = _fold_rows(k, rng)
    n_expert = rw.shape[0]
    x = np.ones(k, np.float32)
    RW, X, LG = dev(gpu, rw), dev(gpu, x), gpu.DeviceBuffer(n_expert * 4)
    L().llamd_fwd_matvec_f32(RW.ptr, X.ptr, LG.ptr, k, n_expert)
    sync()
    got = down(LG, n_expert)
    want = O.matvec_f32(rw, n_expert, k, x)
    bad = [i for i in range(n_expert)
           if not (np.isnan(want[i]) and np.isnan(got[i]))
           and got[i:i + 1].view(np.uint32)[0] != want[i:i + 1].view(np.uint32)[0]]
    assert not bad, [(i, got[i], want[i]) for i in bad]
    # and a real router on a normal activation, every row
    rw2 = (rng.normal(0, 0.02, (128, k))).astype(np.float32)
    x2 = rng.normal(0, 1, k).astype(np.float32)
    RW2, X2, LG2 = dev(gpu, rw2), dev(gpu, x2), gpu.DeviceBuffer(128 * 4)
    L().llamd_fwd_matvec_f32(RW2.ptr, X2.ptr, LG2.ptr, k, 128)
    sync()
    assert bits_equal(down(LG2, 128), O.matvec_f32(rw2, 128, k, x2))
