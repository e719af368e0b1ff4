"""llamd_hip_lmhead_forward_noalloc: the LM-head call with its scratch in a
file-scope device array, so the call allocates nothing. Checked through the
C ABI against llamd_hip_lmhead_forward (the entry point with allocated
scratch) on consecutive calls -- the second smaller than the first, so it
runs on what the first left in the array -- bit for bit (logits and ids),
and the size limits are refused with an error."""
import ctypes as C

import numpy as np
import pytest

from llamd_rs_amd._lib import lib

pytestmark = pytest.mark.gpu
QK_K = 256


def _noalloc(gpu, dw, xbuf, nseq, logits, ids):
    return lib().llamd_hip_lmhead_forward_noalloc(dw.ptr, dw.rows(), dw.blocks(), xbuf.ptr, nseq,
                                                  logits.ptr, ids.ptr)


def _both(gpu, dw, head, x):
    nseq = x.shape[0]
    rows = dw.rows()
    want_logits, want_ids = head.forward(x)
    xb = gpu.DeviceBuffer.from_array(x)
    lb = gpu.DeviceBuffer(nseq * rows * 4)
    ib = gpu.DeviceBuffer(nseq * 4)
    try:
        rc = _noalloc(gpu, dw, xb, nseq, lb, ib)
        assert rc == 0, lib().llamd_hip_last_error()
        got_logits = lb.download(np.empty((nseq, rows), np.float32))
        got_ids = ib.download(np.empty(nseq, np.int32))
    finally:
        for b in (xb, lb, ib):
            b.close()
    assert np.array_equal(got_logits.view(np.uint32), want_logits.view(np.uint32))
    assert np.array_equal(got_ids, want_ids)
    return got_ids


def test_noalloc_lm_head_matches_the_allocating_entry_point(gpu):
    from llamd_rs_amd import synth
    big_rows, small_rows, k = 151936, 4096, 2048
    wb = synth.q6k_matrix(4243, 0.02, big_rows, k)
    ws = synth.q6k_matrix(4244, 0.02, small_rows, 1024)
    big = gpu.DeviceWeights.upload(wb, big_rows, k // QK_K)
    small = gpu.DeviceWeights.upload(ws, small_rows, 1024 // QK_K)
    hb, hs = gpu.LmHead(big, max_seq=16), gpu.LmHead(small, max_seq=16)
    try:
        # a full configs[4] call at b = 16, then smaller ones on what it left behind
        _both(gpu, big, hb, synth.normal(50, 1.0, 16 * k).reshape(16, k))
        _both(gpu, small, hs, synth.normal(51, 1.0, 3 * 1024).reshape(3, 1024))
        _both(gpu, small, hs, synth.normal(52, 1.0, 1024).reshape(1, 1024))
        _both(gpu, big, hb, synth.normal(53, 1.0, k).reshape(1, k))
        # repeated calls take no device memory
        free0 = lib().llamd_rocm_free_mem()
        for s in range(3):
            _both(gpu, small, hs, synth.normal(60 + s, 1.0, 2 * 1024).reshape(2, 1024))
        assert lib().llamd_rocm_free_mem() == free0
    finally:
        for o in (hb, hs, big, small):
            o.close()


def test_noalloc_lm_head_refuses_what_does_not_fit(gpu):
    from llamd_rs_amd import synth
    L = lib()
    assert 0 < L.llamd_rocm_free_mem()
    assert L.llamd_hip_lmhead_noalloc_scratch_bytes() < 4 << 20
    rows, k = 16, 33 * QK_K                    # k beyond the 8192 limit
    w = gpu.DeviceWeights.upload(synth.q6k_matrix(5, 0.02, rows, k), rows, k // QK_K)
    ok = gpu.DeviceWeights.upload(synth.q6k_matrix(6, 0.02, rows, 256), rows, 1)
    x = gpu.DeviceBuffer(17 * k * 4)
    y = gpu.DeviceBuffer(17 * rows * 4)
    i = gpu.DeviceBuffer(17 * 4)
    try:
        assert L.llamd_hip_lmhead_forward_noalloc(w.ptr, rows, k // QK_K, x.ptr, 1, y.ptr, i.ptr) == -1
        assert b"at most" in L.llamd_hip_last_error()
        assert L.llamd_hip_lmhead_forward_noalloc(ok.ptr, rows, 1, x.ptr, 17, y.ptr, i.ptr) == -1
        assert b"at most" in L.llamd_hip_last_error()
        assert L.llamd_hip_lmhead_forward_noalloc(ok.ptr, rows + 1, 1, x.ptr, 1, y.ptr, i.ptr) == -1
        assert L.llamd_hip_lmhead_forward_noalloc(None, rows, 1, x.ptr, 1, y.ptr, i.ptr) == -1
    finally:
        for o in (w, ok, x, y, i):
            o.close()
