"""The reference's own device model, unchanged, over this library: the launch
sequences of DeviceModel::forward (with and without its graph capture) and
DeviceModel::forward_batch (crates/llamd-runtime/src/device.rs:486-962),
issued through the exported llamd_fwd_* / llamd_b_* / llamd_u_* symbols only
(llamd_rs_amd/ffi_replay.py), compared token by token with the CPU forward
composed from the oracle: every logit's bits and every next token."""
import numpy as np
import pytest

import model_fixture as MF

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("use_graph", [True, False])
def test_ffi_forward_matches_the_cpu(gpu, tmp_path, use_graph):
    """forward(): embed .. argmax through llamd_fwd_*, one synchronisation per
    token; with use_graph the first token is captured (the planar weights'
    tiled copies are made inside the capture) and every token replays it."""
    from llamd_rs_amd.ffi_replay import FfiModel
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    w = MF.make(p, seed=6)
    ref = MF.OracleModel(w, max_kv=16)
    with Gguf(p) as g:
        fm = FfiModel(g, max_kv=16, use_graph=use_graph)
    try:
        tok = 11
        for pos in range(5):
            nxt = fm.forward(tok, pos)
            want, want_next = ref.forward(tok, pos)
            assert bits_equal(fm.logits()[0], want), pos
            assert nxt == want_next, pos
            tok = nxt
    finally:
        fm.close()


def test_ffi_forward_batch_matches_the_cpu(gpu, tmp_path):
    """forward_batch(): three independent sequences (the third joins a step
    later, so positions differ), each against its own CPU forward."""
    from llamd_rs_amd.ffi_replay import FfiModel
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    w = MF.make(p, seed=8)
    refs = [MF.OracleModel(w, max_kv=16) for _ in range(3)]
    with Gguf(p) as g:
        fm = FfiModel(g, max_kv=16, max_seq=3, use_graph=False)
    try:
        toks, pos = [3, 500], [0, 0]
        for step in range(4):
            got = fm.forward_batch(toks, pos)
            lg = fm.logits(len(toks))
            for s in range(len(toks)):
                want, want_next = refs[s].forward(toks[s], pos[s])
                assert bits_equal(lg[s], want), (step, s)
                assert got[s] == want_next, (step, s)
            toks = got + ([77] if len(got) == 2 else [])
            pos = [q + 1 for q in pos] + ([0] if len(pos) == 2 else [])
    finally:
        fm.close()


def test_ffi_forward_full_qwen3_30b_a3b_widths(gpu, tmp_path):
    """The unchanged caller at Qwen3-30B-A3B's real widths (hidden 2048, 32/4
    heads of 128, 128 experts top-8 of 768, vocabulary 151936), 4 layers, graph
    capture on: 3 tokens, every logit's bits and the argmax against the CPU."""
    from llamd_rs_amd import synth_model
    from llamd_rs_amd.ffi_replay import FfiModel
    from llamd_rs_amd.gguf import Gguf
    hp = dict(synth_model.QWEN3_30B_A3B, n_layer=4)
    p = tmp_path / "qwen3-30b-a3b-4l.gguf"
    w = synth_model.write_model(p, hp, seed=9, expert_sets=2, distinct_layers=True)
    with Gguf(p) as g:
        fm = FfiModel(g, max_kv=16, use_graph=True)
    p.unlink()
    ref = MF.OracleModel(w, hp=hp, max_kv=16)
    try:
        tok = 4321
        for pos in range(3):
            nxt = fm.forward(tok, pos)
            want, want_next = ref.forward(tok, pos)
            assert bits_equal(fm.logits()[0], want), pos
            assert nxt == want_next, pos
            tok = nxt
    finally:
        fm.close()
