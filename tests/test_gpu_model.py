"""The resident whole-token decode loop (llamd_hip_model_*) on a small
Qwen3-MoE written as GGUF: every token's logits and argmax bit-identical to
the reference CPU forward (crates/llamd-runtime/src/layer.rs:268-304)
composed from the oracle."""
import numpy as np
import pytest

import model_fixture as MF

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


HP_MHA = dict(MF.HP, n_head=4, n_head_kv=4)             # kv groups of one query head
HP_MHA64 = dict(MF.HP, n_head=8, n_head_kv=8, hd=64)   # hd 64: the three-launch path either way


@pytest.mark.parametrize("hp,fused,fnorm,nqkv,n_tok", [
    (MF.HP, 1, 1, 1, 10), (MF.HP, 1, 1, 0, 10), (MF.HP, 0, 0, 1, 10), (MF.HP, 1, 0, 1, 10),
    (MF.HP, 0, 1, 0, 10), (MF.HP, 1, 1, 1, 40), (HP_MHA, 1, 1, 1, 12), (HP_MHA64, 1, 1, 1, 12),
    (HP_MHA64, 0, 0, 0, 12)])
def test_decode_loop_is_bit_identical_to_the_cpu_forward(gpu, tmp_path, hp, fused, fnorm, nqkv,
                                                         n_tok):
    """Every fusion of the step on and off: the attention RMSNorm and its
    Q8_K inside the Q/K/V launch or before it, attend_fused (QK-norm, RoPE,
    KV append, attention and Q8_K in one launch) or the three launches, and
    the FFN norm inside the MoE decode launch or before it."""
    from llamd_rs_amd._lib import lib
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    w = MF.make(p, seed=3, hp=hp)
    L = lib()
    prev = (L.llamd_hip_tune(b"model_fused_attn", fused),   # read when the model is created
            L.llamd_hip_tune(b"model_fused_norm", fnorm),
            L.llamd_hip_tune(b"model_norm_qkv", nqkv))
    try:
        with Gguf(p) as g:
            dm = gpu.DeviceModel(g, max_kv=48)
    finally:
        L.llamd_hip_tune(b"model_fused_attn", prev[0])
        L.llamd_hip_tune(b"model_fused_norm", prev[1])
        L.llamd_hip_tune(b"model_norm_qkv", prev[2])
    ref = MF.OracleModel(w, hp=hp)
    try:
        assert (dm.n_layer, dm.n_embd, dm.n_vocab) == (2, 512, 768)
        tok = 5
        for pos in range(n_tok):
            logits, nxt = dm.forward(tok, pos)
            want, want_next = ref.forward(tok, pos)
            assert bits_equal(logits, want), pos
            assert nxt == want_next, pos
            tok = nxt if pos % 3 else (tok * 37 + 11) % 768   # greedy, with some forced tokens
    finally:
        dm.close()


@pytest.mark.parametrize("hp,max_kv,long_from,n_tok", [
    (MF.HP, 160, -1, 140), (HP_MHA, 160, -1, 140),   # attend_fused throughout
    (MF.HP, 160, 70, 140), (HP_MHA, 160, 70, 140),   # attend_fused, then the split attention
    (MF.HP, 16384, 0, 140), (HP_MHA, 16384, 0, 140),  # split attention throughout
    (MF.HP, 16384, 300, 400)])   # past the split attention's 320-position V chunks
def test_decode_loop_long_context(gpu, tmp_path, hp, max_kv, long_from, n_tok):
    """attend_fused stages cached K and V in LDS 64 positions at a time
    (chunk boundaries at 64 and 128), and the split attention of long
    contexts (logits over the whole GPU, then the softmax and the weighted V
    sum from V chunks in LDS, 320 positions each at max_kv 16384) takes over
    at long_from, with one and two query heads per kv head. Every token's logits bits and
    argmax against the CPU forward, across the switch."""
    from llamd_rs_amd._lib import lib
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    w = MF.make(p, seed=8, hp=hp)
    prev = lib().llamd_hip_tune(b"model_long_from", long_from)   # read when the model is created
    try:
        with Gguf(p) as g:
            dm = gpu.DeviceModel(g, max_kv=max_kv)
    finally:
        lib().llamd_hip_tune(b"model_long_from", prev)
    ref = MF.OracleModel(w, hp=hp, max_kv=n_tok)
    try:
        tok = 7
        for pos in range(n_tok):
            logits, nxt = dm.forward(tok, pos)
            want, want_next = ref.forward(tok, pos)
            assert bits_equal(logits, want), pos
            assert nxt == want_next, pos
            tok = nxt if pos % 5 else (tok * 31 + 3) % 768
    finally:
        dm.close()


def test_decode_loop_refuses_bad_tokens_and_positions(gpu, tmp_path):
    from llamd_rs_amd._lib import HipError
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    MF.make(p, seed=4)
    with Gguf(p) as g:
        dm = gpu.DeviceModel(g, max_kv=8)
    try:
        with pytest.raises(HipError, match="vocabulary"):
            dm.forward(768, 0)
        with pytest.raises(HipError, match="beyond"):
            dm.forward(1, 8)
        logits, nxt = dm.forward(1, 0)
        assert np.all(np.isfinite(logits)) and 0 <= nxt < 768
    finally:
        dm.close()


def test_decode_logits_arrays_held_across_calls(gpu, tmp_path):
    """forward() hands out logits in page-locked buffers taken from a pool
    and returned when an array is collected: arrays the caller still holds
    are never reused, so every one of several held results keeps its own
    token's bits, and buffers freed in between are reused correctly."""
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    w = MF.make(p, seed=6)
    with Gguf(p) as g:
        dm = gpu.DeviceModel(g, max_kv=16)
    ref = MF.OracleModel(w)
    try:
        held, want = [], []
        tok = 3
        for pos in range(6):
            logits, nxt = dm.forward(tok, pos)
            wl, wn = ref.forward(tok, pos)
            assert nxt == wn, pos
            if pos % 2 == 0:
                held.append(logits)        # kept: its buffer stays out of the pool
                want.append(wl)
            view = logits[5:9]             # a view keeps its base array alive
            del logits
            assert view.shape == (4,)
            tok = nxt
        for i, (a, b) in enumerate(zip(held, want)):
            assert bits_equal(a, b), i
        assert len({a.ctypes.data for a in held}) == len(held)
    finally:
        dm.close()
    assert bits_equal(held[0], want[0])    # still readable after close


def test_decode_full_qwen3_30b_a3b_widths(gpu, tmp_path):
    """The whole-token step at Qwen3-30B-A3B's real widths: hidden 2048, 32
    query / 4 kv heads of 128, 128 experts top-8 of n_ff 768, vocabulary
    151936; 4 layers (each with its own norms, router and attention; two
    distinct expert sets alternate), 4 tokens, the last two through the split
    attention of long contexts (8 query heads per kv head). Every logit's bits
    and the argmax against the CPU forward composed from the oracle."""
    from llamd_rs_amd import synth_model
    from llamd_rs_amd._lib import lib
    from llamd_rs_amd.gguf import Gguf
    hp = dict(synth_model.QWEN3_30B_A3B, n_layer=4)
    p = tmp_path / "qwen3-30b-a3b-4l.gguf"
    w = synth_model.write_model(p, hp, seed=7, expert_sets=2, distinct_layers=True)
    prev = lib().llamd_hip_tune(b"model_long_from", 2)
    try:
        with Gguf(p) as g:
            dm = gpu.DeviceModel(g, max_kv=16)
    finally:
        lib().llamd_hip_tune(b"model_long_from", prev)
    p.unlink()
    ref = MF.OracleModel(w, hp=hp, max_kv=16)
    try:
        assert (dm.n_layer, dm.n_embd, dm.n_vocab) == (4, 2048, 151936)
        tok = 1234
        for pos in range(4):
            logits, nxt = dm.forward(tok, pos)
            want, want_next = ref.forward(tok, pos)
            assert bits_equal(logits, want), pos
            assert nxt == want_next, pos
            tok = nxt
    finally:
        dm.close()


def test_decode_loop_exact_when_router_waits_give_up(gpu, tmp_path):
    """The decode step with the FFN norm fused into the MoE launch, with every
    cross-workgroup wait giving up at once (moe_polls = 0): the waiting waves
    fold the router logits themselves from the normed x, same bits."""
    from llamd_rs_amd._lib import lib
    from llamd_rs_amd.gguf import Gguf
    p = tmp_path / "tiny.gguf"
    w = MF.make(p, seed=5)
    with Gguf(p) as g:
        dm = gpu.DeviceModel(g, max_kv=16)
    ref = MF.OracleModel(w)
    prev = lib().llamd_hip_tune(b"moe_polls", 0)
    try:
        tok = 9
        for pos in range(4):
            logits, nxt = dm.forward(tok, pos)
            want, want_next = ref.forward(tok, pos)
            assert bits_equal(logits, want), pos
            assert nxt == want_next, pos
            tok = nxt
    finally:
        lib().llamd_hip_tune(b"moe_polls", prev)
        dm.close()
