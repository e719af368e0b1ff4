"""Weights that arrive in a GGUF file: Q6_K tensors uploaded straight from the
mapping (crates/llamd-runtime/src/device.rs:224-256) and a whole MoE layer
built from blk.0's tensors give the CPU path's bits."""
import numpy as np
import pytest

from llamd_rs_amd import gguf_writer as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu
QK_K = 256


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q6k_tensors_from_a_gguf_file(gpu, tmp_path):
    from llamd_rs_amd import synth
    from llamd_rs_amd.gguf import Gguf
    rows, k, ne = 48, 512, 3
    w2 = synth.q6k_matrix(11, 0.02, rows, k)
    w3 = synth.q6k_matrix(12, 0.02, ne * rows, k)
    p = tmp_path / "w.gguf"
    W.write(p, [("general.alignment", W.U32, 64)],
            [("output.weight", [k, rows], 14, w2.tobytes()),
             ("blk.0.ffn_up_exps.weight", [k, rows, ne], 14, w3.tobytes())], alignment=64)
    with Gguf(p) as g:
        assert bytes(g.tensor_data(g.tensor("output.weight"))) == w2.tobytes()
        x = synth.normal(13, 1.0, k)
        act = gpu.quantize_q8k_on_device(x)
        dw = g.upload_q6k("output.weight")
        assert bits_equal(dw.matvec(act), O.matvec_q6k(w2, rows, k, x))
        de = g.upload_q6k("blk.0.ffn_up_exps.weight")
        ids = np.array([2, 0], np.int32)
        got = de.matvec_grouped(act, ids, rows).reshape(len(ids), rows)
        per = rows * k // QK_K * 210
        for j, e in enumerate(ids):
            assert bits_equal(got[j], O.matvec_q6k(w3[e * per:(e + 1) * per], rows, k, x)), e
        dw.close()
        de.close()


def test_moe_layer_from_a_gguf_file(gpu, tmp_path):
    """blk.0 of a Qwen3-MoE-shaped file (router F32 [n_embd, n_expert], Q6_K
    experts [n_embd, n_ff, n_expert] / [n_ff, n_embd, n_expert]) through
    llamd_gguf_moe_create: logits, ids, weights and output bit-identical."""
    from llamd_rs_amd import synth
    from llamd_rs_amd.gguf import Gguf
    n_embd, n_ff, n_expert, n_used = 512, 256, 16, 4
    router = synth.normal(21, 0.02, n_expert * n_embd).reshape(n_expert, n_embd)
    gate = synth.q6k_matrix(22, 0.02, n_expert * n_ff, n_embd)
    up = synth.q6k_matrix(23, 0.02, n_expert * n_ff, n_embd)
    down = synth.q6k_matrix(24, 0.02, n_expert * n_embd, n_ff)
    p = tmp_path / "moe.gguf"
    W.write(p, [("general.architecture", W.STRING, "qwen3moe"),
                ("qwen3moe.expert_used_count", W.U32, n_used),
                ("qwen3moe.expert_count", W.U32, n_expert)],
            [("blk.0.ffn_gate_inp.weight", [n_embd, n_expert], 0, router.astype(np.float32).tobytes()),
             ("blk.0.ffn_gate_exps.weight", [n_embd, n_ff, n_expert], 14, gate.tobytes()),
             ("blk.0.ffn_up_exps.weight", [n_embd, n_ff, n_expert], 14, up.tobytes()),
             ("blk.0.ffn_down_exps.weight", [n_ff, n_embd, n_expert], 14, down.tobytes())])
    with Gguf(p) as g:
        layer = g.moe_layer(0)
        # the router as the file holds it: [n_expert][n_embd] f32
        r_file = np.frombuffer(bytes(g.tensor_data(g.tensor("blk.0.ffn_gate_inp.weight"))),
                               np.float32).reshape(n_expert, n_embd)
        assert np.array_equal(r_file, router)
        try:
            for t in range(3):
                x = synth.normal(30 + t, 1.0, n_embd)
                res = synth.normal(40 + t, 1.0, n_embd)
                want, lg, ids, w = O.moe_layer(x, res, n_embd, n_ff, n_expert, n_used, router, gate,
                                               up, down)
                out, r, lgd = layer.forward(x, res)
                assert bits_equal(lgd, lg) and list(r.experts) == list(ids), t
                assert bits_equal(r.weights, w) and bits_equal(out, want), t
        finally:
            layer.close()
