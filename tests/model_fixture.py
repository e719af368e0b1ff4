"""A small Qwen3-MoE written as GGUF (tests/gguf_writer.py) and the
reference's CPU forward for it composed from the oracle's functions
(crates/llamd-runtime/src/layer.rs: forward_layer, moe_ffn, forward).
Test infrastructure only."""
from __future__ import annotations

import numpy as np

from llamd_rs_amd import gguf_writer as W
from oracle import oracle as O

HP = dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, hd=128, n_expert=8, n_used=2, n_ff=256,
          n_vocab=768, eps=1e-6, base=1_000_000.0)


def make(path, seed=0, hp=HP):
    from llamd_rs_amd import synth
    E, hd, nh, nkv = hp["n_embd"], hp["hd"], hp["n_head"], hp["n_head_kv"]
    ne, nff, V = hp["n_expert"], hp["n_ff"], hp["n_vocab"]
    s = iter(range(seed * 1000, seed * 1000 + 1000))
    w = {"token_embd.weight": synth.q6k_matrix(next(s), 0.5, V, E),
         "output.weight": synth.q6k_matrix(next(s), 0.05, V, E),
         "output_norm.weight": (1 + 0.1 * synth.normal(next(s), 1.0, E)).astype(np.float32)}
    for il in range(hp["n_layer"]):
        b = f"blk.{il}."
        w[b + "attn_norm.weight"] = (1 + 0.1 * synth.normal(next(s), 1.0, E)).astype(np.float32)
        w[b + "ffn_norm.weight"] = (1 + 0.1 * synth.normal(next(s), 1.0, E)).astype(np.float32)
        w[b + "attn_q_norm.weight"] = (1 + 0.1 * synth.normal(next(s), 1.0, hd)).astype(np.float32)
        w[b + "attn_k_norm.weight"] = (1 + 0.1 * synth.normal(next(s), 1.0, hd)).astype(np.float32)
        w[b + "attn_q.weight"] = synth.q6k_matrix(next(s), 0.05, nh * hd, E)
        w[b + "attn_k.weight"] = synth.q6k_matrix(next(s), 0.05, nkv * hd, E)
        w[b + "attn_v.weight"] = synth.q6k_matrix(next(s), 0.05, nkv * hd, E)
        w[b + "attn_output.weight"] = synth.q6k_matrix(next(s), 0.05, E, nh * hd)
        w[b + "ffn_gate_inp.weight"] = synth.normal(next(s), 0.05, ne * E).reshape(ne, E)
        w[b + "ffn_gate_exps.weight"] = synth.q6k_matrix(next(s), 0.05, ne * nff, E)
        w[b + "ffn_up_exps.weight"] = synth.q6k_matrix(next(s), 0.05, ne * nff, E)
        w[b + "ffn_down_exps.weight"] = synth.q6k_matrix(next(s), 0.05, ne * E, nff)
    dims = {"token_embd.weight": [E, V], "output.weight": [E, V], "output_norm.weight": [E]}
    for il in range(hp["n_layer"]):
        b = f"blk.{il}."
        dims.update({b + "attn_norm.weight": [E], b + "ffn_norm.weight": [E],
                     b + "attn_q_norm.weight": [hd], b + "attn_k_norm.weight": [hd],
                     b + "attn_q.weight": [E, nh * hd], b + "attn_k.weight": [E, nkv * hd],
                     b + "attn_v.weight": [E, nkv * hd], b + "attn_output.weight": [nh * hd, E],
                     b + "ffn_gate_inp.weight": [E, ne], b + "ffn_gate_exps.weight": [E, nff, ne],
                     b + "ffn_up_exps.weight": [E, nff, ne], b + "ffn_down_exps.weight": [nff, E, ne]})
    tensors = [(n, dims[n], 0 if a.dtype == np.float32 else 14, a.tobytes()) for n, a in w.items()]
    p = "qwen3moe"
    kvs = [("general.architecture", W.STRING, p), (p + ".block_count", W.U32, hp["n_layer"]),
           (p + ".embedding_length", W.U32, E), (p + ".attention.head_count", W.U32, nh),
           (p + ".attention.head_count_kv", W.U32, nkv), (p + ".attention.key_length", W.U32, hd),
           (p + ".attention.layer_norm_rms_epsilon", W.F32, hp["eps"]),
           (p + ".rope.freq_base", W.F32, hp["base"]), (p + ".expert_count", W.U32, ne),
           (p + ".expert_used_count", W.U32, hp["n_used"]),
           (p + ".expert_feed_forward_length", W.U32, nff),
           (p + ".feed_forward_length", W.U32, nff), (p + ".context_length", W.U32, 4096)]
    W.write(path, kvs, tensors)
    return w


class OracleModel:
    """The reference CPU forward, one token at a time (layer.rs:268-304)."""

    def __init__(self, w, hp=HP, max_kv=64):
        self.w, self.hp = w, hp
        kv_dim = hp["n_head_kv"] * hp["hd"]
        self.K = np.zeros((hp["n_layer"], max_kv, kv_dim), np.float32)
        self.V = np.zeros_like(self.K)
        self.row_bytes = hp["n_embd"] // 256 * 210   # one Q6_K embedding row

    def embed(self, token):
        rb = self.row_bytes
        row = np.asarray(self.w["token_embd.weight"]).reshape(-1)[token * rb:(token + 1) * rb]
        return O.dequantize(14, row, self.hp["n_embd"])

    def lm_head(self, xn):
        """matvec_quant over the vocabulary, rows split over a thread pool
        (rows are independent: the same bits as one call)."""
        import helpers as H
        V, E = self.hp["n_vocab"], self.hp["n_embd"]
        wo = np.asarray(self.w["output.weight"]).reshape(V, -1)
        cuts = np.linspace(0, V, 17).astype(int) if V >= 4096 else np.array([0, V])
        parts = H.par_map(lambda i: O.matvec_q6k(wo[cuts[i]:cuts[i + 1]].reshape(-1),
                                                 int(cuts[i + 1] - cuts[i]), E, xn),
                          range(len(cuts) - 1))
        return np.concatenate(parts)

    def forward(self, token, pos):
        hp, w = self.hp, self.w
        E, hd, nh, nkv, eps = hp["n_embd"], hp["hd"], hp["n_head"], hp["n_head_kv"], hp["eps"]
        f32 = np.float32
        x = self.embed(token)
        for il in range(hp["n_layer"]):
            b = f"blk.{il}."
            attn_norm = O.rms_norm(x, 1, E, eps) * w[b + "attn_norm.weight"]
            q = O.matvec_q6k(w[b + "attn_q.weight"], nh * hd, E, attn_norm)
            k = O.matvec_q6k(w[b + "attn_k.weight"], nkv * hd, E, attn_norm)
            v = O.matvec_q6k(w[b + "attn_v.weight"], nkv * hd, E, attn_norm)
            q = O.rms_norm(q, nh, hd, eps) * np.tile(w[b + "attn_q_norm.weight"], nh)
            k = O.rms_norm(k, nkv, hd, eps) * np.tile(w[b + "attn_k_norm.weight"], nkv)
            q = O.rope(q, nh, hd, pos, hp["base"])
            k = O.rope(k, nkv, hd, pos, hp["base"])
            self.K[il, pos], self.V[il, pos] = k, v
            attn = O.attend(q, self.K[il, :pos + 1], self.V[il, :pos + 1], pos + 1, nh, nkv, hd)
            o = O.matvec_q6k(w[b + "attn_output.weight"], E, nh * hd, attn)
            ffn_inp = (x + o).astype(f32)
            fn = O.rms_norm(ffn_inp, 1, E, eps) * w[b + "ffn_norm.weight"]
            x, _, _, _ = O.moe_layer(fn, ffn_inp, E, hp["n_ff"], hp["n_expert"], hp["n_used"],
                                     w[b + "ffn_gate_inp.weight"], w[b + "ffn_gate_exps.weight"],
                                     w[b + "ffn_up_exps.weight"], w[b + "ffn_down_exps.weight"])
        xn = O.rms_norm(x, 1, E, eps) * w["output_norm.weight"]
        logits = self.lm_head(xn)
        return logits, O.argmax(logits)
