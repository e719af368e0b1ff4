"""A synthetic Qwen3-MoE GGUF at a given shape, for benchmarks: seeded
random weights (Q6_K attention, experts, embeddings and output; F32 norms and
router), every layer sharing ONE copy of its tensors' data in the file (the
device still receives a separate upload per layer), so a 48-layer
Qwen3-30B-A3B-shaped model costs about 1 GB of file."""
from __future__ import annotations

import numpy as np

from . import gguf_writer as W
from . import synth

QWEN3_30B_A3B = dict(n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, hd=128, n_expert=128,
                     n_used=8, n_ff=768, n_vocab=151936, eps=1e-6, base=1_000_000.0)


def write_model(path, hp=QWEN3_30B_A3B, seed=0) -> None:
    E, hd, nh, nkv = hp["n_embd"], hp["hd"], hp["n_head"], hp["n_head_kv"]
    ne, nff, V = hp["n_expert"], hp["n_ff"], hp["n_vocab"]
    s = seed * 100
    norm = lambda k, n: (1 + 0.1 * synth.normal(k, 1.0, n)).astype(np.float32).tobytes()
    layer = {  # one copy, shared by every layer
        "attn_norm.weight": ([E], 0, norm(s + 1, E)),
        "ffn_norm.weight": ([E], 0, norm(s + 2, E)),
        "attn_q_norm.weight": ([hd], 0, norm(s + 3, hd)),
        "attn_k_norm.weight": ([hd], 0, norm(s + 4, hd)),
        "attn_q.weight": ([E, nh * hd], 14, synth.q6k_matrix(s + 5, 0.05, nh * hd, E).tobytes()),
        "attn_k.weight": ([E, nkv * hd], 14, synth.q6k_matrix(s + 6, 0.05, nkv * hd, E).tobytes()),
        "attn_v.weight": ([E, nkv * hd], 14, synth.q6k_matrix(s + 7, 0.05, nkv * hd, E).tobytes()),
        "attn_output.weight": ([nh * hd, E], 14, synth.q6k_matrix(s + 8, 0.05, E, nh * hd).tobytes()),
        "ffn_gate_inp.weight": ([E, ne], 0, synth.normal(s + 9, 0.05, ne * E).tobytes()),
        "ffn_gate_exps.weight": ([E, nff, ne], 14, synth.q6k_matrix(s + 10, 0.05, ne * nff, E).tobytes()),
        "ffn_up_exps.weight": ([E, nff, ne], 14, synth.q6k_matrix(s + 11, 0.05, ne * nff, E).tobytes()),
        "ffn_down_exps.weight": ([nff, E, ne], 14, synth.q6k_matrix(s + 12, 0.05, ne * E, nff).tobytes()),
    }
    tensors = [("token_embd.weight", [E, V], 14, synth.q6k_matrix(s + 13, 0.5, V, E).tobytes()),
               ("output.weight", [E, V], 14, synth.q6k_matrix(s + 14, 0.05, V, E).tobytes()),
               ("output_norm.weight", [E], 0, norm(s + 15, E))]
    for il in range(hp["n_layer"]):
        tensors += [(f"blk.{il}.{n}", d, t, b) for n, (d, t, b) in layer.items()]
    p = "qwen3moe"
    kvs = [("general.architecture", W.STRING, p), (p + ".block_count", W.U32, hp["n_layer"]),
           (p + ".embedding_length", W.U32, E), (p + ".attention.head_count", W.U32, nh),
           (p + ".attention.head_count_kv", W.U32, nkv), (p + ".attention.key_length", W.U32, hd),
           (p + ".attention.layer_norm_rms_epsilon", W.F32, hp["eps"]),
           (p + ".rope.freq_base", W.F32, hp["base"]), (p + ".expert_count", W.U32, ne),
           (p + ".expert_used_count", W.U32, hp["n_used"]),
           (p + ".expert_feed_forward_length", W.U32, nff),
           (p + ".feed_forward_length", W.U32, 6144), (p + ".context_length", W.U32, 40960)]
    W.write(path, kvs, tensors)
