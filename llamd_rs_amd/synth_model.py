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


def write_model(path, hp=QWEN3_30B_A3B, seed=0, expert_sets: int = 1,
                distinct_layers: bool = False) -> dict:
    """Write the model and return its tensors {name: array} (arrays may be
    shared between layers). With distinct_layers, every layer gets its own
    norms, router and attention matrices; the expert tensors cycle through
    `expert_sets` distinct copies (layer L uses set L % expert_sets)."""
    E, hd, nh, nkv = hp["n_embd"], hp["hd"], hp["n_head"], hp["n_head_kv"]
    ne, nff, V = hp["n_expert"], hp["n_ff"], hp["n_vocab"]
    s = seed * 100
    norm = lambda k, n: (1 + 0.1 * synth.normal(k, 1.0, n)).astype(np.float32)
    experts = [{
        "ffn_gate_exps.weight": ([E, nff, ne], synth.q6k_matrix(s + 10 + 1000 * i, 0.05, ne * nff, E)),
        "ffn_up_exps.weight": ([E, nff, ne], synth.q6k_matrix(s + 11 + 1000 * i, 0.05, ne * nff, E)),
        "ffn_down_exps.weight": ([nff, E, ne], synth.q6k_matrix(s + 12 + 1000 * i, 0.05, ne * E, nff)),
    } for i in range(expert_sets)]

    def small(k):  # the per-layer tensors other than the experts
        return {
            "attn_norm.weight": ([E], norm(k + 1, E)),
            "ffn_norm.weight": ([E], norm(k + 2, E)),
            "attn_q_norm.weight": ([hd], norm(k + 3, hd)),
            "attn_k_norm.weight": ([hd], norm(k + 4, hd)),
            "attn_q.weight": ([E, nh * hd], synth.q6k_matrix(k + 5, 0.05, nh * hd, E)),
            "attn_k.weight": ([E, nkv * hd], synth.q6k_matrix(k + 6, 0.05, nkv * hd, E)),
            "attn_v.weight": ([E, nkv * hd], synth.q6k_matrix(k + 7, 0.05, nkv * hd, E)),
            "attn_output.weight": ([nh * hd, E], synth.q6k_matrix(k + 8, 0.05, E, nh * hd)),
            "ffn_gate_inp.weight": ([E, ne], synth.normal(k + 9, 0.05, ne * E).reshape(ne, E)),
        }

    shared = small(s)
    w = {"token_embd.weight": ([E, V], synth.q6k_matrix(s + 13, 0.5, V, E)),
         "output.weight": ([E, V], synth.q6k_matrix(s + 14, 0.05, V, E)),
         "output_norm.weight": ([E], norm(s + 15, E))}
    for il in range(hp["n_layer"]):
        lay = small(s + 50 + 20 * il) if distinct_layers else shared
        lay = dict(lay, **experts[il % expert_sets])
        w.update({f"blk.{il}.{n}": v for n, v in lay.items()})
    tensors = [(n, d, 0 if a.dtype == np.float32 else 14, a) for n, (d, a) in w.items()]
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
    return {n: a for n, (d, a) in w.items()}
