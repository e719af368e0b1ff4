"""Named device workloads of the path, for profilers:

    python -m llamd_rs_amd.workloads NAME [--iters N] [--tune KEY=VALUE ...]

runs NAME's launches N times on synthetic seeded inputs (the shapes of
BASELINE.json's configs, weights rotating where one copy would sit in the
Infinity Cache) and prints one line when done. Meant to be run under
rocprofv3 (--kernel-trace, --pmc) so a profile covers exactly one workload:

    configs1     Q6_K gate/up/down matvecs at batch 1 (768x2048, 2048x768)
    configs1_grouped  the same shapes 128 matrices per launch (all experts
                 of one expert tensor, one grouped launch each), 3 tensors
                 rotating
    lm_head_b1   the LM head call (151936x2048), batch 1 and 16
    lm_head_b16
    lm_head_b16_reduction  the b=16 call with LLAMD_HIP_REDUCTION (tolerance
                 logits, certified exact arg-max)
    moe_decode   one MoE decode layer per call, 4 layers rotating
    prefill      the expert-grouped FFN of 512 tokens, top-8 of 128, Zipf 1.1
    prefill_reduction  the same with LLAMD_HIP_REDUCTION (tolerance GEMMs)
    decode       whole-token decode of a Qwen3-30B-A3B-shaped model cut to 4
                 layers (plain launches, no graph), positions 3..3+N
    ffi_decode   the same model through the reference's own DeviceModel call
                 sequence on the exported FFI (ffi_replay.py), plain launches
    ffi_decode_batch16  its forward_batch at 16 sequences
"""
from __future__ import annotations

import argparse
import sys
import time

import numpy as np

from . import rocm, synth
from ._lib import lib

QK_K = 256


def _sync(L):
    if L.llamd_fwd_sync() or L.llamd_fwd_last_error():
        raise RuntimeError("device error")


def configs1(L, iters):
    shapes = [(768, 2048, 11), (768, 2048, 12), (2048, 768, 13)]
    mats = [synth.q6k_matrix(s, 0.02, r, k) for r, k, s in shapes]
    n = 280  # 280 x 3.9 MB copies rotate (1.1 GB, beyond the 256 MB Infinity Cache)
    ws = [[rocm.DeviceWeights.upload(m, r, k // QK_K) for _ in range(n)] for m, (r, k, _) in zip(mats, shapes)]
    acts = {k: rocm.quantize_q8k_on_device(synth.normal(21 + k, 1.0, k)) for _, k, _ in shapes}
    dq = {k: (rocm.DeviceBuffer.from_array(a.qs), rocm.DeviceBuffer.from_array(a.d)) for k, a in acts.items()}
    outs = [rocm.DeviceBuffer(r * 4) for r, _, _ in shapes]
    for i in range(iters):
        for j, (r, k, _) in enumerate(shapes):
            q, d = dq[k]
            L.llamd_fwd_matvec(ws[j][i % n].ptr, q.ptr, d.ptr, outs[j].ptr, k // QK_K, r)
    _sync(L)


def configs1_grouped(L, iters):
    n_expert = 128
    shapes = [(768, 2048, 501), (2048, 768, 503)]
    ids = rocm.DeviceBuffer.from_array(np.arange(n_expert, dtype=np.int32))
    for rows, k, seed in shapes:
        host = synth.q6k_matrix(seed, 0.02, n_expert * rows, k)
        cps = [rocm.DeviceWeights.upload_experts(host, n_expert, rows, k // QK_K) for _ in range(3)]
        a = rocm.quantize_q8k_on_device(synth.normal(23 + k, 1.0, k))
        q, d = rocm.DeviceBuffer.from_array(a.qs), rocm.DeviceBuffer.from_array(a.d)
        y = rocm.DeviceBuffer(n_expert * rows * 4)
        for i in range(iters):
            L.llamd_fwd_matvec_grouped(cps[i % 3].ptr, ids.ptr, q.ptr, d.ptr, y.ptr, k // QK_K, rows,
                                       n_expert)
        _sync(L)
        for c in cps:
            c.close()


def lm_head(L, iters, nseq, flags=0):
    rows, k = 151936, 2048
    w = synth.q6k_matrix(4242, 0.02, rows, k)
    heads = []
    for _ in range(2):
        dw = rocm.DeviceWeights.upload(w, rows, k // QK_K)
        heads.append((dw, rocm.LmHead(dw, max_seq=16)))
    xb = rocm.DeviceBuffer.from_array(synth.normal(31, 1.0, 16 * k))
    lg, ids = rocm.DeviceBuffer(16 * rows * 4), rocm.DeviceBuffer(64)
    for i in range(iters):
        if L.llamd_hip_lmhead_forward_ex(heads[i % 2][1].handle, xb.ptr, nseq, lg.ptr, ids.ptr, flags):
            raise RuntimeError("lmhead")
    _sync(L)


def _moe_layers(n):
    n_embd, n_ff, n_expert, n_used = 2048, 768, 128, 8
    router = synth.normal(500, 0.02, n_expert * n_embd).reshape(n_expert, n_embd)
    gate = synth.q6k_matrix(501, 0.02, n_expert * n_ff, n_embd)
    up = synth.q6k_matrix(502, 0.02, n_expert * n_ff, n_embd)
    down = synth.q6k_matrix(503, 0.02, n_expert * n_embd, n_ff)
    return [rocm.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used) for _ in range(n)]


def moe_decode(L, iters):
    layers = _moe_layers(4)
    X = rocm.DeviceBuffer.from_array(synth.normal(600, 1.0, 64 * 2048))
    O = rocm.DeviceBuffer(2048 * 4)
    for i in range(iters):
        if L.llamd_hip_moe_forward(layers[i % 4].handle, X.ptr + (i % 64) * 2048 * 4, 0, O.ptr, 0):
            raise RuntimeError("moe")
    _sync(L)


def prefill(L, iters, flags=0):
    layers = _moe_layers(2)
    n_tok = 512
    xs = rocm.DeviceBuffer.from_array(synth.normal(700, 1.0, n_tok * 2048))
    ids, w = synth.zipf_routing(701, 1.1, n_tok, 128, 8)
    di, dw = rocm.DeviceBuffer.from_array(ids.astype(np.int32)), rocm.DeviceBuffer.from_array(w)
    out = rocm.DeviceBuffer(n_tok * 2048 * 4)
    for i in range(iters):
        if L.llamd_hip_moe_prefill_ex(layers[i % 2].handle, xs.ptr, di.ptr, dw.ptr, out.ptr, n_tok, flags):
            raise RuntimeError("prefill")
    _sync(L)


def decode(L, iters):
    import os
    import tempfile
    from . import synth_model
    from .gguf import Gguf
    hp = dict(synth_model.QWEN3_30B_A3B, n_layer=4)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    if L.llamd_hip_tune(b"model_graph", 0) < 0:  # read when the model is created
        raise RuntimeError("tune")
    try:
        synth_model.write_model(path, hp)
        with Gguf(path) as g:
            dm = rocm.DeviceModel(g, max_kv=1024)
    finally:
        os.unlink(path)
    tok = 1
    for pos in range(3 + iters):
        _, tok = dm.forward(tok, pos)
    dm.close()


def decode_long(L, iters):
    """The decode step near position 1000 (the split attention of long
    contexts): the 4-layer cut of the Qwen3-30B-A3B shapes, its cache filled
    in order to position 999, then `iters` tokens; plain launches."""
    import os
    import tempfile
    from . import synth_model
    from .gguf import Gguf
    hp = dict(synth_model.QWEN3_30B_A3B, n_layer=4)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    if L.llamd_hip_tune(b"model_graph", 0) < 0:  # read when the model is created
        raise RuntimeError("tune")
    try:
        synth_model.write_model(path, hp)
        with Gguf(path) as g:
            dm = rocm.DeviceModel(g, max_kv=1024)
    finally:
        os.unlink(path)
    tok = 1
    for pos in range(1000 + iters):
        _, tok = dm.forward(tok, pos)
    dm.close()


def ffi_decode(L, iters, nseq=1):
    """The reference's DeviceModel call sequence on the exported FFI
    (ffi_replay.py), the 4-layer cut of the Qwen3-30B-A3B shapes; plain
    launches (no graph) so a kernel trace sees every launch."""
    import os
    import tempfile
    from . import synth_model
    from .ffi_replay import FfiModel
    from .gguf import Gguf
    hp = dict(synth_model.QWEN3_30B_A3B, n_layer=4)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    try:
        synth_model.write_model(path, hp)
        with Gguf(path) as g:
            fm = FfiModel(g, max_kv=1024, max_seq=max(nseq, 1), use_graph=False)
    finally:
        os.unlink(path)
    if nseq == 1:
        tok = 1
        for pos in range(3 + iters):
            tok = fm.forward(tok, pos)
    else:
        toks = list(range(1, nseq + 1))
        for pos in range(iters):
            toks = fm.forward_batch(toks, [pos] * nseq)
    fm.close()


WORKLOADS = {
    "configs1": configs1,
    "configs1_grouped": configs1_grouped,
    "lm_head_b1": lambda L, n: lm_head(L, n, 1),
    "lm_head_b16": lambda L, n: lm_head(L, n, 16),
    "lm_head_b16_reduction": lambda L, n: lm_head(L, n, 16, 1),
    "moe_decode": moe_decode,
    "prefill": prefill,
    "prefill_reduction": lambda L, n: prefill(L, n, 1),
    "decode": decode,
    "decode_long": decode_long,
    "ffi_decode": ffi_decode,
    "ffi_decode_batch16": lambda L, n: ffi_decode(L, n, 16),
}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("name", choices=sorted(WORKLOADS))
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--tune", action="append", default=[], metavar="KEY=VALUE",
                    help="llamd_hip_tune overrides applied before the workload")
    args = ap.parse_args(argv)
    L = lib()
    if not rocm.available():
        raise SystemExit("no ROCm device visible")
    for kv in args.tune:
        key, _, val = kv.partition("=")
        if L.llamd_hip_tune(key.encode(), int(val)) < 0:
            raise SystemExit(f"unknown tune key {key}")
    t0 = time.time()
    WORKLOADS[args.name](L, args.iters)
    print(f"{args.name}: {args.iters} iterations in {time.time() - t0:.2f}s", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
