"""The reference runtime's device model, driven through this library's C ABI
exactly as the reference drives its own: the launch sequence of
`DeviceModel::forward` (queue_token, crates/llamd-runtime/src/device.rs:486-649,
with graph capture and replay, :651-722) and of `DeviceModel::forward_batch`
(:741-962), issued through the exported llamd_fwd_* / llamd_b_* / llamd_u_*
symbols only -- no llamd_hip_* entry point, no handle of this library's own.

Weights arrive in the reference's layouts, as its loader leaves them
(device.rs:221-262, 318-399): the token embedding as the file's ggml bytes
(DevBuf::from_bytes), every projection and expert tensor in the planar repack
(PlanarWeights::upload, repack_q6k_planar, crates/llamd-quant/src/dot.rs:
380-423), norms and the router in f32. Scratch and KV cache are sized as
device.rs:401-452 sizes them. So this is the unchanged caller, token for token:
what the Rust crate would submit, and what a test compares with the CPU
forward and a benchmark times.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import HipError, last_error, lib

QK_K = 256
ARGMAX_BLOCKS = 512  # device.rs:202
F = C.c_float


def planar_repack(raw: np.ndarray, rows: int, blocks: int):
    """repack_q6k_planar (dot.rs:400-423): the ql, qh, scales and d planes of
    rows * blocks ggml Q6_K blocks, and PlanarQ6K::layout's plane offsets
    (dot.rs:380-393) as the size_t[4] the planar entry points take."""
    n = rows * blocks
    b = np.asarray(raw, np.uint8)[: n * 210].reshape(n, 210)
    out = np.concatenate([b[:, :128].ravel(), b[:, 128:192].ravel(), b[:, 192:208].ravel(),
                          b[:, 208:210].ravel()])
    off = (C.c_size_t * 4)(0, n * 128, n * 192, n * 208)
    return out, off


class DevBuf:
    """forward.rs:29-220: one llamd_fwd_alloc allocation, freed exactly once."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = lib().llamd_fwd_alloc(self.nbytes)
        if not self.ptr:
            raise HipError(f"llamd_fwd_alloc({self.nbytes}): {last_error()}")

    @classmethod
    def from_bytes(cls, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    @classmethod
    def zeroed(cls, nbytes: int) -> "DevBuf":
        b = cls(nbytes)
        if lib().llamd_fwd_memset(b.ptr, 0, b.nbytes):
            raise HipError(f"llamd_fwd_memset: {last_error()}")
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        if lib().llamd_fwd_upload(self.ptr, a.ctypes.data, a.nbytes):
            raise HipError(f"llamd_fwd_upload: {last_error()}")

    def download(self, out: np.ndarray) -> np.ndarray:
        if lib().llamd_fwd_download(out.ctypes.data, self.ptr, out.nbytes):
            raise HipError(f"llamd_fwd_download: {last_error()}")
        return out

    def free(self):
        if self.ptr:
            lib().llamd_fwd_free(self.ptr)
            self.ptr = None


class Planar:
    """PlanarWeights: the repacked bytes on the device and their offsets."""

    def __init__(self, raw: np.ndarray, rows: int, blocks: int):
        data, self.off = planar_repack(raw, rows, blocks)
        self.buf = DevBuf.from_bytes(data)
        self.rows, self.blocks = rows, blocks


def _check():
    """The reference's sync() (forward.rs:240-262): the stream drained, then
    the sticky launch-refusal flag."""
    if lib().llamd_fwd_sync() or lib().llamd_fwd_last_error():
        raise HipError(f"device: {last_error()}")


class FfiModel:
    """DeviceModel::load_batched (device.rs:262-470) and its two token entry
    points, on the exported C ABI only."""

    def __init__(self, g, max_kv: int, max_seq: int = 1, use_graph: bool = True):
        L = self.L = lib()
        if L.llamd_fwd_stream_init():
            raise HipError(f"stream_init: {last_error()}")
        md = g.metadata
        a = md["general.architecture"]
        hp = self.hp = dict(
            n_layer=md[a + ".block_count"], n_embd=md[a + ".embedding_length"],
            n_head=md[a + ".attention.head_count"], n_head_kv=md[a + ".attention.head_count_kv"],
            hd=md[a + ".attention.key_length"], eps=md[a + ".attention.layer_norm_rms_epsilon"],
            base=md[a + ".rope.freq_base"], n_expert=md[a + ".expert_count"],
            n_used=md[a + ".expert_used_count"], n_ff=md[a + ".expert_feed_forward_length"])
        hp["n_vocab"] = g.tensor("output.weight").dims[1]
        if max_seq < 1 or max_seq > L.llamd_batch_max_seq():
            raise HipError(f"max_seq {max_seq} outside 1..{L.llamd_batch_max_seq()}")
        self.max_kv, self.max_seq, self.use_graph = max_kv, max_seq, use_graph
        self._bufs = []
        E, nh, nkv, hd = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["hd"]
        ne, nu, nff, V = hp["n_expert"], hp["n_used"], hp["n_ff"], hp["n_vocab"]
        kv_dim = nkv * hd

        def raw(name):
            return g.tensor_data(g.tensor(name))

        def planar(name):
            t = g.tensor(name)
            k = t.dims[0]
            p = Planar(raw(name), t.elems() // k, k // QK_K)
            self._bufs.append(p.buf)
            return p

        def f32(name):
            b = DevBuf.from_bytes(np.frombuffer(raw(name), np.float32))
            self._bufs.append(b)
            return b

        self.tok_embd = DevBuf.from_bytes(raw("token_embd.weight"))
        self._bufs.append(self.tok_embd)
        self.embd_blocks = E // QK_K
        self.output_norm = f32("output_norm.weight")
        self.output = planar("output.weight")
        self.layers = []
        for il in range(hp["n_layer"]):
            b = f"blk.{il}."
            self.layers.append(dict(
                attn_norm=f32(b + "attn_norm.weight"), attn_q=planar(b + "attn_q.weight"),
                attn_k=planar(b + "attn_k.weight"), attn_v=planar(b + "attn_v.weight"),
                attn_q_norm=f32(b + "attn_q_norm.weight"), attn_k_norm=f32(b + "attn_k_norm.weight"),
                attn_out=planar(b + "attn_output.weight"), ffn_norm=f32(b + "ffn_norm.weight"),
                ffn_gate_inp=f32(b + "ffn_gate_inp.weight"),
                ffn_gate_exps=planar(b + "ffn_gate_exps.weight"),
                ffn_up_exps=planar(b + "ffn_up_exps.weight"),
                ffn_down_exps=planar(b + "ffn_down_exps.weight")))
        # the scratch of device.rs:416-450, every activation max_seq deep
        ms = max_seq
        max_act = max(E, nh * hd, nu * nff)
        max_blocks = -(-max_act // QK_K)
        ad_len = max(max_blocks, (nff // QK_K) * nu)

        def f(n):
            b = DevBuf.zeroed(n * ms * 4)
            self._bufs.append(b)
            return b

        def z(nbytes):
            b = DevBuf.zeroed(nbytes)
            self._bufs.append(b)
            return b
        self.s = dict(
            x=f(E), xb=f(E), xb2=f(E), q=f(nh * hd), k=f(kv_dim), v=f(kv_dim), attn=f(nh * hd),
            aq=z(max_blocks * 256 * ms), ad=f(ad_len), router_logits=f(ne), router_probs=f(ne),
            expert_ids=z(nu * 4 * ms), expert_w=f(nu), e_gate=f(nu * nff), e_up=f(nu * nff),
            e_act=f(nu * nff), e_down=f(nu * E), scores=f(nh * max_kv), logits=f(V),
            amax_v=f(ARGMAX_BLOCKS), amax_i=z(ARGMAX_BLOCKS * 4 * ms), out_token=z(4 * ms),
            meta=z(8 * ms), inv=f(1), qb=z(ad_len * 256 * ms), sb=z(ad_len * 16 * 4 * ms))
        self.kc = [z(max_kv * kv_dim * 4 * ms) for _ in range(hp["n_layer"])]
        self.vc = [z(max_kv * kv_dim * 4 * ms) for _ in range(hp["n_layer"])]
        self._captured = False
        _check()

    # ---- DeviceModel::queue_token (device.rs:486-649) ------------------------------
    def queue_token(self):
        L, hp, s = self.L, self.hp, {k: v.ptr for k, v in self.s.items()}
        E, nh, nkv, hd = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["hd"]
        ne, nu, nff = hp["n_expert"], hp["n_used"], hp["n_ff"]
        eps, fb = F(hp["eps"]), F(hp["base"])
        kv_dim = nkv * hd
        L.llamd_fwd_embed_meta(self.tok_embd.ptr, s["meta"], s["x"], self.embd_blocks)
        for il, l in enumerate(self.layers):
            L.llamd_fwd_rms_norm_quant(s["x"], l["attn_norm"].ptr, s["xb"], s["aq"], s["ad"], s["inv"],
                                       E, eps)
            q, k, v = l["attn_q"], l["attn_k"], l["attn_v"]
            L.llamd_fwd_planar_x3(q.buf.ptr, q.off, k.buf.ptr, k.off, v.buf.ptr, v.off, s["aq"], s["ad"],
                                  s["q"], s["k"], s["v"], q.blocks, nh * hd, kv_dim, kv_dim)
            L.llamd_fwd_norm_rope(s["q"], l["attn_q_norm"].ptr, nh, hd, s["meta"], fb, eps)
            L.llamd_fwd_k_norm_rope_store(s["k"], l["attn_k_norm"].ptr, s["v"], self.kc[il].ptr,
                                          self.vc[il].ptr, nkv, hd, kv_dim, s["meta"], fb, eps)
            L.llamd_fwd_attention_meta(s["q"], self.kc[il].ptr, self.vc[il].ptr, s["attn"], s["scores"],
                                       nh, nkv, hd, s["meta"], self.max_kv)
            L.llamd_fwd_quantize(s["attn"], s["aq"], s["ad"], (nh * hd) // QK_K)
            o = l["attn_out"]
            L.llamd_fwd_planar_matvec(o.buf.ptr, o.off, s["aq"], s["ad"], s["xb2"], o.blocks, E)
            L.llamd_fwd_add(s["x"], s["xb2"], s["x"], E)
            L.llamd_fwd_rms_norm_quant(s["x"], l["ffn_norm"].ptr, s["xb"], s["aq"], s["ad"], s["inv"],
                                       E, eps)
            L.llamd_fwd_matvec_f32(l["ffn_gate_inp"].ptr, s["xb"], s["router_logits"], E, ne)
            L.llamd_fwd_router(s["router_logits"], ne, nu, s["expert_ids"], s["expert_w"],
                               s["router_probs"])
            ga, up, dn = l["ffn_gate_exps"], l["ffn_up_exps"], l["ffn_down_exps"]
            L.llamd_fwd_planar_grouped_x2(ga.buf.ptr, ga.off, up.buf.ptr, up.off, s["expert_ids"], s["aq"],
                                          s["ad"], s["e_gate"], s["e_up"], ga.blocks, nff, nu)
            L.llamd_fwd_silu_mul(s["e_gate"], s["e_up"], s["e_act"], nu * nff)
            L.llamd_fwd_quantize(s["e_act"], s["aq"], s["ad"], (nu * nff) // QK_K)
            L.llamd_fwd_planar_grouped_pa(dn.buf.ptr, dn.off, s["expert_ids"], s["aq"], s["ad"],
                                          s["e_down"], dn.blocks, E, nu)
            L.llamd_fwd_moe_combine_add(s["e_down"], s["expert_w"], s["x"], s["x"], nu, E)
        L.llamd_fwd_rms_norm_mul(s["x"], self.output_norm.ptr, s["xb"], E, eps)
        L.llamd_fwd_quantize(s["xb"], s["aq"], s["ad"], E // QK_K)
        out = self.output
        L.llamd_fwd_planar_matvec(out.buf.ptr, out.off, s["aq"], s["ad"], s["logits"], out.blocks,
                                  hp["n_vocab"])
        L.llamd_fwd_argmax(s["logits"], hp["n_vocab"], s["amax_v"], s["amax_i"], s["out_token"],
                           ARGMAX_BLOCKS)

    # ---- DeviceModel::capture / forward (device.rs:651-722) -------------------------
    def _capture(self):
        if self.L.llamd_fwd_begin_capture():
            raise HipError(f"begin_capture: {last_error()}")
        try:
            self.queue_token()
        except Exception:
            self.L.llamd_fwd_end_capture()
            self.L.llamd_fwd_graph_destroy()
            raise
        if self.L.llamd_fwd_end_capture():
            raise HipError(f"end_capture: {last_error()}")
        self._captured = True

    def enqueue(self, token: int, pos: int):
        """forward() up to its one synchronisation: meta upload, then the
        graph's replay (captured on first use) or the queued launches."""
        if pos >= self.max_kv:
            raise HipError(f"position {pos} beyond the {self.max_kv} allocated")
        self.s["meta"].upload(np.array([token, pos], np.int32))
        if self.use_graph:
            if not self._captured or not self.L.llamd_fwd_has_graph():
                self.L.llamd_fwd_graph_destroy()
                self._capture()
            if self.L.llamd_fwd_graph_launch():
                raise HipError(f"graph_launch: {last_error()}")
        else:
            self.queue_token()

    def forward(self, token: int, pos: int) -> int:
        self.enqueue(token, pos)
        _check()  # THE ONE SYNCHRONISE (device.rs:709)
        got = self.s["out_token"].download(np.zeros(1, np.int32))
        if not 0 <= got[0] < self.hp["n_vocab"]:
            raise HipError(f"argmax returned {got[0]}")
        return int(got[0])

    def logits(self, nseq: int = 1) -> np.ndarray:
        return self.s["logits"].download(np.empty((nseq, self.hp["n_vocab"]), np.float32))

    # ---- DeviceModel::forward_batch (device.rs:741-962) ----------------------------
    def forward_batch(self, tokens, positions) -> list:
        L, hp = self.L, self.hp
        nseq = len(tokens)
        if nseq == 0 or nseq != len(positions) or nseq > self.max_seq:
            raise HipError(f"{nseq} tokens, {len(positions)} positions, max_seq {self.max_seq}")
        if any(p >= self.max_kv for p in positions):
            raise HipError("a position beyond the cache")
        self.s["meta"].upload(np.array([v for tp in zip(tokens, positions) for v in tp], np.int32))
        s = {k: v.ptr for k, v in self.s.items()}
        E, nh, nkv, hd = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["hd"]
        ne, nu, nff, V = hp["n_expert"], hp["n_used"], hp["n_ff"], hp["n_vocab"]
        eps, fb = F(hp["eps"]), F(hp["base"])
        kv_dim = nkv * hd
        L.llamd_b_embed(self.tok_embd.ptr, s["meta"], s["x"], self.embd_blocks, nseq)
        for il, l in enumerate(self.layers):
            L.llamd_u_norm_quant(s["x"], l["attn_norm"].ptr, s["xb"], s["qb"], s["sb"], s["ad"], s["inv"],
                                 E, nseq, eps)
            q, k, v = l["attn_q"], l["attn_k"], l["attn_v"]
            L.llamd_u_x3(q.buf.ptr, q.off, k.buf.ptr, k.off, v.buf.ptr, v.off, s["qb"], s["sb"], s["ad"],
                         s["q"], s["k"], s["v"], q.blocks, nh * hd, kv_dim, kv_dim, nseq)
            L.llamd_b_norm_rope(s["q"], l["attn_q_norm"].ptr, nh, hd, s["meta"], nseq, fb, eps)
            L.llamd_b_k_norm_rope_store(s["k"], l["attn_k_norm"].ptr, s["v"], self.kc[il].ptr,
                                        self.vc[il].ptr, nkv, hd, kv_dim, self.max_kv, s["meta"], nseq,
                                        fb, eps)
            L.llamd_b_attention(s["q"], self.kc[il].ptr, self.vc[il].ptr, s["attn"], s["scores"], nh,
                                nkv, hd, self.max_kv, s["meta"], nseq)
            L.llamd_u_quantize(s["attn"], s["qb"], s["sb"], s["ad"], ((nh * hd) // QK_K) * nseq)
            o = l["attn_out"]
            L.llamd_u_matvec(o.buf.ptr, o.off, s["qb"], s["sb"], s["ad"], s["xb2"], o.blocks, E, nseq)
            L.llamd_b_add(s["x"], s["xb2"], s["x"], E * nseq)
            L.llamd_u_norm_quant(s["x"], l["ffn_norm"].ptr, s["xb"], s["qb"], s["sb"], s["ad"], s["inv"],
                                 E, nseq, eps)
            L.llamd_b_matvec_f32(l["ffn_gate_inp"].ptr, s["xb"], s["router_logits"], E, ne, nseq)
            L.llamd_b_router(s["router_logits"], ne, nu, s["expert_ids"], s["expert_w"],
                             s["router_probs"], nseq)
            ga, up, dn = l["ffn_gate_exps"], l["ffn_up_exps"], l["ffn_down_exps"]
            L.llamd_u_grouped_x2(ga.buf.ptr, ga.off, up.buf.ptr, up.off, s["expert_ids"], s["qb"], s["sb"],
                                 s["ad"], s["e_gate"], s["e_up"], ga.blocks, nff, nu, nseq)
            L.llamd_b_silu_mul(s["e_gate"], s["e_up"], s["e_act"], nu * nff * nseq)
            L.llamd_u_quantize(s["e_act"], s["qb"], s["sb"], s["ad"], ((nu * nff) // QK_K) * nseq)
            L.llamd_u_grouped_pa(dn.buf.ptr, dn.off, s["expert_ids"], s["qb"], s["sb"], s["ad"],
                                 s["e_down"], dn.blocks, E, nu, nseq)
            L.llamd_b_moe_combine_add(s["e_down"], s["expert_w"], s["x"], s["x"], nu, E, nseq)
        L.llamd_b_rms_norm_mul(s["x"], self.output_norm.ptr, s["xb"], E, nseq, eps)
        L.llamd_u_quantize(s["xb"], s["qb"], s["sb"], s["ad"], (E // QK_K) * nseq)
        out = self.output
        L.llamd_u_matvec(out.buf.ptr, out.off, s["qb"], s["sb"], s["ad"], s["logits"], out.blocks, V,
                         nseq)
        L.llamd_b_argmax(s["logits"], V, s["amax_v"], s["amax_i"], s["out_token"], ARGMAX_BLOCKS, nseq)
        _check()  # ONE synchronise for the whole batch (device.rs:946)
        got = self.s["out_token"].download(np.zeros(nseq, np.int32))
        if ((got < 0) | (got >= V)).any():
            raise HipError(f"argmax returned {got}")
        return [int(t) for t in got]

    def close(self):
        if self._captured:
            self.L.llamd_fwd_graph_destroy()
            self._captured = False
        _check()
        for b in self._bufs + self.kc + self.vc:
            b.free()
        self._bufs, self.kc, self.vc = [], [], []
