/*
 * llamd_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul backend for
 * llamd.rs.
 *
 * The boundary is the one the reference's llamd-rocm crate binds through
 * `unsafe extern "C"` (crates/llamd-rocm/src/lib.rs:67-137): plain pointers,
 * int sizes, int return codes (0 ok, -1 failure; pointer-returning calls give
 * NULL on failure). Functions that exist in the reference keep its name and
 * signature; each cites the definition it replaces. Functions the reference
 * does not have are prefixed llamd_hip_ and say so.
 *
 * Weights: the kernels read Q6_K in this backend's tiled device layout (a
 * pure byte/bit permutation of ggml's, see llamd_hip_q6k_tile), uploaded with
 * llamd_rocm_upload_q6k. Every Q6_K entry point also accepts the reference's
 * own device forms, unchanged: ggml bytes (llamd_rocm_upload, or
 * llamd_fwd_alloc + llamd_fwd_upload) and the planar repack (the
 * llamd_fwd_planar_* / llamd_u_* entry points, with its plane offsets). Such
 * a tensor gets a tiled copy on first use, re-made when the library writes
 * its bytes (llamd_fwd_upload / llamd_fwd_memset) and freed with it
 * (llamd_fwd_free / llamd_rocm_release); it must lie in memory from
 * llamd_fwd_alloc or llamd_rocm_upload. Rows of one matrix are
 * k = blocks*256 weights; an expert tensor is n_expert matrices uploaded as
 * one (rows*n_expert rows, rows % 16 == 0) or with
 * llamd_rocm_upload_q6k_experts.
 *
 * Activations follow the reference's BlockQ8K split into arrays: qs (int8,
 * 256 per block), d (f32 per block), bsums (int16, 16 per block).
 *
 * Results: every Q6_K matvec output, Q8_K quantization, dequantization,
 * expert id, routing weight, MoE decode-layer output and argmax id is
 * bit-identical to the reference CPU path (llamd-quant/llamd-models/
 * llamd-runtime); Q8_0/F32 matvecs are within
 * llamd-core::tolerance::REDUCTION.
 *
 * Threading: all device work is queued on one library-owned stream
 * (llamd_fwd_get_stream). Host-in/host-out calls synchronise that stream and
 * are serialised internally. Device-pointer calls (llamd_fwd_*) are
 * asynchronous; call llamd_fwd_sync before reading results.
 */
#ifndef LLAMD_HIP_H
#define LLAMD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device inventory ------------------------------------------------------ */
/* crates/llamd-rocm/kernels/llamd.hip:36-40 */
int llamd_rocm_device_count(void);
/* llamd.hip:42-61. On CDNA `wgp_count` is the compute-unit count (256 on
 * MI355X) and `warp_size` is 64. */
int llamd_rocm_device_info(int dev, char *name, int name_len, char *arch, int arch_len,
                           size_t *total_mem, int *wgp_count, int *warp_size);
/* llamd.hip:63-67 */
size_t llamd_rocm_free_mem(void);
/* Not in the reference: message for the last -1/NULL returned on this thread. */
const char *llamd_hip_last_error(void);
/* Not in the reference: overrides that pin one of the library's live code
 * paths, for tests and measurement (every path gives the same bits). Returns
 * the previous value, -1 for an unknown key or value.
 *   "mv_ks": waves per 16-row tile of the Q6_K matvec, 1, 4 or 8 (0: by
 *     shape, the default; all three are chosen by shape somewhere);
 *   "batched_twin": the grouped prefill GEMM's waves take two 16-token
 *     chunks of one expert (1, default) or one (0, the kernel ungrouped
 *     batches always use);
 *   "moe_polls": loads a wait inside the MoE decode kernel makes before the
 *     waiting wave computes the awaited router logit itself (default 2^18;
 *     0 = at once);
 *   "batch_decode_max", "model_graph", "model_fused_attn",
 *     "model_fused_norm", "model_norm_qkv", "model_prefetch": batched-decode threshold and
 *     decode-step choices;
 *   "model_long_from": the decode step's position from which the attention
 *     runs split over the GPU (default 256; -1 never), read at model create. */
int llamd_hip_tune(const char *key, int value);

/* ---- raw device memory and the stream ------------------------------------ */
/* llamd.hip:153-165 */
void *llamd_rocm_upload(const void *host, size_t bytes);
void llamd_rocm_release(void *dev);
/* llamd_forward.hip:711-745 */
void *llamd_fwd_get_stream(void);
int llamd_fwd_stream_init(void);
/* forward.rs:613-617 / llamd_forward.hip:879-910: capture the library
 * stream into one graph, replay it, query and drop it. Nothing runs between
 * begin and end; the first results come from the first replay. */
int llamd_fwd_begin_capture(void);
int llamd_fwd_end_capture(void);
int llamd_fwd_graph_launch(void);
int llamd_fwd_has_graph(void);
void llamd_fwd_graph_destroy(void);
void *llamd_fwd_alloc(size_t bytes);
void llamd_fwd_free(void *p);
int llamd_fwd_upload(void *dst, const void *src, size_t bytes);
int llamd_fwd_download(void *dst, const void *src, size_t bytes);
int llamd_fwd_sync(void);
/* -1 if queued work failed, or if a void device-pointer entry point refused
 * its arguments since the last call (the reason is in llamd_hip_last_error). */
int llamd_fwd_last_error(void);
/* llamd_forward.hip:735-737, as a fill kernel on the library stream (no
 * memset node when captured). */
int llamd_fwd_memset(void *p, int value, size_t bytes);
/* llamd_forward.hip:747-751 */
size_t llamd_fwd_free_mem(void);

/* ---- weight layouts (host-side, no device needed) ------------------------- */
/* Not in the reference (its closest relative is the planar repack,
 * crates/llamd-quant/src/dot.rs:349-423). Tiled Q6_K: see llamd_rs_amd/csrc/
 * host/layout.cpp for the byte map. */
size_t llamd_hip_q6k_tiled_bytes(int rows, int blocks);
int llamd_hip_q6k_tile(const void *ggml, int rows, int blocks, void *out);
int llamd_hip_q6k_untile(const void *tiled, int rows, int blocks, void *ggml_out);
size_t llamd_hip_q8_0_planar_bytes(int rows, int k);
int llamd_hip_q8_0_planarize(const void *ggml, int rows, int k, void *out);

/* ---- weight upload -------------------------------------------------------- */
/* Replaces the llamd_rocm_upload call in DeviceWeights::upload
 * (crates/llamd-rocm/src/lib.rs:277-308): ggml Q6_K bytes [rows][blocks*210]
 * -> tiled device copy. Release with llamd_rocm_release. */
void *llamd_rocm_upload_q6k(const void *ggml, int rows, int blocks);
/* Not in the reference: n_expert matrices of [rows][blocks*210] each (the 3D
 * expert tensor of crates/llamd-models/src/model.rs:188-227), each tiled on
 * its own so rows need not be a multiple of 16. */
void *llamd_rocm_upload_q6k_experts(const void *ggml, int n_expert, int rows, int blocks);
/* Not in the reference: Q8_0 [rows][k/32*34] -> planar device copy. */
void *llamd_hip_upload_q8_0(const void *ggml, int rows, int k);

/* ---- host-in / host-out (correctness and tests) --------------------------- */
/* llamd.hip:1053-1085: y[r] = dot_q6k_q8k(row r, act), all rows. */
int llamd_rocm_matvec_q6k_resident(const void *d_w, const int8_t *aq, const float *ad, float *out,
                                   int blocks, int rows);
/* llamd.hip:1164-1199: out[e][r] for the n_used experts eid[e] of a weight
 * uploaded as rows*n_expert rows. Refuses ids out of range, rows that do not
 * divide the upload, rows <= 0, n_used <= 0 (grouped_expert.rs:204-224). */
int llamd_rocm_matvec_grouped(const void *d_w, const int32_t *eid, const int8_t *aq,
                              const float *ad, float *out, int blocks, int rows, int n_used);
/* Counterpart of llamd_fwd_matvec_grouped_pa (llamd.hip:1334-1346), host in
 * and out: slot e uses its own activation (aq/ad hold n_used activations). */
int llamd_hip_matvec_grouped_pa(const void *d_w, const int32_t *eid, const int8_t *aq,
                                const float *ad, float *out, int blocks, int rows, int n_used);
/* Not in the reference (its batched kernels cap at 8, llamd_batch.hip:41):
 * out[s][r] = dot_q6k_q8k(row r, act s) for nseq activations, weights read
 * once per 16 sequences. */
int llamd_hip_matvec_q6k_batched(const void *d_w, const int8_t *aq, const float *ad, float *out,
                                 int blocks, int rows, int nseq);
/* llamd.hip:1258-1298: bit-exact quantize_q8_k on the device. bsums may be NULL. */
int llamd_rocm_quantize_q8k(const float *x, int nblocks, int8_t *qs, float *d, int16_t *bsums);
/* Not in the reference: act = silu(gate) * up (CpuBackend::silu/mul) then
 * Q8_K, fused. act may be NULL. */
int llamd_hip_swiglu_q8k(const float *gate, const float *up, int nblocks, float *act, int8_t *qs,
                         float *d, int16_t *bsums);
/* Not in the reference: device dequantization (for the EXACT weight check). */
int llamd_hip_dequant_q6k(const void *d_w, int rows, int blocks, float *out);
int llamd_hip_dequant_q8_0(const void *d_w, int rows, int k, float *out);
/* Model::matvec_quant fallback for Q8_0 / F32 (model.rs:253-262), f32 act. */
int llamd_hip_matvec_q8_0(const void *d_w, const float *x, float *out, int rows, int k);
/* route(logits, n_used) (crates/llamd-models/src/moe.rs:73-113) on the device. */
int llamd_hip_route(const float *logits, int n_expert, int n_used, int32_t *ids, float *weights);
/* argmax per row of x[nseq][n], lowest index on ties (device_forward.rs:23-37). */
int llamd_hip_argmax(const float *x, int n, int nseq, int32_t *ids);

/* ---- device-pointer launchers on the library stream (asynchronous) -------- */
/* llamd.hip:1313-1320 */
void llamd_fwd_matvec(const void *d_w, const int8_t *d_aq, const float *d_ad, float *d_out,
                      int blocks, int rows);
/* llamd.hip:1322-1332 */
void llamd_fwd_matvec_grouped(const void *d_w, const int32_t *d_ids, const int8_t *d_aq,
                              const float *d_ad, float *d_out, int blocks, int rows, int n_used);
/* llamd.hip:1334-1346 */
void llamd_fwd_matvec_grouped_pa(const void *d_w, const int32_t *d_ids, const int8_t *d_aq,
                                 const float *d_ad, float *d_out, int blocks, int rows,
                                 int n_used);
/* llamd.hip:1400-1411: Q, K, V (any three Q6_K matrices with the same k)
 * on one activation in ONE launch. */
void llamd_fwd_matvec_x3(const void *w0, const void *w1, const void *w2, const int8_t *d_aq,
                         const float *d_ad, float *o0, float *o1, float *o2, int blocks, int rows0,
                         int rows1, int rows2);
/* llamd.hip:1413-1424: gate and up of the same experts in ONE launch;
 * oa, ob: [n_used][rows]. */
void llamd_fwd_matvec_grouped_x2(const void *wa, const void *wb, const int32_t *d_ids,
                                 const int8_t *d_aq, const float *d_ad, float *oa, float *ob,
                                 int blocks, int rows, int n_used);
/* llamd.hip:1426-1466: the split-K variants. nsub is accepted and ignored:
 * the library chooses the split of K itself (the results do not depend on
 * it: every split folds the per-block terms in block order). */
void llamd_fwd_matvec_x3_splitk(const void *w0, const void *w1, const void *w2, const int8_t *d_aq,
                                const float *d_ad, float *o0, float *o1, float *o2, int blocks,
                                int rows0, int rows1, int rows2, int nsub);
void llamd_fwd_matvec_grouped_x2_splitk(const void *wa, const void *wb, const int32_t *d_ids,
                                        const int8_t *d_aq, const float *d_ad, float *oa,
                                        float *ob, int blocks, int rows, int n_used, int nsub);
void llamd_fwd_matvec_grouped_pa_splitk(const void *d_w, const int32_t *d_ids, const int8_t *d_aq,
                                        const float *d_ad, float *d_out, int blocks, int rows,
                                        int n_used, int nsub);
/* llamd.hip:1607-1611: qs, d in the reference's layout (no bsums) */
void llamd_fwd_quantize(const float *d_x, int8_t *d_qs, float *d_d, int nblocks);
/* llamd_forward.hip:802-805 (exact SiLU: glibc-identical expf) */
void llamd_fwd_silu_mul(const float *gate, const float *up, float *out, int n);
/* llamd_forward.hip:807-811, from given logits (n_expert <= 256). probs
 * (optional) receives route()'s softmax over every expert. */
void llamd_fwd_router(const float *logits, int n_expert, int n_used, int32_t *ids,
                      float *weights, float *probs);
/* llamd_forward.hip:759-763: out = rms_norm(x) * w over one row of n.
 * Bit-identical to CpuBackend::rms_norm + mul (llamd-cpu/src/lib.rs:55-75,
 * 112-113): in-order f32 sum of squares, correctly rounded sqrt and divide.
 * n <= 8192. */
void llamd_fwd_rms_norm_mul(const float *d_x, const float *d_w, float *d_out, int n, float eps);
/* llamd_forward.hip:765-770: the same per head (QK-norm, layer.rs:62-79):
 * n_head rows of hd, each multiplied by w[0..hd). */
void llamd_fwd_head_rms_norm_mul(const float *d_x, const float *d_w, float *d_out, int n_head,
                                 int hd, float eps);
/* llamd_forward.hip:845-855: rms_norm(x) * w, then Q8_K of the result (qs,
 * d in the reference's layout) for the Q/K/V matvecs; out (the f32 result)
 * and inv_scratch (the row's scale) are written when non-NULL. n % 256 == 0,
 * n <= 8192. */
void llamd_fwd_rms_norm_quant(const float *d_x, const float *d_w, float *d_out, int8_t *d_qs,
                              float *d_d, float *d_inv_scratch, int n, float eps);
/* llamd_forward.hip:813-817: out = sum_e w[e] * down[e] (no residual). */
void llamd_fwd_moe_combine(const float *d_down, const float *d_weights, float *d_out, int n_used,
                           int n_embd);
void llamd_fwd_moe_combine_add(const float *down, const float *weights, const float *residual,
                               float *out, int n_used, int n_embd);
/* llamd_forward.hip:819-825; scratch_v/scratch_i hold nblocks partials. */
void llamd_fwd_argmax(const float *x, int n, float *scratch_v, int32_t *scratch_i, int32_t *out,
                      int nblocks);
/* llamd_forward.hip:792-796. Each row is the CPU path's sequential f32 fold
 * (model.rs:253-262: rounded products added in order), bit for bit, when k is
 * a multiple of 256 up to 2048 (the MoE router's shape); other k use FMA
 * accumulation (REDUCTION). */
void llamd_fwd_matvec_f32(const float *w, const float *x, float *out, int k, int rows);
/* Not in the reference (its Q8_0 path is CPU-only, model.rs:253-262): Q8_0
 * weight from llamd_hip_upload_q8_0 times an f32 activation. */
void llamd_hip_fwd_matvec_q8_0(const void *d_w, const float *d_x, float *d_out, int rows, int k);
/* llamd.hip:1389-1398; nsub ignored as for the other split-K spellings. */
void llamd_fwd_matvec_splitk(const void *d_w, const int8_t *d_aq, const float *d_ad, float *d_out,
                             int blocks, int rows, int nsub);
/* llamd.hip:1348-1387: timing of llamd_fwd_matvec (host activations), ms. */
int llamd_rocm_splitk_bench(const void *d_w, const int8_t *aq, const float *ad, int blocks,
                            int rows, int nsub, int iters, float *ms_out);

/* ---- the planar repack (PlanarWeights, crates/llamd-rocm/src/lib.rs:619-843) */
/* off = {ql, qh, sc, d} plane offsets from PlanarQ6K::layout
 * (crates/llamd-quant/src/dot.rs:349-398), a host array; base a device
 * buffer holding the repack. Same results as the ggml-layout calls. */
/* llamd.hip:1470-1478 */
void llamd_fwd_planar_matvec(const void *base, const size_t *off, const int8_t *d_aq,
                             const float *d_ad, float *d_out, int blocks, int rows);
/* llamd.hip:1480-1491 */
void llamd_fwd_planar_grouped(const void *base, const size_t *off, const int32_t *d_ids,
                              const int8_t *d_aq, const float *d_ad, float *d_out, int blocks,
                              int rows, int n_used);
/* llamd.hip:1493-1504 */
void llamd_fwd_planar_grouped_pa(const void *base, const size_t *off, const int32_t *d_ids,
                                 const int8_t *d_aq, const float *d_ad, float *d_out, int blocks,
                                 int rows, int n_used);
/* llamd.hip:1506-1522 */
void llamd_fwd_planar_x3(const void *b0, const size_t *f0, const void *b1, const size_t *f1,
                         const void *b2, const size_t *f2, const int8_t *d_aq, const float *d_ad,
                         float *o0, float *o1, float *o2, int blocks, int rows0, int rows1,
                         int rows2);
/* llamd.hip:1524-1538 */
void llamd_fwd_planar_grouped_x2(const void *ba, const size_t *fa, const void *bb, const size_t *fb,
                                 const int32_t *d_ids, const int8_t *d_aq, const float *d_ad,
                                 float *oa, float *ob, int blocks, int rows, int n_used);
/* llamd.hip:1542-1564: host activations in, host results out. */
int llamd_rocm_planar_matvec(const void *base, const size_t *off, const int8_t *aq,
                             const float *ad, float *out, int blocks, int rows);
/* llamd.hip:1567-1605: ms for iters launches. */
int llamd_rocm_planar_bench(const void *base, const size_t *off, const int8_t *aq, const float *ad,
                            int blocks, int rows, int iters, float *ms_out);

/* ---- the rest of the decode step (llamd_forward.hip), bit-exact ----------- */
/* Each matches the reference CPU path's f32 operations (crates/llamd-cpu,
 * crates/llamd-runtime/src/layer.rs, attention.rs) bit for bit. RoPE angles
 * come from a table filled on the host with the reference's libm calls,
 * covering 32768 positions (more when a max_kv says so); a position beyond
 * it gives NaN. Attention covers at most 16384 positions; the scores buffer
 * is not used. meta = {token, pos} on the device. */
/* llamd_forward.hip:753-757: row `token` of a ggml Q6_K table, dequantized */
void llamd_fwd_embed(const void *table, int token, float *out, int blocks);
/* llamd_forward.hip:863-868: the token read from meta[0] */
void llamd_fwd_embed_meta(const void *table, const int32_t *meta, float *out, int blocks);
/* llamd_forward.hip:772-776: NeoX RoPE in place at pos */
void llamd_fwd_rope(float *x, int pos, int n_head, int hd, float freq_base);
/* llamd_forward.hip:827-833: per-head QK-norm (w may be NULL) + RoPE at meta[1] */
void llamd_fwd_norm_rope(float *x, const float *w, int n_head, int hd, const int32_t *meta,
                         float freq_base, float eps);
/* llamd_forward.hip:835-843: the same for K (in place), then K and V stored
 * at cache row meta[1]; kv_dim must be n_head_kv * hd */
void llamd_fwd_k_norm_rope_store(float *k, const float *w, const float *v, float *kc, float *vc,
                                 int n_head_kv, int hd, int kv_dim, const int32_t *meta,
                                 float freq_base, float eps);
/* llamd_forward.hip:778-782 */
void llamd_fwd_kv_store(float *kc, float *vc, const float *k, const float *v, int pos, int kv_dim);
/* llamd_forward.hip:784-790: attend over n_kv cached positions */
void llamd_fwd_attention(const float *q, const float *kc, const float *vc, float *out,
                         float *scores, int n_head, int n_head_kv, int hd, int n_kv);
/* llamd_forward.hip:870-877: n_kv = meta[1] + 1 */
void llamd_fwd_attention_meta(const float *q, const float *kc, const float *vc, float *out,
                              float *scores, int n_head, int n_head_kv, int hd, const int32_t *meta,
                              int max_kv);
/* llamd_forward.hip:798-800 */
void llamd_fwd_add(const float *a, const float *b, float *out, int n);

/* ---- batched decode (crates/llamd-rocm/kernels/llamd_batch.hip) ----------- */
/* nseq independent sequences; activations [nseq][...], results [nseq][...],
 * meta [nseq][2] = {token, pos}; each sequence owns a max_kv * kv_dim slice
 * of a layer's cache. Weights in ggml layout are read once per 16
 * sequences. Results equal nseq single-sequence calls, bit for bit. */
/* llamd_batch.hip:837: sequences per call (16) */
int llamd_batch_max_seq(void);
/* llamd_batch.hip:839-844 */
void llamd_b_embed(const void *table, const int32_t *meta, float *out, int blocks, int nseq);
/* llamd_batch.hip:846-853 */
void llamd_b_rms_norm_quant(const float *x, const float *w, float *out, int8_t *qs, float *d,
                            float *inv, int n, int nseq, float eps);
/* llamd_batch.hip:855-859 */
void llamd_b_rms_norm_mul(const float *x, const float *w, float *out, int n, int nseq, float eps);
/* llamd_batch.hip:861-864 */
void llamd_b_quantize(const float *x, int8_t *qs, float *d, int nblocks);
/* llamd_batch.hip:875-887 */
void llamd_b_matvec(const void *w, const int8_t *aq, const float *ad, float *out, int blocks,
                    int rows, int nseq);
/* llamd_batch.hip:889-906 */
void llamd_b_matvec_x3(const void *w0, const void *w1, const void *w2, const int8_t *aq,
                       const float *ad, float *o0, float *o1, float *o2, int blocks, int r0, int r1,
                       int r2, int nseq);
/* llamd_batch.hip:908-916: ids [nseq][n_used]; oa, ob [nseq][n_used][rows] */
void llamd_b_grouped_x2(const void *wa, const void *wb, const int32_t *ids, const int8_t *aq,
                        const float *ad, float *oa, float *ob, int blocks, int rows, int n_used,
                        int nseq);
/* llamd_batch.hip:918-925: activation (s, k) for slot (s, k) */
void llamd_b_grouped_pa(const void *w, const int32_t *ids, const int8_t *aq, const float *ad,
                        float *out, int blocks, int rows, int n_used, int nseq);
/* llamd_batch.hip:927-933 */
void llamd_b_norm_rope(float *x, const float *w, int n_head, int hd, const int32_t *meta, int nseq,
                       float freq_base, float eps);
/* llamd_batch.hip:935-944 */
void llamd_b_k_norm_rope_store(float *k, const float *w, const float *v, float *kc, float *vc,
                               int n_head_kv, int hd, int kv_dim, int max_kv, const int32_t *meta,
                               int nseq, float freq_base, float eps);
/* llamd_batch.hip:946-952 */
void llamd_b_attention(const float *q, const float *kc, const float *vc, float *out, float *scores,
                       int n_head, int n_head_kv, int hd, int max_kv, const int32_t *meta,
                       int nseq);
/* llamd_batch.hip:954-960 */
void llamd_b_add(const float *a, const float *b, float *o, int n);
void llamd_b_silu_mul(const float *g, const float *u, float *o, int n);
/* llamd_batch.hip:962-966: as llamd_fwd_matvec_f32 for every sequence, in
 * one launch (rows x nseq workgroups) when the fold applies */
void llamd_b_matvec_f32(const float *w, const float *x, float *out, int k, int rows, int nseq);
/* llamd_batch.hip:968-972 (n_expert <= 256) */
void llamd_b_router(const float *logits, int n_expert, int n_used, int32_t *ids, float *weights,
                    float *probs, int nseq);
/* llamd_batch.hip:974-980 */
void llamd_b_moe_combine_add(const float *down, const float *weights, const float *residual,
                             float *out, int n_used, int n_embd, int nseq);
/* llamd_batch.hip:982-988: sv, si hold nchunk partials per sequence */
void llamd_b_argmax(const float *x, int n, float *sv, int32_t *si, int32_t *out, int nchunk,
                    int nseq);

/* ---- unsigned-activation form (crates/llamd-rocm/kernels/llamd_udot.hip) -- */
/* qb = Q8_K quants biased to unsigned (q ^ 0x80), sb = per-16 sums of qb,
 * d as usual; weights in the planar repack. The matvecs recover the signed
 * quants exactly, so results are dot_q6k_q8k's bits (the reference's udot
 * kernels are only within REDUCTION of them); sb is produced, not read. */
/* llamd_udot.hip:599-600: accepted and reported; the kernels choose their tiling */
void llamd_u_set_tile(int t);
int llamd_u_get_tile(void);
/* llamd_udot.hip:584-587 (kernel uk_bias_sums, :55-75) */
void llamd_u_bias_sums(const int8_t *qs, uint8_t *qb, int32_t *sb, int nblocks);
/* llamd_udot.hip:569-576: rms_norm(x) * w -> out, qb, sb, d */
void llamd_u_norm_quant(const float *x, const float *w, float *out, uint8_t *qb, int32_t *sb,
                        float *d, float *inv, int n, int nseq, float eps);
/* llamd_udot.hip:578-582 */
void llamd_u_quantize(const float *x, uint8_t *qb, int32_t *sb, float *d, int nblocks);
/* llamd_udot.hip:602-663: out [nseq][rows] */
void llamd_u_matvec(const void *base, const size_t *off, const uint8_t *qb, const int32_t *sb,
                    const float *ad, float *out, int blocks, int rows, int nseq);
void llamd_u_x3(const void *b0, const size_t *f0, const void *b1, const size_t *f1, const void *b2,
                const size_t *f2, const uint8_t *qb, const int32_t *sb, const float *ad, float *o0,
                float *o1, float *o2, int blocks, int r0, int r1, int r2, int nseq);
void llamd_u_grouped_x2(const void *ba, const size_t *fa, const void *bb, const size_t *fb,
                        const int32_t *ids, const uint8_t *qb, const int32_t *sb, const float *ad,
                        float *oa, float *ob, int blocks, int rows, int n_used, int nseq);
void llamd_u_grouped_pa(const void *base, const size_t *off, const int32_t *ids, const uint8_t *qb,
                        const int32_t *sb, const float *ad, float *out, int blocks, int rows,
                        int n_used, int nseq);
/* llamd_udot.hip:714-751, 756-785: host in, host out */
int llamd_u_norm_quant_host(const float *x, const float *w, int n, int nseq, float eps, float *out,
                            uint8_t *qb, int32_t *sb, float *d);
int llamd_u_quantize_host(const float *x, int nblocks, uint8_t *qb, int32_t *sb, float *d);
/* llamd_udot.hip:789-826: signed quants qs [nseq][blocks*256] from the host */
int llamd_u_matvec_host(const void *base, const size_t *off, const int8_t *qs, const float *ad,
                        float *out, int blocks, int rows, int nseq);
/* llamd_udot.hip:668-711: ms for iters launches */
int llamd_u_matvec_bench(const void *base, const size_t *off, const int8_t *qs, const float *ad,
                         int blocks, int rows, int nseq, int iters, float *ms_out);

/* ---- llamd-tensor Backend ops on device tensors --------------------------- */
/* Not in the reference's C ABI: the f32 half of the Backend trait
 * (crates/llamd-tensor/src/lib.rs:148-174), row-major [rows][n] device
 * tensors, bit-identical to CpuBackend (crates/llamd-cpu/src/lib.rs:55-224).
 * Asynchronous on the library stream except be_rope (host positions). */
int llamd_hip_be_rms_norm(const float *x, float *out, int rows, int n, float eps);
int llamd_hip_be_softmax(const float *x, float *out, int rows, int n);
int llamd_hip_be_silu(const float *x, float *out, size_t n);
int llamd_hip_be_add(const float *a, const float *b, float *out, size_t n);
int llamd_hip_be_mul(const float *a, const float *b, float *out, size_t n);
int llamd_hip_be_scale(const float *x, float by, float *out, size_t n);
/* out [n][m] = w [m][k] . x [n][k] (ggml order: w [k, m], x [k, n]) */
int llamd_hip_be_matmul(const float *w, const float *x, float *out, int m, int n, int k);
/* NeoX RoPE of rows [rows][row_len] (heads of head_dim), row r at
 * positions[r] * freq_scale; positions is a host array */
int llamd_hip_be_rope(float *x, int rows, int row_len, const uint32_t *positions, int head_dim,
                      float freq_base, float freq_scale);
/* rows ids[j] (host array) of table [table_rows][row_len] -> out [n_ids][row_len] */
int llamd_hip_be_get_rows(const float *table, int table_rows, int row_len, const uint32_t *ids,
                          int n_ids, float *out);

/* ---- one MoE decode layer (R8 router -> R9 route -> R11 moe_ffn -> R12) ---- */
/* Not in the reference as one call: DeviceModel::queue_token's MoE phases
 * (crates/llamd-runtime/src/device.rs:486-655) behind a handle.
 * router: f32 [n_expert][n_embd]; gate/up: ggml Q6_K [n_expert][n_ff][n_embd];
 * down: ggml Q6_K [n_expert][n_embd][n_ff]. */
void *llamd_hip_moe_create(const float *router, const void *gate, const void *up,
                           const void *down, int n_embd, int n_ff, int n_expert, int n_used);
void llamd_hip_moe_destroy(void *h);
/* router (the reference's sequential f32 fold) -> route -> gate/up -> SwiGLU
 * -> down -> weighted combine (+ residual), bit-identical to the CPU path on
 * every call. flags: reserved, pass 0 (bit 0, "exact", is accepted and is
 * what every call does). Device pointers, asynchronous. d_res may be NULL
 * (then out = moe_ffn only). */
int llamd_hip_moe_forward(void *h, const float *d_x, const float *d_res, float *d_out, int flags);
/* Host in/out; ids/weights/logits (optional) receive the routing. */
int llamd_hip_moe_forward_host(void *h, const float *x, const float *res, float *out,
                               int32_t *ids, float *weights, float *logits, int flags);
/* Prefill / grouped path: n_tok tokens with GIVEN routing ids/weights
 * [n_tok][n_used] (device pointers), out [n_tok][n_embd] = moe_ffn per token.
 * Device ids are not read by the host: a pair whose id is outside
 * [0, n_expert) adds no term to its token (no memory outside the layer's
 * buffers is touched). The _host variant refuses such ids with an error. */
int llamd_hip_moe_prefill(void *h, const float *d_x, const int32_t *d_ids, const float *d_w,
                          float *d_out, int n_tok);
int llamd_hip_moe_prefill_host(void *h, const float *x, const int32_t *ids, const float *w,
                               float *out, int n_tok);
/* Not in the reference. flags 0: llamd_hip_moe_prefill. flags
 * LLAMD_HIP_REDUCTION: the grouped GEMMs accumulate a block's eight classes
 * in the matrix-core accumulators and fold one float term per (row, token,
 * block), instead of the reference's eight ordered class sums. Outputs are
 * then within tolerance::REDUCTION (rms-scaled, grouped_expert.rs:147-175) of
 * the CPU path, not bit-identical; the Q8_K bytes of x and of the SwiGLU
 * activations are the exact path's whenever the gate/up outputs round the
 * same way. Any other flag bit is an error. */
#define LLAMD_HIP_REDUCTION 1
int llamd_hip_moe_prefill_ex(void *h, const float *d_x, const int32_t *d_ids, const float *d_w,
                             float *d_out, int n_tok, int flags);
int llamd_hip_moe_prefill_host_ex(void *h, const float *x, const int32_t *ids, const float *w,
                                  float *out, int n_tok, int flags);
/* Batched decode (device.rs:741-962, forward_batch's MoE block): nseq
 * sequences x [nseq][n_embd], each routed by ITS OWN router logits (the
 * reference's sequential fold, all nseq x n_expert folds at once; then
 * softmax / top-k / renormalise per sequence), then the experts grouped
 * across the sequences so an expert's weights are read once per 16 tokens
 * routed to it; out = res + moe_ffn per sequence (res optional). Up to
 * llamd_hip_tune("batch_decode_max") sequences (12 by default) the decode
 * kernels run for every sequence instead. Bit-identical to nseq calls of
 * llamd_hip_moe_forward either way. Device pointers. */
int llamd_hip_moe_forward_batch(void *h, const float *d_x, const float *d_res, float *d_out,
                                int nseq);
/* Host in/out; ids / weights [nseq][n_used] and logits [nseq][n_expert] optional. */
int llamd_hip_moe_forward_batch_host(void *h, const float *x, const float *res, float *out,
                                     int32_t *ids, float *weights, float *logits, int nseq);
/* Routing statistics since create: calls, and calls routed on the exact
 * sequential router fold (every call, so the two are equal). */
int llamd_hip_moe_stats(void *h, int *calls, int *exact_calls);
/* Diagnostics, no counterpart in the reference: counters[4] = {calls,
 * exact calls, calls whose top-k set was certified from the logit estimates
 * (gate/up started before the exact fold ended), 1 if a wait inside the
 * decode kernel ever gave up and computed the awaited logit itself (same
 * bits; a timing event only)}; estimates (optional) [2][n_expert] = the
 * last call's estimates T and bounds E, |logit - T| <= E. Synchronous. */
int llamd_hip_moe_counters(void *h, int *counters, double *estimates);

/* ---- LM head: Q6_K matvec over the vocabulary + argmax -------------------- */
/* Not in the reference as one call (device.rs:640-655 queues the same ops).
 * d_x: [nseq][k] f32, d_logits: [nseq][rows] (always written), d_ids: [nseq].
 * Scratch for max_seq sequences is allocated at create and kept. */
void *llamd_hip_lmhead_create(const void *d_w, int rows, int blocks, int max_seq);
void llamd_hip_lmhead_destroy(void *h);
int llamd_hip_lmhead_forward(void *h, const float *d_x, int nseq, float *d_logits,
                             int32_t *d_ids);
/* flags 0: llamd_hip_lmhead_forward. flags LLAMD_HIP_REDUCTION with nseq > 1:
 * the logits come from the matrix-core kernel that folds one float term per
 * (row, token, block) and are within tolerance::REDUCTION of the CPU's
 * (rows whose tile could hold the maximum are recomputed exactly and carry
 * the CPU's bits); d_ids are still the reference's arg-max of the EXACT
 * logits, bit for bit: a rounding bound certifies which 16-row tiles can hold
 * the maximum, and only those are recomputed exactly. At nseq == 1 the call
 * is the exact one. Any other flag bit is an error. */
int llamd_hip_lmhead_forward_ex(void *h, const float *d_x, int nseq, float *d_logits,
                                int32_t *d_ids, int flags);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): llamd_hip_lmhead_forward without a handle, allocating nothing.
 * Its scratch is one file-scope device array per GPU (about 2.3 MB, held
 * until the process ends), so rows <= 262144, blocks <= 32 (k <= 8192) and
 * nseq <= 16; larger requests return -1. d_w is a tiled Q6_K handle of
 * exactly rows x blocks. Calls that overlap on one GPU race on the array. */
int llamd_hip_lmhead_forward_noalloc(const void *d_w, int rows, int blocks, const float *d_x,
                                     int nseq, float *d_logits, int32_t *d_ids);
/* Bytes of that array (for the caller's memory budget). */
size_t llamd_hip_lmhead_noalloc_scratch_bytes(void);

/* ---- timing on the library stream ---------------------------------------- */
/* Diagnostics, not in the reference. While d_slots is set, every Q6_K
 * batch-1 matvec launch (q6k_mv_b1: llamd_fwd_matvec, _grouped, _x3, the LM
 * head at batch 1, ...) records into the next of n_slots device records, in
 * turn: record r is 2048 uint64 words at d_slots + 2048 r; wave w of the grid
 * (w < 1024) stores its start at word w and its end at word 1024 + w, in
 * s_memrealtime ticks (100 MHz on gfx950). The launch's duration inside the
 * caller's back-to-back enqueue (not a tracer's isolated dispatch) is then
 * max(ends) - min(starts) over the words written; the caller zeroes the
 * records first. NULL turns it off. Not for captured graphs (the record is
 * chosen at launch). */
int llamd_hip_kernel_clock(unsigned long long *d_slots, int n_slots);

/* Not in the reference (its llamd_rocm_matvec_bench, llamd.hip:1101-1148,
 * times one kernel; these let the caller bracket any queued sequence). */
void *llamd_hip_event_create(void);
void llamd_hip_event_destroy(void *ev);
int llamd_hip_event_record(void *ev);
float llamd_hip_event_elapsed_ms(void *start, void *stop);
/* Not in the reference: a plain 16-byte-vector device copy of `bytes` (a
 * multiple of 16) on the library stream, asynchronous. Its known traffic
 * (bytes read, bytes written) calibrates the profiler's HBM counters. */
int llamd_hip_copy_calibration(void *d_dst, const void *d_src, size_t bytes);
/* Not in the reference: n launches of a read-only kernel (grid workgroups of
 * 256 threads) over `bytes` at d_src[i], back to back on the library stream,
 * asynchronous; bytes = 0 launches an empty kernel (d_src may be NULL). The
 * launch-cost reference for short kernels: what a launch costs with no work,
 * and with only the reads. */
int llamd_hip_read_many(const void *const *d_src, size_t bytes, int grid, int n);
/* Not in the reference: n launches of llamd_fwd_matvec (w[i], aq[i], ad[i],
 * out[i], blocks[i], rows[i]) enqueued by one call, for timing short launches
 * back to back without the caller's per-call overhead. 0, or -1 at the first
 * refused or failed launch (the earlier ones stay queued). */
int llamd_hip_matvec_many(const void *const *w, const int8_t *const *aq, const float *const *ad,
                          float *const *out, const int *blocks, const int *rows, int n);
/* llamd.hip:1101-1148: one warm launch, then iters launches, total ms. */
int llamd_rocm_matvec_bench(const void *d_w, const int8_t *aq, const float *ad, int blocks,
                            int rows, int iters, float *ms_out);
/* llamd.hip:1201-1252 */
int llamd_rocm_matvec_grouped_bench(const void *d_w, const int32_t *eid, const int8_t *aq,
                                    const float *ad, int blocks, int rows, int n_used, int iters,
                                    float *ms_out);

/* ---- GGUF: the model file in front of the path --------------------------- */
/* crates/llamd-gguf/src/lib.rs (Gguf::open / get / tensor / tensor_data) and
 * the upload side of crates/llamd-runtime/src/device.rs:224-256. Host-only
 * except the two uploads; the file is memory-mapped read-only and every
 * length in it is checked before use (lib.rs:141-236). NULL / -1 on failure,
 * with the reason in llamd_hip_last_error(). Pointers returned by
 * llamd_gguf_tensor_data stay valid until llamd_gguf_close. */
void *llamd_gguf_open(const char *path);
void llamd_gguf_close(void *g);
int llamd_gguf_header(void *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                      uint64_t *alignment, uint64_t *data_offset, uint64_t *file_size);
/* metadata entry i, keys in byte order (lib.rs:118 BTreeMap); types are
 * ggml's gguf_type (0 u8 .. 12 f64, 8 string, 9 array) */
int llamd_gguf_kv(void *g, uint64_t i, char *key, size_t cap, uint32_t *type,
                  uint32_t *arr_type, uint64_t *arr_len);
int64_t llamd_gguf_find_kv(void *g, const char *key);          /* -1 if absent */
int llamd_gguf_kv_bits(void *g, uint64_t i, uint64_t elem, uint64_t *bits);
int llamd_gguf_kv_str(void *g, uint64_t i, uint64_t elem, char *buf, size_t cap, uint64_t *len);
int llamd_gguf_get_u64(void *g, const char *key, uint64_t *out); /* Value::as_u64, lib.rs:55-67 */
int llamd_gguf_get_f32(void *g, const char *key, float *out);    /* Value::as_f32, lib.rs:68-74 */
/* tensor i in file order; dims in ggml order (dims[0] fastest), unused = 1 */
int llamd_gguf_tensor(void *g, uint64_t i, char *name, size_t cap, uint32_t *n_dims,
                      uint64_t dims[4], uint32_t *type, uint64_t *offset);
int64_t llamd_gguf_find_tensor(void *g, const char *name);     /* -1 if absent */
/* Gguf::tensor_data (lib.rs:256-278): F32, F16, Q8_0, Q6_K only */
const void *llamd_gguf_tensor_data(void *g, uint64_t i, uint64_t *nbytes);
/* A Q6_K tensor to the device, tiled (device.rs:236-248): 2D [k, rows] as
 * llamd_rocm_upload_q6k, 3D [k, rows, n_expert] as llamd_rocm_upload_q6k_experts. */
void *llamd_gguf_upload_q6k(void *g, const char *name);
/* blk.<layer>'s MoE FFN (ffn_gate_inp F32 router, ffn_{gate,up,down}_exps
 * Q6_K) as llamd_hip_moe_create, n_used from <arch>.expert_used_count. */
void *llamd_gguf_moe_create(void *g, int layer);

/* ---- resident whole-token decode (Qwen3-MoE) ------------------------------ */
/* DeviceModel::load / forward (crates/llamd-runtime/src/device.rs:262-722):
 * every weight of a qwen3moe GGUF uploaded once (Q6_K attention, experts and
 * output; F32 norms and router), a KV cache of max_kv positions (<= 16384),
 * and one synchronisation per token. A step is bit-identical to the
 * reference CPU composition (crates/llamd-runtime/src/layer.rs: forward).
 * The GGUF handle may be closed after create. */
void *llamd_hip_model_create(void *gguf, int max_kv);
void llamd_hip_model_destroy(void *m);
int llamd_hip_model_info(void *m, int *n_layer, int *n_embd, int *n_vocab, int *max_kv);
/* One token at position pos (positions 0..pos-1 already in the cache):
 * logits [n_vocab] and next = argmax (lowest index on ties), both optional. */
int llamd_hip_model_forward(void *m, int token, int pos, float *logits, int32_t *next);

#ifdef __cplusplus
}
#endif
#endif
