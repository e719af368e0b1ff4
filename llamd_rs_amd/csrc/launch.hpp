// launch.hpp -- host-side launchers of the gfx950 kernels (one per kernel
// family). Every launcher enqueues on the given stream and returns 0, or -1
// if the launch was rejected. Shapes are validated by the callers in capi.cpp
// before any launcher is reached.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace llamd {

// Tuning overrides (0 = automatic); set through llamd_hip_tune.
extern int g_tune_batched_twin;
extern int g_tune_fast_lds;  // LLAMD_HIP_REDUCTION LM head: the chunk's quants staged in LDS
extern int g_tune_fast_ks;  // LLAMD_HIP_REDUCTION batched kernels: waves per item (K split), 0 = by shape  // grouped q6k_mv_batched: two chunks of one expert per wave
extern int g_tune_mv_ks;  // waves per 16-row tile in q6k_mv_b1: 1, 2, 4 or 8 (0: automatic)
extern int g_tune_model_graph;  // 1: the decode step of llamd_hip_model_* is a captured graph
extern int g_tune_model_fused_attn;  // 1: attend_fused in the decode step
extern int g_tune_model_fused_norm;  // 1: the FFN norm inside the MoE decode launch
extern int g_tune_model_norm_qkv;    // 1: the attention norm inside the Q/K/V launch
extern int g_tune_model_prefetch;    // 1: the O weights read into L2 under the attention
extern int g_tune_model_long_from;   // decode step: the split attention from this position (-1: never)

// q6k_mv.hip
// y[slot][rows] = W[ids[slot]] . act; with w_b, also y[n_slots + slot] from
// w_b (gate and up in one launch). act_per_slot 0: every slot reads
// activation 0; d > 0: slot i reads activation i / d.
int launch_q6k_mv_b1(const void *w, size_t expert_stride, const int32_t *ids, const int8_t *aq,
                     const float *ad, float *y, int rows, int blocks, int n_slots, int act_per_slot,
                     hipStream_t st, const void *w_b = nullptr, float *amax_v = nullptr,
                     int *amax_i = nullptr);
// Down projection of n_slots routed experts (activation e for slot e) and the
// routing-weighted combine (+ residual) into out, one workgroup per 16 rows.
// One launch over up to three matrices sharing the activation (Q, K, V):
// y[i] = W[i] x, rows[i] each; n_mat in 1..3.
int launch_q6k_mv_x3(const void *const w[3], float *const y[3], const int rows[3], int n_mat,
                     const int8_t *aq, const float *ad, int blocks, hipStream_t st);
// Two expert tensors (same shape and stride) on the same ids and activation:
// oa = Wa[ids] x, ob = Wb[ids] x, each [n_used][rows].
int launch_q6k_mv_grouped_x2(const void *wa, const void *wb, size_t expert_stride,
                             const int32_t *ids, const int8_t *aq, const float *ad, float *oa,
                             float *ob, int rows, int blocks, int n_used, hipStream_t st,
                             int act_per_slot = 0);
// Gate and up of the routed experts in one launch, routing (softmax, top-k,
// renormalise) in the prologue on exact logits; y = [gate | up][n_used][rows].
int launch_q6k_mv_routed(const void *w, const void *w_b, size_t expert_stride,
                        const float *logits, int n_expert, int n_used, int32_t *ids_out,
                        float *w_out, int *stats, const int8_t *aq, const float *ad, float *y,
                        int rows, int blocks, hipStream_t st);
// Down projection of the routed experts' Q8_K activations [n_slots] + the
// weighted combine in routing order + residual.
int launch_q6k_down_combine(const void *w, size_t expert_stride, const int32_t *ids,
                            const int8_t *aq, const float *ad, const float *weights,
                            const float *res, float *out, int rows, int blocks, int n_slots,
                            hipStream_t st);
// Expert-grouped batched matvec (see q6k_mv.hip). Activations are in the
// token-chunked layout (q8k_wave.hpp): chunk k holds the 16 tokens of
// sub-tile k. sub_start has 2 * (n_groups + 1) entries: the prefix of
// ceil(count/16) per group, then (read while g_tune_batched_twin is on) the
// prefix of ceil(chunks/2), as launch_moe_group writes them; max_chunks bounds
// sub_start[n_groups] and sizes the grid. The output of the
// pair at sorted position i is row pair_out[i] of y (nullptr: row i). With
// grp_expert == nullptr there is a single group (expert 0) of n_groups tokens.
// moe_decode.hip: one MoE decode layer (router, top-k, gate, up, SwiGLU,
// down, combine, residual) in two launches, bit-identical to the reference.
struct MoeDecodeLaunch {
    const void *w_gate, *w_up, *w_down;
    size_t gu_stride, down_stride;
    const float *router, *x, *res;  // res may be null
    float *out, *logits;            // [k], [n_expert]
    double *est;                    // [2 * n_expert] diagnostic copy of the estimates
    unsigned long long *slots;      // [2 * n_expert] all ones before the first call (every call leaves them so)
    float *act;                     // [n_used * n_ff]
    int32_t *spec_ids;              // [n_used]
    int32_t *ids_out;
    float *w_out;
    int *stats;                     // [4]
    int k, n_expert, n_used, n_ff;
    int nseq = 1;  // a batch: every per-token array holds nseq rows (moe_decode.hip for_seq)
    // Optional fused FFN norm: when norm_w is set, x = rms_norm(norm_a + norm_b) * norm_w is
    // formed inside launch 1 (x is then unused), norm_a + norm_b is written to norm_sum for
    // launch 2's residual (res must point at norm_sum). One sequence only.
    const float *norm_a = nullptr, *norm_b = nullptr, *norm_w = nullptr;
    float norm_eps = 0.0f;
    float *norm_sum = nullptr;
    // Loads a wait on another workgroup of launch 1 makes before it computes
    // the awaited router logit itself (bit-identical either way). 0 forces
    // that path on every wait; tests use it.
    int polls = 1 << 18;
};
int launch_moe_decode(const MoeDecodeLaunch &l, hipStream_t st);
// The decode step's FFN block with its norm (model.cpp): sum_out = x + o;
// out = sum_out + moe(rms_norm(sum_out) * w). Only for layers where
// moe_normed_applies() holds (decided once, at model create); -1 is an error.
bool moe_normed_applies(void *moe);
// The layer's router matrix on the device ([n_expert][n_embd] f32) and its row count.
const float *moe_router(void *moe);
int moe_router_rows(void *moe);
int moe_forward_normed(void *moe, const float *x, const float *o, const float *w, float eps,
                       float *sum_out, float *out);
int launch_q6k_mv_batched(const void *w, size_t expert_stride, const int32_t *grp_expert,
                          const int32_t *grp_start, const int32_t *grp_count,
                          const int32_t *sub_start, const int32_t *pair_out, const int8_t *act_q,
                          const float *act_d, float *y, int ldy, int rows, int blocks,
                          int n_groups, int max_chunks, hipStream_t st, float *amax_v = nullptr,
                          int *amax_i = nullptr, bool group_tables = false,
                          const void *w2 = nullptr, float *y2 = nullptr, bool fast = false);
// Grouped (grp_expert set): sub_start holds 2 * (n_groups + 1) entries, the
// chunk prefix sub_start[0..n_groups] and the twin prefix after it
// (launch_moe_group's layout); group_tables: the GroupItem records follow
// (written with the same max_chunks). act_q / act_d: the token-chunked
// activations (q8k_wave.hpp). w2 / y2: a second matrix of the same shape on
// the same activations, in the same launch. fast: the REDUCTION-tolerance
// kernels (one float accumulator per output instead of the reference's eight
// class sums; outputs within REDUCTION of dot_q6k_q8k, not bit-identical).
// Up to three matrices with their own row counts (Q, K, V) against the same
// nseq token-chunked activations, one launch: y[i] [nseq][rows[i]].
int launch_q6k_mv_batched_x3(const void *const w[3], float *const y[3], const int rows[3], int n_mat,
                             const int8_t *act_q, const float *act_d, int blocks, int nseq,
                             hipStream_t st);
int launch_q6k_dequant(const void *w, int rows, int blocks, float *out, hipStream_t st);
// Per 16-row tile t of a tiled Q6_K matrix: mt[t] = the largest over its rows
// of sum_b |f16(d_b)| * sum_e |sc(e) * (q_e - 32)| (an upper bound of the
// row's sum of |dequantized weight| products' scale, for the arg-max
// certificate below).
int launch_q6k_tile_bound(const void *w, int rows, int blocks, float *mt, hipStream_t st);
// The LM head's certified arg-max over REDUCTION-tolerance logits (the fast
// batched kernel's per-(token, tile) candidates pv / pi, pi < 0 marking a tile
// with a NaN logit): per token, every tile whose candidate can reach the
// largest certified lower bound is recomputed exactly (dot_q6k_q8k's bits,
// written back into logits), and ids = the reference's arg-max of the exact
// logits. nq / nd: the tokens' Q8_K in the natural layout.
// y[rows] = W (tiled Q6_K, blocks <= 16) . Q8_K(x), x f32 [blocks * 256]: the
// bits of launch_q8k_quantize + launch_q6k_mv_b1 in one launch
int launch_q6k_mv_f32x(const void *w, const float *x, float *y, int rows, int blocks,
                       hipStream_t st);
int launch_lmhead_certify(const void *w, int rows, int blocks, int nseq, const int8_t *nq,
                          const float *nd, const float *pv, const int *pi, const float *mt,
                          float *logits, int32_t *ids, hipStream_t st);

// q8k.hip
int launch_q8k_quantize(const float *x, int8_t *qs, float *d, int16_t *bsums, int nblocks,
                        hipStream_t st);
// rows of x to the token-chunked layout, each row to `fan` slots slot_of[r*fan+k]
// (slot_of == nullptr: row r to slot r)
// (nq, nd: optionally also the natural layout, row r at nq[r * blocks * 256], nd[r * blocks])
int launch_q8k_quantize_chunks(const float *x, int rows, int blocks, const int32_t *slot_of,
                               int fan, int8_t *cq, float *cd, hipStream_t st,
                               int8_t *nq = nullptr, float *nd = nullptr);
int launch_swiglu_q8k(const float *gate, const float *up, float *act_out, int8_t *qs, float *d,
                      int16_t *bsums, int nblocks, hipStream_t st);
int launch_swiglu_q8k_chunks(const float *gate, const float *up, int rows, int blocks,
                             const int32_t *slot_of, int8_t *cq, float *cd, hipStream_t st);
// moe grouping (group.hip): counting sort of the (token, k) pairs by expert.
// Outputs grp_* per expert, sub_start (prefix of ceil(count/16), then the
// twin prefix of ceil(chunks/2): 2 * (n_expert + 1) entries; with
// max_chunks > 0 then a GroupItem per chunk and per twin, from
// group_items_offset(n_expert), 2 * max_chunks records), for each
// pair p = token * n_used + k its chunk slot slot_of_pair[p], and for each
// sorted position its pair index pair_idx.
// One work item of the expert-grouped batched kernels: a 16-token chunk, or a
// twin (two consecutive chunks of one expert), with its group's fields.
struct __attribute__((aligned(32))) GroupItem {
    int32_t expert;  // = its group
    int32_t st;      // first chunk's index within the group
    int32_t sub;     // first chunk's global index (its activation chunk)
    int32_t count;   // pairs in the group
    int32_t start;   // the group's first sorted pair
    int32_t twin2;   // twins: 1 when the second chunk exists
    int32_t pad0, pad1;
};
// The records start at this int32 offset of sub_start (32-byte aligned
// when sub_start is).
constexpr size_t group_items_offset(int n_expert) { return ((2 * (size_t)(n_expert + 1)) + 7) & ~(size_t)7; }
int launch_moe_group(const int32_t *ids, int n_pairs, int n_used, int n_expert,
                     int32_t *grp_expert, int32_t *grp_start, int32_t *grp_count,
                     int32_t *sub_start, int32_t *slot_of_pair, int32_t *pair_idx,
                     hipStream_t st, int max_chunks = 0);
int launch_silu_mul(const float *gate, const float *up, float *out, int n, hipStream_t st);

// norm.hip: CpuBackend::rms_norm (+ weight), bit-exact. rows of n; the
// weight repeats every w_len elements (per-head QK norm: w_len = n = hd).
int launch_rms_norm_mul(const float *x, const float *w, float *out, int rows, int n, int w_len,
                        float eps, hipStream_t st);
// rms_norm(x) * w, then Q8_K (qs, d natural layout); out and inv_out optional.
// rows > 1: rows of n each ([rows][n] x / out / qs, [rows][n/256] d, [rows] inv_out).
// RMSNorm -> Q8_K -> the Q, K and V matvecs in one launch (norm.hip): y[i] =
// W[i] (tiled Q6_K, rows[i] rows) . quantize_q8_k(rms_norm(x) * w), the bits of
// launch_rms_norm_quant followed by the exact matvecs. n <= 2048.
bool norm_qkv_fits(int n, const int rows[3]);
int launch_norm_qkv(const float *x, const float *w, float eps, const void *const wt[3],
                    float *const y[3], const int rows[3], int n, hipStream_t st);
int launch_rms_norm_quant(const float *x, const float *w, float *out, int8_t *qs, float *d,
                          float *inv_out, int n, float eps, hipStream_t st, int rows = 1);

// decode.hip: the whole-token step around the matvecs (token / position read
// from device memory)
// nseq rows: sequence s embeds token tok[s * tok_stride] (tok null: tok_fixed)
int launch_embed_q6k(const void *table, const int32_t *tok, int blocks, float *out, hipStream_t st,
                     int nseq = 1, int tok_stride = 0, int tok_fixed = 0);
int attend_max_kv();
bool attend_fused_fits(int n_head, int n_head_kv, int hd, int max_kv);
// raises attend_fused's dynamic LDS limit for max_kv positions (outside graph capture)
int attend_fused_prepare(int n_head, int n_head_kv, int hd, int max_kv);
int launch_attend_fused(const float *q, const float *k, const float *v, const float *qw,
                        const float *kw, const float2 *cs, const int32_t *pos, int n_head,
                        int n_head_kv, int hd, float eps, float scale, int max_kv, float *kc,
                        float *vc, int8_t *oq, float *od, float *out, hipStream_t st,
                        const void *pf0 = nullptr, size_t b0 = 0, int n0 = 0,
                        const void *pf1 = nullptr, size_t b1 = 0, int n1 = 0);
// (pf0 / pf1: n0 + n1 extra workgroups read b0 (b1) bytes each from pf0 + i * b0
// (pf1 + i * b1) into the L2 of XCD i % 8, where workgroup i of the later launch that
// reads them runs; needs n_head / 2 and n0 to be multiples of 8, else skipped)
// Attention over long contexts in two launches (after launch_qk_norm_rope_store):
// logits spread over 256 workgroups, then the softmax (exact in-order sum)
// and the in-order weighted V sum (two workgroups per head) into out
// [n_head * hd], and its Q8_K; the bits of launch_attend_fused. scores:
// [n_head][max_kv] floats.
bool attend_split_fits(int n_head, int n_head_kv, int hd, int max_kv);
// raises attend_finish's dynamic LDS limit for max_kv positions (outside graph capture)
int attend_split_prepare(int n_head, int n_head_kv, int hd, int max_kv);
int launch_attend_split(const float *q, const float *kc, const float *vc, const int32_t *pos,
                        int n_head, int n_head_kv, int hd, float scale, int max_kv, float *scores,
                        int8_t *oq, float *od, float *out, hipStream_t st);
// nseq sequences: n_kv = pos[s * pos_stride] + 1 (pos null: n_kv_fixed); q, out
// [nseq][n_head * hd]; sequence s's cache starts cache_seq_stride floats after s-1's.
int launch_attend_decode(const float *q, const float *kc, const float *vc, const int32_t *pos,
                         int n_head, int n_head_kv, int hd, float scale, float *out,
                         hipStream_t st, int nseq = 1, int n_kv_fixed = 0, int pos_stride = 0,
                         size_t cache_seq_stride = 0);

// norm.hip, decode step: per-head QK-norm (w null: none) + RoPE, Q in place,
// K and V into the cache row of *pos; and ffn_inp = x + o, out = rms_norm(ffn_inp) * w.
int launch_qk_norm_rope_store(float *q, const float *k, const float *v, const float *qw,
                              const float *kw, const float2 *cs, const int32_t *pos, int n_head,
                              int n_head_kv, int hd, float eps, float *kc, float *vc,
                              hipStream_t st);
int launch_add_rms_norm_mul(const float *x, const float *o, const float *w, float *sum_out,
                            float *out, int n, float eps, hipStream_t st);

// moe.hip
// The reference's router logits (sequential f32 fold per expert) and, in the
// same launch, Q8_K of x for the expert matvecs. k % 256 == 0, k <= 2048.
int launch_copy_calibration(void *dst, const void *src, size_t bytes, hipStream_t st);
int launch_read_calibration(const void *src, size_t bytes, int grid, hipStream_t st);
struct RouterLaunch {
    const float *w, *x;
    int n_expert, k;
    float *logits;
    int8_t *xq;
    float *xd;
    int xblocks;
    int nseq = 1;  // x [nseq][k] -> logits [nseq][n_expert]; xblocks only with nseq = 1
};
int launch_router(const RouterLaunch &l, hipStream_t st);
// y [nseq][rows] = w [rows][k] . x [nseq][k], each row's sum the reference's
// sequential f32 fold (model.rs:253-262: products rounded, added in order
// from -0.0) in one launch for every sequence; k outside the fold kernel's
// range (a multiple of 256 up to 2048) falls back to the FMA matvec
// (REDUCTION), one launch per sequence.
int launch_matvec_f32_exact(const float *w, const float *x, float *y, int rows, int k, int nseq,
                            hipStream_t st);
// nseq sequences: logits [nseq][n_expert] -> ids, weights [nseq][n_used];
// probs (optional): the softmax over every expert, [nseq][n_expert]
int launch_route_logits(const float *logits, int n_expert, int n_used, int32_t *ids,
                        float *weights, hipStream_t st, int nseq = 1, float *probs = nullptr);
// out[t] = res[t] + sum_e weights[t][e] * down[t][e] in e order; with skip,
// pairs whose skip entry is negative add nothing.
int launch_moe_combine(const float *down, const float *weights, const float *res, float *out,
                       int n_used, int n_embd, int n_tok, hipStream_t st,
                       const int32_t *skip = nullptr);
int argmax_parts(int n);
// Reduce nparts (value, index) candidates per sequence ([nseq][nparts]) to the
// reference's arg-max of row x[seq * ld ..] (index 0 wins if x[0] is NaN).
int launch_argmax_final(const float *x, int ld, int nseq, const float *pv, const int *pi,
                        int nparts, int32_t *out, hipStream_t st);
// pv, pi hold [nseq][parts] candidates, parts = argmax_parts(n) capped at
// max_parts (> 0)
int launch_argmax(const float *x, int n, int ld, int nseq, float *pv, int *pi, int32_t *out,
                  hipStream_t st, int max_parts = 0);
int launch_q8_0_mv(const void *planar, const float *x, float *y, int rows, int k, hipStream_t st);
int launch_q8_0_dequant(const void *planar, int rows, int k, float *out, hipStream_t st);
int launch_f32_mv(const float *w, const float *x, float *y, int rows, int k, hipStream_t st);

// compat.hip: the reference's own weight layouts and operand forms.
// A Q6_K tensor in device memory as the reference lays it out: byte j of
// field f (ql 128 B, qh 64 B, sc 16 B, d 2 B) of block i = row * blocks + b
// at base + off[f] + i * stride[f] + j. ggml blocks: off = {0, 128, 192, 208},
// stride 210; the planar repack: off = the plane offsets, stride = field size.
struct Q6kSource {
    const uint8_t *base;
    size_t off[4];
    size_t stride[4];
};
// Gather rows x blocks of a Q6kSource into the tiled layout
// (llamd_hip_q6k_tiled_bytes(rows, blocks) bytes at tiled).
int launch_q6k_retile(const Q6kSource &s, int rows, int blocks, void *tiled, hipStream_t st);
// memset as a kernel (capturable, no memset graph node)
int launch_fill(void *p, int value, size_t bytes, hipStream_t st);
// Q8_K quants [n_act][blocks*256], signed or biased (q ^ 0x80) -> signed copy
int launch_act_unbias(const void *q, bool biased, int n_act, int blocks, int8_t *out,
                      hipStream_t st);
// natural [n_act] quants + scales -> token-chunked operand layout (zero past n_act)
int launch_act_to_chunks(const void *q, const float *d, bool biased, int n_act, int blocks,
                         int8_t *cq, float *cd, hipStream_t st);
// signed quants -> biased quants (may be the same memory) + per-16 sums of them
int launch_bias_sums(const int8_t *qs, uint8_t *qb, int32_t *sb, int nblocks, hipStream_t st);
// Per-head QK-norm (w optional) + NeoX RoPE in place, with a position per
// sequence; optionally stores the rotated head (and v) into a KV cache.
struct HeadRopeArgs {
    float *x;                 // [nseq][n_heads][hd]
    const float *w;           // [hd] or null
    float eps;
    const float2 *cs;         // [cs_rows][hd / 2] (cos, sin)
    int cs_rows;
    const float *den;         // [hd / 2] base^(2i/hd) (the table's): positions
                              // at or past cs_rows are rotated on the device
    const int32_t *pos_p;     // pos of sequence s at pos_p[s * pos_stride]
    int pos_stride;
    int pos_fixed;            // without pos_p: this position (< 0: pos = s)
    int n_heads, hd;
    float *kc, *vc;           // null: no store
    int cache_rows;           // positions the cache slice holds (no store at or past it)
    const float *v;           // [nseq][n_heads][hd] with kc
    int kv_dim;               // n_heads * hd
    size_t cache_seq_stride;  // floats between sequences' cache slices
};
int launch_head_norm_rope(const HeadRopeArgs &a, int nseq, hipStream_t st);
int launch_kv_store(float *kc, float *vc, const float *k, const float *v, int pos, int kv_dim,
                    hipStream_t st);
enum { EW_ADD = 0, EW_MUL = 1, EW_SCALE = 2, EW_SILU = 3 };
int launch_ew(int op, const float *a, const float *b, float by, float *o, size_t n,
              hipStream_t st);
int launch_softmax_rows(const float *x, float *o, int rows, int n, hipStream_t st);
// out [n][m] = w [m][k] . x [n][k], each sum in order (CpuBackend::matmul)
int launch_matmul_f32_seq(const float *w, const float *x, float *out, int m, int n, int k,
                          hipStream_t st);

// ---- shared by the C ABI's host files ----
// The library's stream (capi.cpp).
hipStream_t lib_stream();
// A void device-pointer entry point refused its arguments (the text is in
// llamd_hip_last_error); llamd_fwd_last_error reports it once (capi.cpp).
void fwd_refused();
// A Q6_K weight as the kernels read it: the tiled layout, experts
// expert_stride bytes apart (capi.cpp resolve_q6k).
struct Q6kView {
    const void *tiled;
    size_t expert_stride;
    int n_expert;
};
int resolve_q6k(const void *w, const size_t *planar_off, int rows, int blocks, bool grouped,
                Q6kView *v);
// compat_abi.cpp: device memory the library handed out, and the tiled copies of
// Q6_K tensors that live in it in the reference's layouts (ggml blocks when
// planar_off is null, else the planar repack with plane offsets planar_off).
// shadow_q6k gives the copy (made on first use) and the row count it holds.
void note_alloc(void *p, size_t bytes);
void note_free(void *p);
// after a write of [p, p + bytes) queued on st: re-make the copies of what it touched
int note_write(const void *p, size_t bytes, hipStream_t st);
int shadow_q6k(const void *w, const size_t *planar_off, int rows, int blocks, const void **tiled,
               int *rows_total);
// Shape of a tiled Q6_K handle from llamd_rocm_upload_q6k[_experts]; -1 if p
// is not one.
int q6k_handle_shape(const void *p, int *rows, int *blocks, int *n_expert);
// Device scratch of one LM-head call (capi.cpp lmhead_enqueue): Q8_K of x
// (nseq == 1: xq [blocks*256], xd [blocks]; nseq > 1: the token-chunked cq,
// cd of lmhead_chunk_*_bytes) and the per-tile arg-max candidates pv, pi
// [nseq][ceil(rows/16)].
struct LmHeadScratch {
    int8_t *xq;
    float *xd;
    int8_t *cq;
    float *cd;
    float *pv;
    int *pi;
    // non-null: REDUCTION-tolerance logits with a certified exact arg-max
    // (nseq > 1; mt from launch_q6k_tile_bound)
    const float *mt = nullptr;
};
size_t lmhead_chunk_q_bytes(int nseq, int blocks);
size_t lmhead_chunk_d_bytes(int nseq, int blocks);
int lmhead_enqueue(const void *w, int rows, int blocks, const float *d_x, int nseq,
                   float *d_logits, int32_t *d_ids, const LmHeadScratch &sc);
// One sequence whose activation is already Q8_K (xq [blocks*256], xd
// [blocks]) through an LM-head handle: matvec + arg-max.
int lmhead_forward_q8k(void *h, const int8_t *xq, const float *xd, float *d_logits, int32_t *d_ids);

}  // namespace llamd
