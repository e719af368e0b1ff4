/*
 * llamd_oracle.h -- CPU restatement of llamd.rs's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity oracle for the HIP
 * kernels in llamd_rs_amd/ and the CPU baseline that bench.py times beside
 * them. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker -- never as the thing measured on the
 * GPU path, never as a fallback.
 *
 * Every function restates one Rust function of the reference and cites it
 * (paths relative to the reference checkout). The reference is Rust; no Rust
 * toolchain exists in this image, so the reference cannot be built and this
 * C restatement is checked instead against the reference's own in-source
 * known-answer tests plus closed-form and brute-force properties (see
 * tests/test_oracle_*.py).
 *
 * Floating-point discipline, matching rustc's defaults:
 *   - compiled with -O2 -ffp-contract=off, no fast-math: Rust neither
 *     contracts a*b+c into an FMA nor reassociates;
 *   - f32::exp is glibc expf (linux-gnu), used here directly;
 *   - round_ties_even is nearbyintf under FE_TONEAREST;
 *   - an f32 `.iter().sum()` folds left to right starting at -0.0.
 *
 * Parity status per function is recorded in the header comment of
 * llamd_oracle.c.
 */
#ifndef LLAMD_ORACLE_H
#define LLAMD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_QK8_0 32
#define ORC_Q6K_BLOCK_BYTES 210
#define ORC_Q8_0_BLOCK_BYTES 34
#define ORC_Q8K_BLOCK_BYTES 292
#define ORC_WEIGHT_SUM_FLOOR 6.103515625e-5f

/* R4: binary16 -> binary32 (crates/llamd-quant/src/lib.rs:104-108). */
float orc_f16_to_f32(uint16_t h);

/* ggml element/byte accounting (crates/llamd-quant/src/lib.rs:72-101).
 * type: 0=F32 1=F16 8=Q8_0 14=Q6K. Returns bytes, or -1 when n is not a
 * whole number of blocks or the type is unknown. */
long long orc_bytes_for(uint32_t type, size_t n);

/* R2/R3: dequantize (crates/llamd-quant/src/lib.rs:116-226).
 * Returns 0, or -1 when src_len is short or n is not whole blocks. */
int orc_dequantize(uint32_t type, const uint8_t *src, size_t src_len, size_t n, float *out);

/* R5: ggml nearest_int and quantize_q8_k (crates/llamd-quant/src/dot.rs:80-128).
 * n must be a multiple of 256; writes n/256 blocks. */
int32_t orc_nearest_int(float v);
int orc_quantize_q8_k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums);

/* R6: Q6_K x Q8_K dot product (crates/llamd-quant/src/dot.rs:138-196). */
float orc_dot_q6k_q8k(const uint8_t *w, const float *ad, const int8_t *aq, size_t n);

/* R7 given an already-quantized activation: rows independent dot products
 * (crates/llamd-models/src/model.rs:265-275). */
void orc_matvec_q6k_act(const uint8_t *w, size_t rows, size_t k, const float *ad,
                        const int8_t *aq, float *y);

/* R7: Model::matvec_quant, Q6_K branch: quantize x then dot every row
 * (crates/llamd-models/src/model.rs:241-276). */
int orc_matvec_q6k(const uint8_t *w, size_t rows, size_t k, const float *x, float *y);
/* orc_matvec_q6k_act over nthreads host threads (same bits); returns the threads used */
int orc_matvec_q6k_act_mt(const uint8_t *w, size_t rows, size_t k, const float *ad,
                          const int8_t *aq, float *y, int nthreads);

/* R8: Model::matvec_quant fallback for F32 weights: sequential f32 sum
 * (crates/llamd-models/src/model.rs:253-262). */
void orc_matvec_f32(const float *w, size_t rows, size_t k, const float *x, float *y);

/* R8 for Q8_0: dequantize every row then the same sequential f32 sum
 * (crates/llamd-models/src/model.rs:253-262 with lib.rs:154-162). */
int orc_matvec_q8_0(const uint8_t *w, size_t rows, size_t k, const float *x, float *y);

/* R9: route (crates/llamd-models/src/moe.rs:73-113). Returns -1 when
 * n_used == 0 or n_used > n_expert. Any output pointer may be NULL. */
int orc_route(const float *logits, size_t n_expert, size_t n_used, uint32_t *experts,
              float *weights_raw, float *weight_sum, float *weights);

/* CpuBackend::silu / mul / softmax (crates/llamd-cpu/src/lib.rs:81-113). */
void orc_silu(const float *x, float *y, size_t n);
void orc_rms_norm(const float *x, int rows, int n, float eps, float *out);
void orc_mul(const float *a, const float *b, float *y, size_t n);
void orc_softmax(const float *x, float *y, size_t n);

/* R10: matvec_expert_quant over one expert of a 3D Q6_K tensor laid out
 * [k, rows, n_expert] with the expert on the slowest axis
 * (crates/llamd-models/src/model.rs:188-227, 279-318). */
int orc_matvec_expert_q6k(const uint8_t *w, size_t n_expert, size_t rows, size_t k,
                          size_t expert, const float *x, float *y);

/* R11: moe_ffn (crates/llamd-runtime/src/layer.rs:230-260).
 * gate/up: [n_ff x n_embd] per expert, down: [n_embd x n_ff] per expert. */
int orc_moe_ffn(const float *x, size_t n_embd, size_t n_ff, size_t n_expert,
                const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                const uint32_t *experts, const float *weights, size_t n_used, float *out);

/* One MoE decode layer as the reference composes it: router logits through
 * R8, R9 route, R11 moe_ffn, R12 residual (layer.rs:281-287):
 * out = x_res + moe_ffn(x). Optional outputs (may be NULL): logits, ids,
 * weights. */
int orc_moe_layer(const float *x, const float *x_res, size_t n_embd, size_t n_ff,
                  size_t n_expert, size_t n_used, const float *router,
                  const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                  float *out, float *logits, uint32_t *ids, float *weights);

/* R13: argmax with strict '>' -- lowest index wins ties
 * (crates/llamd-testing/tests/device_forward.rs:23-37). */
uint32_t orc_argmax(const float *v, size_t n);

/* R14, token-major: the expert-grouped prefill computes, for every token, the
 * same moe_ffn as decode (crates/llamd-testing/tests/vulkan_prefill.rs:268-333
 * holds expert-major == token-major). Routing is given (ids/weights per
 * token), out is [n_tok x n_embd]. */
int orc_moe_ffn_tokens(const float *x, size_t n_tok, size_t n_embd, size_t n_ff,
                       size_t n_expert, const uint8_t *gate, const uint8_t *up,
                       const uint8_t *down, const uint32_t *ids, const float *weights,
                       size_t n_used, float *out);

/* tolerance.rs:116-151 */
int orc_close(float a, float b, float tol);

/* CpuBackend::rope, in place (llamd-cpu/src/lib.rs:158-209) */
void orc_rope(float *x, int heads, int hd, uint32_t pos, float base);
/* attend (llamd-runtime/src/attention.rs:73-125) */
int orc_attend(const float *q, const float *k, const float *v, int n_kv, int n_head,
               int n_head_kv, int hd, float *out);

#ifdef __cplusplus
}
#endif
#endif
