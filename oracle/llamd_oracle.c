/*
 * llamd_oracle.c -- CPU restatement of llamd.rs's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see llamd_oracle.h). Not linked into, loaded by or
 * called from the product library; the GPU path fails loudly without its HIP
 * extension instead of falling back here.
 *
 * Parity status (how each function is pinned, see tests/test_oracle_*.py):
 *   orc_f16_to_f32        exhaustive over all 65536 codes vs numpy float16
 *   orc_dequantize        reference known answers (lib.rs:235-323) + single-
 *                         element probes of every Q6_K position
 *   orc_quantize_q8_k     reference known answers (dot.rs:209-255,
 *                         grouped_expert.rs:235-240) + reconstruction bound
 *   orc_dot_q6k_q8k       reference known answers (dot.rs:284-346), single-
 *                         element brute force at every position, float64
 *                         dequant-product bound
 *   orc_matvec_*          composition of the above + float64 bound
 *   orc_route             reference known answers (moe.rs:120-246)
 *   orc_silu/mul/softmax  closed form (float64) within 1 ulp
 *   orc_rms_norm          reference known answers (llamd-cpu lib.rs:237-259),
 *                         order probes of the sequential sum, float64 bound
 *   orc_moe_ffn/_layer    composition; float64 restatement bound
 *   orc_argmax            closed form incl. ties
 *   orc_moe_ffn_tokens    composition of orc_moe_ffn per token
 *   orc_rope              reference known answers (llamd-cpu lib.rs:313-357:
 *                         position 0 identity, pairs across the half boundary,
 *                         pair norms kept) + float64 rotation bound
 *   orc_attend            reference known answers (attention.rs tests: one
 *                         position returns v, convex combination, GQA by
 *                         integer division, scale 1/sqrt(hd), no overflow) +
 *                         float64 restatement bound
 * Nothing here is "parity unpinned"; the Q6_K/Q8_0 weight QUANTIZERS (input
 * generators, not part of the reference) live with the synthetic-data code.
 */
#include <omp.h>
#include "llamd_oracle.h"

#include <fenv.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QK_K ORC_QK_K
#define QK8_0 ORC_QK8_0
#define Q6K_BB ORC_Q6K_BLOCK_BYTES
#define Q8_0_BB ORC_Q8_0_BLOCK_BYTES

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 -> binary32, exact for every code including subnormals,
 * infinities and NaN (quieted, payload kept), as half 2.7.1's to_f32 does.
 * crates/llamd-quant/src/lib.rs:104-108 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1F) {
        if (man == 0) return u2f(sign | 0x7F800000u);
        return u2f(sign | 0x7FC00000u | (man << 13));
    }
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: value = man * 2^-24, exactly representable */
        int e = -1;
        do { man <<= 1; e++; } while ((man & 0x400u) == 0);
        man &= 0x3FFu;
        return u2f(sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13));
    }
    return u2f(sign | ((exp + 127 - 15) << 23) | (man << 13));
}

static inline uint16_t rd_u16(const uint8_t *b) { return (uint16_t)(b[0] | (b[1] << 8)); }

/* crates/llamd-quant/src/lib.rs:72-101 (block_elems, block_bytes, bytes_for) */
long long orc_bytes_for(uint32_t type, size_t n) {
    size_t be, bb;
    switch (type) {
    case 0: be = 1; bb = 4; break;
    case 1: be = 1; bb = 2; break;
    case 8: be = QK8_0; bb = Q8_0_BB; break;
    case 14: be = QK_K; bb = Q6K_BB; break;
    default: return -1;
    }
    if (n % be) return -1;
    return (long long)(n / be * bb);
}

/* dequantize_q8_0: crates/llamd-quant/src/lib.rs:154-162 */
static void deq_q8_0(const uint8_t *src, size_t n, float *out) {
    for (size_t b = 0; b < n / QK8_0; ++b) {
        const uint8_t *blk = src + b * Q8_0_BB;
        float d = orc_f16_to_f32(rd_u16(blk));
        for (int j = 0; j < QK8_0; ++j) out[b * QK8_0 + j] = d * (float)(int8_t)blk[2 + j];
    }
}

/* dequantize_q6_k: crates/llamd-quant/src/lib.rs:181-226. Same two-halves
 * walk; the product is d * sc first, then * q, left to right as in Rust. */
static void deq_q6_k(const uint8_t *src, size_t n, float *out) {
    const int QL = 0, QH = QK_K / 2, SC = QK_K / 2 + QK_K / 4, D = SC + QK_K / 16;
    for (size_t b = 0; b < n / QK_K; ++b) {
        const uint8_t *blk = src + b * Q6K_BB;
        float d = orc_f16_to_f32(rd_u16(blk + D));
        float *y0 = out + b * QK_K;
        for (int half = 0; half < 2; ++half) {
            int ql = QL + half * 64, qh = QH + half * 32, sc = SC + half * 8;
            float *y = y0 + half * 128;
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                uint8_t h = blk[qh + l], lo0 = blk[ql + l], lo1 = blk[ql + l + 32];
                int8_t q1 = (int8_t)((lo0 & 0x0F) | ((h >> 0) & 3) << 4) - 32;
                int8_t q2 = (int8_t)((lo1 & 0x0F) | ((h >> 2) & 3) << 4) - 32;
                int8_t q3 = (int8_t)((lo0 >> 4) | ((h >> 4) & 3) << 4) - 32;
                int8_t q4 = (int8_t)((lo1 >> 4) | ((h >> 6) & 3) << 4) - 32;
                y[l] = d * (float)(int8_t)blk[sc + is] * (float)q1;
                y[l + 32] = d * (float)(int8_t)blk[sc + is + 2] * (float)q2;
                y[l + 64] = d * (float)(int8_t)blk[sc + is + 4] * (float)q3;
                y[l + 96] = d * (float)(int8_t)blk[sc + is + 6] * (float)q4;
            }
        }
    }
}

/* dequantize: crates/llamd-quant/src/lib.rs:116-149 */
int orc_dequantize(uint32_t type, const uint8_t *src, size_t src_len, size_t n, float *out) {
    long long need = orc_bytes_for(type, n);
    if (need < 0 || (long long)src_len < need) return -1;
    switch (type) {
    case 0:
        for (size_t i = 0; i < n; ++i) memcpy(&out[i], src + 4 * i, 4);
        break;
    case 1:
        for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(rd_u16(src + 2 * i));
        break;
    case 8: deq_q8_0(src, n, out); break;
    case 14: deq_q6_k(src, n, out); break;
    default: return -1;
    }
    return 0;
}

/* nearest_int: crates/llamd-quant/src/dot.rs:80-86 (round_ties_even). */
int32_t orc_nearest_int(float v) {
    /* the oracle library never changes the rounding mode; nearbyintf rounds
     * in the current mode, which is FE_TONEAREST (ties to even). */
    return (int32_t)nearbyintf(v);
}

/* quantize_q8_k: crates/llamd-quant/src/dot.rs:89-128 */
int orc_quantize_q8_k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums) {
    if (n % QK_K) return -1;
    for (size_t b = 0; b < n / QK_K; ++b) {
        const float *c = x + b * QK_K;
        int8_t *q = qs + b * QK_K;
        int16_t *bs = bsums + b * (QK_K / 16);
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < QK_K; ++i) {
            float a = fabsf(c[i]);
            if (a > amax) { amax = a; max = c[i]; }
        }
        if (amax == 0.0f) {
            d[b] = 0.0f;
            memset(q, 0, QK_K);
            memset(bs, 0, sizeof(int16_t) * (QK_K / 16));
            continue;
        }
        float iscale = -127.0f / max;
        for (int i = 0; i < QK_K; ++i) {
            int32_t v = orc_nearest_int(iscale * c[i]);
            q[i] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < QK_K / 16; ++g) {
            int16_t s = 0;
            for (int j = 0; j < 16; ++j) s = (int16_t)(s + q[g * 16 + j]);
            bs[g] = s;
        }
        d[b] = 1.0f / iscale;
    }
    return 0;
}

/* dot_q6k_q8k: crates/llamd-quant/src/dot.rs:138-196. Integer per-lane
 * accumulation (8 lanes = element index mod 8), then the ordered f32 epilogue
 * sums[l] += d * aux32[l] (no FMA), then the lanes summed in order. */
float orc_dot_q6k_q8k(const uint8_t *w, const float *ad, const int8_t *aq, size_t n) {
    const int QL = 0, QH = QK_K / 2, SC = QK_K / 2 + QK_K / 4, D = SC + QK_K / 16;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t i = 0; i < n / QK_K; ++i) {
        const uint8_t *blk = w + i * Q6K_BB;
        const int8_t *yq = aq + i * QK_K;
        int8_t aux8[QK_K];
        for (int half = 0; half < 2; ++half) {
            int ql = QL + half * 64, qh = QH + half * 32, o = half * 128;
            for (int l = 0; l < 32; ++l) {
                uint8_t h = blk[qh + l], lo0 = blk[ql + l], lo1 = blk[ql + l + 32];
                aux8[o + l] = (int8_t)((lo0 & 0x0F) | (h & 3) << 4) - 32;
                aux8[o + l + 32] = (int8_t)((lo1 & 0x0F) | ((h >> 2) & 3) << 4) - 32;
                aux8[o + l + 64] = (int8_t)((lo0 >> 4) | ((h >> 4) & 3) << 4) - 32;
                aux8[o + l + 96] = (int8_t)((lo1 >> 4) | ((h >> 6) & 3) << 4) - 32;
            }
        }
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < QK_K / 16; ++j) {
            int32_t scale = (int8_t)blk[SC + j];
            for (int half = 0; half < 2; ++half) {
                int o = j * 16 + half * 8;
                for (int l = 0; l < 8; ++l) {
                    int16_t p = (int16_t)((int16_t)yq[o + l] * (int16_t)aux8[o + l]);
                    aux32[l] += scale * (int32_t)p;
                }
            }
        }
        float dd = orc_f16_to_f32(rd_u16(blk + D)) * ad[i];
        for (int l = 0; l < 8; ++l) sums[l] += dd * (float)aux32[l];
    }
    float s = -0.0f;
    for (int l = 0; l < 8; ++l) s += sums[l];
    return s;
}

/* model.rs:265-275: rows independent dots against one quantized activation */
void orc_matvec_q6k_act(const uint8_t *w, size_t rows, size_t k, const float *ad,
                        const int8_t *aq, float *y) {
    size_t rb = k / QK_K * Q6K_BB;
    for (size_t r = 0; r < rows; ++r) y[r] = orc_dot_q6k_q8k(w + r * rb, ad, aq, k);
}

/* orc_matvec_q6k_act with the rows split over nthreads host threads (one
 * OpenMP team, kept by the runtime between calls). Rows are independent, so
 * the result is the same bits; only the CPU baseline's all-core figure uses
 * it. Returns the team size. */
int orc_matvec_q6k_act_mt(const uint8_t *w, size_t rows, size_t k, const float *ad,
                          const int8_t *aq, float *y, int nthreads) {
    size_t rb = k / QK_K * Q6K_BB;
    int used = 1;
#pragma omp parallel num_threads(nthreads)
    {
#pragma omp single
        used = omp_get_num_threads();
#pragma omp for schedule(static)
        for (long r = 0; r < (long)rows; ++r)
            y[r] = orc_dot_q6k_q8k(w + (size_t)r * rb, ad, aq, k);
    }
    return used;
}

/* Model::matvec_quant, Q6_K branch: crates/llamd-models/src/model.rs:241-276 */
int orc_matvec_q6k(const uint8_t *w, size_t rows, size_t k, const float *x, float *y) {
    if (k % QK_K) return -1;
    size_t nb = k / QK_K;
    float *ad = (float *)malloc(nb * sizeof(float));
    int8_t *aq = (int8_t *)malloc(k);
    int16_t *bs = (int16_t *)malloc(nb * 16 * sizeof(int16_t));
    if (!ad || !aq || !bs) { free(ad); free(aq); free(bs); return -1; }
    orc_quantize_q8_k(x, k, ad, aq, bs);
    orc_matvec_q6k_act(w, rows, k, ad, aq, y);
    free(ad); free(aq); free(bs);
    return 0;
}

/* Model::matvec_quant fallback: crates/llamd-models/src/model.rs:253-262.
 * row.iter().zip(x).map(|(a, b)| a * b).sum() -- products rounded, then a
 * sequential fold from -0.0. */
void orc_matvec_f32(const float *w, size_t rows, size_t k, const float *x, float *y) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = w + r * k;
        float s = -0.0f;
        for (size_t t = 0; t < k; ++t) {
            float p = row[t] * x[t];
            s += p;
        }
        y[r] = s;
    }
}

/* model.rs:253-262 for a Q8_0 tensor: self.tensor() dequantizes the whole
 * tensor (lib.rs:154-162), then the same fold as orc_matvec_f32. */
int orc_matvec_q8_0(const uint8_t *w, size_t rows, size_t k, const float *x, float *y) {
    if (k % QK8_0) return -1;
    float *row = (float *)malloc(k * sizeof(float));
    if (!row) return -1;
    size_t rb = k / QK8_0 * Q8_0_BB;
    for (size_t r = 0; r < rows; ++r) {
        deq_q8_0(w + r * rb, k, row);
        float s = -0.0f;
        for (size_t t = 0; t < k; ++t) {
            float p = row[t] * x[t];
            s += p;
        }
        y[r] = s;
    }
    free(row);
    return 0;
}

/* route: crates/llamd-models/src/moe.rs:73-113.
 * Softmax over all experts, stable sort by probability descending with ties
 * to the lower index, take n_used, gather, renormalise with the 2^-14 floor. */
static const float *g_sort_probs;
static int cmp_route(const void *pa, const void *pb) {
    uint32_t a = *(const uint32_t *)pa, b = *(const uint32_t *)pb;
    float x = g_sort_probs[a], y = g_sort_probs[b];
    /* probs[b].partial_cmp(&probs[a]).unwrap_or(Equal).then(a.cmp(&b)) */
    if (y < x) return -1; /* b < a in value -> a first */
    if (y > x) return 1;
    return (a < b) ? -1 : (a > b);
}

int orc_route(const float *logits, size_t n_expert, size_t n_used, uint32_t *experts,
              float *weights_raw, float *weight_sum, float *weights) {
    if (n_used == 0 || n_used > n_expert) return -1;
    float max = -INFINITY;
    for (size_t i = 0; i < n_expert; ++i) max = fmaxf(max, logits[i]); /* f32::max */
    float *probs = (float *)malloc(n_expert * sizeof(float));
    uint32_t *idx = (uint32_t *)malloc(n_expert * sizeof(uint32_t));
    if (!probs || !idx) { free(probs); free(idx); return -1; }
    for (size_t i = 0; i < n_expert; ++i) probs[i] = expf(logits[i] - max);
    float total = -0.0f;
    for (size_t i = 0; i < n_expert; ++i) total += probs[i];
    for (size_t i = 0; i < n_expert; ++i) probs[i] /= total;
    for (size_t i = 0; i < n_expert; ++i) idx[i] = (uint32_t)i;
    /* the comparator is a total order on finite probabilities (ties broken by
     * index), so any correct sort yields Rust's stable sort_by order */
    g_sort_probs = probs;
    qsort(idx, n_expert, sizeof(uint32_t), cmp_route);
    float raw[1024];
    float s = -0.0f;
    for (size_t k = 0; k < n_used && k < 1024; ++k) {
        raw[k] = probs[idx[k]];
        s += raw[k];
    }
    s = fmaxf(s, ORC_WEIGHT_SUM_FLOOR);
    for (size_t k = 0; k < n_used; ++k) {
        if (experts) experts[k] = idx[k];
        if (weights_raw) weights_raw[k] = raw[k];
        if (weights) weights[k] = raw[k] / s;
    }
    if (weight_sum) *weight_sum = s;
    free(probs);
    free(idx);
    return 0;
}

/* CpuBackend::silu: crates/llamd-cpu/src/lib.rs:103-106 -- v / (1 + exp(-v)) */
void orc_silu(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        y[i] = v / (1.0f + expf(-v));
    }
}

/* CpuBackend::rms_norm: crates/llamd-cpu/src/lib.rs:55-75. Per row: the sum
 * of squares in f32, in order, from 0.0; scale = 1 / sqrt(sum / n + eps);
 * out = x * scale. */
void orc_rms_norm(const float *x, int rows, int n, float eps, float *out) {
    for (int r = 0; r < rows; ++r) {
        const float *src = x + (size_t)r * n;
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) {
            const float sq = src[i] * src[i];
            sum = sum + sq;
        }
        const float mean = sum / (float)n;
        const float t = mean + eps;
        const float scale = 1.0f / sqrtf(t);
        for (int i = 0; i < n; ++i) out[(size_t)r * n + i] = src[i] * scale;
    }
}

/* CpuBackend::mul: crates/llamd-cpu/src/lib.rs:112-113 */
void orc_mul(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
}

/* CpuBackend::softmax: crates/llamd-cpu/src/lib.rs:81-101 (one row) */
void orc_softmax(const float *x, float *y, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float e = expf(x[i] - max);
        y[i] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) y[i] *= inv;
}

/* Model::matvec_expert_quant Q6_K branch: crates/llamd-models/src/model.rs:279-318
 * (expert e starts at e * per_expert bytes, model.rs:188-227). */
int orc_matvec_expert_q6k(const uint8_t *w, size_t n_expert, size_t rows, size_t k,
                          size_t expert, const float *x, float *y) {
    if (expert >= n_expert || k % QK_K) return -1;
    size_t per = rows * (k / QK_K) * Q6K_BB;
    return orc_matvec_q6k(w + expert * per, rows, k, x, y);
}

/* moe_ffn: crates/llamd-runtime/src/layer.rs:230-260 */
int orc_moe_ffn(const float *x, size_t n_embd, size_t n_ff, size_t n_expert,
                const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                const uint32_t *experts, const float *weights, size_t n_used, float *out) {
    float *g = (float *)malloc(n_ff * sizeof(float));
    float *u = (float *)malloc(n_ff * sizeof(float));
    float *act = (float *)malloc(n_ff * sizeof(float));
    float *dn = (float *)malloc(n_embd * sizeof(float));
    int rc = -1;
    if (!g || !u || !act || !dn) goto done;
    for (size_t i = 0; i < n_embd; ++i) out[i] = 0.0f;
    for (size_t k = 0; k < n_used; ++k) {
        size_t e = experts[k];
        float w = weights[k];
        if (orc_matvec_expert_q6k(gate, n_expert, n_ff, n_embd, e, x, g)) goto done;
        if (orc_matvec_expert_q6k(up, n_expert, n_ff, n_embd, e, x, u)) goto done;
        orc_silu(g, act, n_ff);
        orc_mul(act, u, act, n_ff);
        if (orc_matvec_expert_q6k(down, n_expert, n_embd, n_ff, e, act, dn)) goto done;
        for (size_t i = 0; i < n_embd; ++i) {
            float p = w * dn[i];
            out[i] += p;
        }
    }
    rc = 0;
done:
    free(g); free(u); free(act); free(dn);
    return rc;
}

/* One decode layer's FFN half: router (R8) -> route (R9) -> moe_ffn (R11)
 * -> residual (R12, crates/llamd-runtime/src/layer.rs:281-287). */
int orc_moe_layer(const float *x, const float *x_res, size_t n_embd, size_t n_ff,
                  size_t n_expert, size_t n_used, const float *router,
                  const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                  float *out, float *logits_out, uint32_t *ids_out, float *weights_out) {
    float logits[1024];
    uint32_t ids[1024];
    float wts[1024];
    if (n_expert > 1024 || n_used > n_expert) return -1;
    orc_matvec_f32(router, n_expert, n_embd, x, logits);
    if (orc_route(logits, n_expert, n_used, ids, NULL, NULL, wts)) return -1;
    if (orc_moe_ffn(x, n_embd, n_ff, n_expert, gate, up, down, ids, wts, n_used, out)) return -1;
    for (size_t i = 0; i < n_embd; ++i) {
        float f = out[i];
        out[i] = x_res[i];
        out[i] += f;
    }
    if (logits_out) memcpy(logits_out, logits, n_expert * sizeof(float));
    if (ids_out) memcpy(ids_out, ids, n_used * sizeof(uint32_t));
    if (weights_out) memcpy(weights_out, wts, n_used * sizeof(float));
    return 0;
}

/* argmax: crates/llamd-testing/tests/device_forward.rs:23-37 */
uint32_t orc_argmax(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

/* R14: token-major composition (vulkan_prefill.rs:268-333 holds the grouped
 * path to exactly this). */
int orc_moe_ffn_tokens(const float *x, size_t n_tok, size_t n_embd, size_t n_ff,
                       size_t n_expert, const uint8_t *gate, const uint8_t *up,
                       const uint8_t *down, const uint32_t *ids, const float *weights,
                       size_t n_used, float *out) {
    for (size_t t = 0; t < n_tok; ++t) {
        if (orc_moe_ffn(x + t * n_embd, n_embd, n_ff, n_expert, gate, up, down,
                        ids + t * n_used, weights + t * n_used, n_used, out + t * n_embd))
            return -1;
    }
    return 0;
}

/* tolerance.rs:116-129 */
int orc_close(float a, float b, float tol) {
    if (tol == 0.0f) return f2u(a) == f2u(b);
    if (isnan(a) || isnan(b)) return isnan(a) && isnan(b);
    float diff = fabsf(a - b);
    float scale = fmaxf(fmaxf(fabsf(a), fabsf(b)), 1.0f);
    return diff / scale <= tol;
}

/* CpuBackend::rope (crates/llamd-cpu/src/lib.rs:158-209), NeoX pairing, in
 * place over `heads` heads of `hd` values at position `pos`:
 *   theta = (pos * freq_scale) / powf(base, (2 * i) / hd)
 *   x[i] = a*cos - b*sin,  x[i + hd/2] = a*sin + b*cos   (a = x[i], b = x[i+hd/2])
 * with Rust's f32 powf / sin / cos, i.e. glibc's powf, sinf, cosf. */
void orc_rope(float *x, int heads, int hd, uint32_t pos, float base) {
    const int half = hd / 2;
    const float p = (float)pos * 1.0f;
    for (int h = 0; h < heads; ++h) {
        float *v = x + (size_t)h * hd;
        for (int i = 0; i < half; ++i) {
            const float exponent = 2.0f * (float)i / (float)hd;
            const float theta = p / powf(base, exponent);
            const float sn = sinf(theta), cs = cosf(theta);
            const float a = v[i], b = v[i + half];
            v[i] = a * cs - b * sn;
            v[i + half] = a * sn + b * cs;
        }
    }
}

/* attend (crates/llamd-runtime/src/attention.rs:73-125): for each head h
 * (kv head h / (n_head / n_head_kv)):
 *   logit_t = (sum_d q[d] * k_t[d], in order from 0.0) * (1 / sqrt(hd))
 *   max fold; e_t = expf(logit_t - max); sum in order from 0.0; inv = 1 / sum
 *   out[d] = sum_t (e_t * inv) * v_t[d], in order from 0.0
 * k, v: [n_kv][n_head_kv * hd]; q, out: [n_head * hd]. */
int orc_attend(const float *q, const float *k, const float *v, int n_kv, int n_head,
               int n_head_kv, int hd, float *out) {
    if (n_head_kv <= 0 || n_head % n_head_kv || hd <= 0 || n_kv <= 0) return -1;
    const int kv_dim = n_head_kv * hd, ratio = n_head / n_head_kv;
    const float scale = 1.0f / sqrtf((float)hd);
    float *logits = (float *)malloc((size_t)n_kv * sizeof(float));
    if (!logits) return -1;
    for (int i = 0; i < n_head * hd; ++i) out[i] = 0.0f;
    for (int h = 0; h < n_head; ++h) {
        const int kvh = h / ratio, qo = h * hd;
        for (int t = 0; t < n_kv; ++t) {
            const float *kr = k + (size_t)t * kv_dim + (size_t)kvh * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += q[qo + d] * kr[d];
            logits[t] = dot * scale;
        }
        float mx = -INFINITY;
        for (int t = 0; t < n_kv; ++t) mx = fmaxf(mx, logits[t]);
        float sum = 0.0f;
        for (int t = 0; t < n_kv; ++t) {
            logits[t] = expf(logits[t] - mx);
            sum += logits[t];
        }
        const float inv = 1.0f / sum;
        for (int t = 0; t < n_kv; ++t) {
            const float w = logits[t] * inv;
            const float *vr = v + (size_t)t * kv_dim + (size_t)kvh * hd;
            for (int d = 0; d < hd; ++d) out[qo + d] += w * vr[d];
        }
    }
    free(logits);
    return 0;
}
