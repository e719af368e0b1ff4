// decode.hip -- the pieces of a whole-token decode step around the
// quantized matvecs: embedding row and attention over the KV cache (QK-norm,
// RoPE and the cache store are in norm.hip, beside the norms they fuse with). Each reproduces the reference CPU path's f32
// operations in its order, so a step is bit-identical to
// crates/llamd-runtime/src/layer.rs:forward (single token, single sequence).
//
// The token and position are read from device memory (not kernel
// arguments), so a step's launches do not change from token to token.
#include "common.hpp"
#include "exact_sum.hpp"
#include "expf_ref.h"
#include "launch.hpp"
#include "q8k_wave.hpp"
#include "row_scale.hpp"

namespace llamd {
namespace {

// One row of a ggml-layout Q6_K table, dequantized as dequantize_q6_k
// (crates/llamd-quant/src/lib.rs:181-226): y = (f16(d) * sc) * (q - 32), all
// products exact in f32. get_rows of the dequantized table
// (crates/llamd-cpu/src/lib.rs:211-224). One wave per 256-value block; lane
// (half h, l) writes elements l, l+32, l+64, l+96 of half h.
// Sequence s = blockIdx.y reads its token at tok[s * tok_stride] (tok null:
// tok_fixed) and writes row s of out.
__global__ __launch_bounds__(64) void embed_q6k(const uint8_t *table, const int32_t *tok,
                                                int tok_stride, int tok_fixed, int blocks,
                                                float *out) {
    const int b = blockIdx.x, lane = threadIdx.x, sq = blockIdx.y;
    const int token = tok ? tok[(size_t)sq * tok_stride] : tok_fixed;
    out += (size_t)sq * blocks * 256;
    const uint8_t *blk = table + ((size_t)token * blocks + b) * 210;
    const int half = lane >> 5, l = lane & 31;
    const uint8_t *ql = blk + half * 64, *qh = blk + 128 + half * 32;
    const int8_t *sc = (const int8_t *)(blk + 192 + half * 8);
    const float d = f16_bits_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
    const int is = l / 16;
    const uint8_t h = qh[l], lo0 = ql[l], lo1 = ql[l + 32];
    const int q1 = ((lo0 & 0x0F) | ((h >> 0) & 3) << 4) - 32;
    const int q2 = ((lo1 & 0x0F) | ((h >> 2) & 3) << 4) - 32;
    const int q3 = ((lo0 >> 4) | ((h >> 4) & 3) << 4) - 32;
    const int q4 = ((lo1 >> 4) | ((h >> 6) & 3) << 4) - 32;
    float *y = out + (size_t)b * 256 + half * 128;
    y[l] = d * (float)sc[is] * (float)q1;
    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
}

constexpr int ATT_MAX_KV = 16384;  // positions whose logits fit in LDS

// attend (crates/llamd-runtime/src/attention.rs:73-125), one workgroup per
// query head (kv head h / (n_head / n_head_kv)), n_kv = pos + 1:
//   logit_t = (sum_d q[d] k_t[d], in order from 0) * scale       one lane per t
//   max; e_t = expf(logit_t - max)                                all lanes
//   sum_t e_t in order from 0; inv = 1 / sum                      one lane
//   out[d] = sum_t (e_t * inv) v_t[d] in order from 0             one lane per d
// Sequence s = blockIdx.y: n_kv = pos_p[s * pos_stride] + 1 (pos_p null:
// n_kv_fixed), q / out row s, its cache slice at s * cache_seq_stride. An
// n_kv outside 1..ATT_MAX_KV writes NaN.
__global__ __launch_bounds__(256) void attend_decode(const float *q, const float *kc,
                                                     const float *vc, const int32_t *pos_p,
                                                     int n_head, int n_head_kv, int hd, float scale,
                                                     float *out, int n_kv_fixed, int pos_stride,
                                                     size_t cache_seq_stride) {
    __shared__ float lg[ATT_MAX_KV];
    __shared__ float qs[256];
    __shared__ float red[4];
    __shared__ uint64_t tab[32];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sq = blockIdx.y;
    const int n_kv = pos_p ? pos_p[(size_t)sq * pos_stride] + 1 : n_kv_fixed;
    q += (size_t)sq * n_head * hd;
    out += (size_t)sq * n_head * hd;
    kc += (size_t)sq * cache_seq_stride;
    vc += (size_t)sq * cache_seq_stride;
    if (n_kv < 1 || n_kv > ATT_MAX_KV) {
        for (int d = tid; d < hd; d += 256) out[h * hd + d] = __builtin_nanf("");
        return;
    }
    const int kv_dim = n_head_kv * hd, kvh = h / (n_head / n_head_kv);
    if (wave == 0) expf_ref_tab_fill(tab);
    for (int d = tid; d < hd; d += 256) qs[d] = q[h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (int t = tid; t < n_kv; t += 256) {
        const float *kr = kc + (size_t)t * kv_dim + kvh * hd;
        float dot = 0.0f;
        for (int d = 0; d < hd; d += 4) {
            const float4 k4 = *(const float4 *)(kr + d);
            dot = dot + qs[d] * k4.x;
            dot = dot + qs[d + 1] * k4.y;
            dot = dot + qs[d + 2] * k4.z;
            dot = dot + qs[d + 3] * k4.w;
        }
        const float l = dot * scale;
        lg[t] = l;
        mx = fmaxf(mx, l);  // f32::max fold: NaN-ignoring, order-free
    }
    mx = wave_reduce(mx, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int t = tid; t < n_kv; t += 256) lg[t] = expf_ref_tab(lg[t] - mx, tab);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t < n_kv; ++t) sum = sum + lg[t];
        red[0] = __fdiv_rn(1.0f, sum);
    }
    __syncthreads();
    const float inv = red[0];
    for (int d = tid; d < hd; d += 256) {
        const float *vr = vc + (size_t)kvh * hd + d;
        float acc = 0.0f;
        int t = 0;
        for (; t + 8 <= n_kv; t += 8) {
            float vv[8];  // eight loads in flight, then the eight ordered adds
#pragma unroll
            for (int j = 0; j < 8; ++j) vv[j] = vr[(size_t)(t + j) * kv_dim];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float w = lg[t + j] * inv;
                acc = acc + w * vv[j];
            }
        }
        for (; t < n_kv; ++t) {
            const float w = lg[t] * inv;
            acc = acc + w * vr[(size_t)t * kv_dim];
        }
        out[h * hd + d] = acc;
    }
}

// Norm + RoPE of one head (hd values from src) into dst in LDS, as
// qk_norm_rope_store does: (x * scale) * w, then a*cos - b*sin and
// a*sin + b*cos on the halves. One wave; w null skips the norm.
__device__ void head_norm_rope(const float *src, const float *w, const float2 *row, int hd,
                               float eps, float *sq, float *buf, float *dst) {
    const int lane = threadIdx.x & 63, half = hd / 2;
    // every global value this wave needs, loaded before any is used (hd <= 256)
    float xv[4], wv[4];
    float2 cv[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + WAVE * j;
        xv[j] = d < hd ? src[d] : 0.0f;
        wv[j] = d < hd && w ? w[d] : 1.0f;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = lane + WAVE * j;
        cv[j] = i < half ? row[i] : make_float2(0.0f, 0.0f);
    }
    float scale = 1.0f;
    if (w) {
        // the sum of squares in order by lane 0 (row_scale_wave's fold)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + WAVE * j < hd) sq[lane + WAVE * j] = xv[j] * xv[j];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (lane == 0) {
            float sum = 0.0f;
            for (int d = 0; d < hd; d += 32) {
                float4 v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = *(const float4 *)(sq + d + 4 * j);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    sum = sum + v[j].x;
                    sum = sum + v[j].y;
                    sum = sum + v[j].z;
                    sum = sum + v[j].w;
                }
            }
            const float mean = __fdiv_rn(sum, (float)hd);
            scale = __fdiv_rn(1.0f, sqrt_rn(mean + eps));
        }
        scale = __shfl(scale, 0, WAVE);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + WAVE * j;
        if (d < hd) buf[d] = w ? (xv[j] * scale) * wv[j] : xv[j];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = lane + WAVE * j;
        if (i < half) {
            const float a = buf[i], b = buf[i + half];
            dst[i] = a * cv[j].x - b * cv[j].y;
            dst[i + half] = a * cv[j].y + b * cv[j].x;
        }
    }
}

// One decode step's attention block after the Q/K/V matvecs, two query
// heads (hd = 128) per workgroup -- one 256-value Q8_K block of the output:
//   1. per head: QK-norm + RoPE of Q (wave 0 of the head's 256 threads) and
//      of this position's K, plus its V (wave 1); the first query head of
//      each kv group also appends K and V to the cache. The other workgroups
//      of the group use their own copy of the same values for position pos,
//      so no workgroup waits on another.
//   2. attention exactly as attend_decode: the logits' dot products in
//      order, the max, expf_ref, the in-order sum, 1 / sum, the in-order
//      weighted V sum.
//   3. Q8_K of the workgroup's 256 outputs (quantize_q8_k bits) for the O
//      projection, and the f32 outputs if `out` is set.
// Cached K and V rows reach LDS in chunks of ATT_CHUNK positions with
// coalesced loads (all of a chunk's loads in flight at once; the first
// chunk's while the norms run): one thread per position then folds its K
// row, and one per dimension its V column, from LDS.
// Bit-identical to qk_norm_rope_store + attend_decode + q8k_quantize.
constexpr int ATT_HD = 128;
constexpr int ATT_CHUNK = 64;
constexpr int ATT_KS = ATT_HD + 4;  // padded K row in LDS (fewer bank conflicts)

// Staging of cached K or V positions [c0, c0 + ATT_CHUNK) below pos into LDS
// for the workgroup's nkv kv slots (512 threads): each thread loads its
// float4s first (ATT_PER at most), then stores them.
constexpr int ATT_PER = 2 * ATT_CHUNK * (ATT_HD / 4) / 512;
// a native vector (HIP's float4 struct copies stayed in scratch memory here)
typedef float att_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void att_stage_load(att_f4 (&r)[ATT_PER], const float *cache, int c0,
                                               int pos, int nkv, int h0, int group, int kv_dim) {
    constexpr int C = ATT_CHUNK, D4 = ATT_HD / 4;
    const int np = min(C, pos - c0), last = np > 0 ? np - 1 : 0;
#pragma unroll
    for (int k = 0; k < ATT_PER; ++k) {
        const int i = threadIdx.x + 512 * k;  // over [slot][t][d4]
        const int sl = i / (C * D4), t = min((i / D4) % C, last), d4 = i % D4;
        // a slot past nkv reads slot 0's row again (same lines; never stored)
        const int kh = (h0 + (sl < nkv ? sl : 0)) / group;
        r[k] = *(const att_f4 *)(cache + (size_t)(c0 + t) * kv_dim + (size_t)kh * ATT_HD + 4 * d4);
    }
}

__device__ __forceinline__ void att_stage_store(const att_f4 (&r)[ATT_PER], float *dst, int stride,
                                                int c0, int pos, int nkv) {
    constexpr int C = ATT_CHUNK, D4 = ATT_HD / 4;
    const int np = min(C, pos - c0);
#pragma unroll
    for (int k = 0; k < ATT_PER; ++k) {
        const int i = threadIdx.x + 512 * k;
        const int sl = i / (C * D4), t = (i / D4) % C, d4 = i % D4;
        if (sl < nkv && t < np) *(att_f4 *)(dst + ((size_t)sl * C + t) * stride + 4 * d4) = r[k];
    }
}

// Up to two regions of a later launch's weights to read into L2 under the
// attention (n0 pieces of b0 bytes from p0, then n1 of b1 from p1).
struct AttPrefetch {
    const uint8_t *p0, *p1;
    unsigned b0, b1;
    int n0, n1;
};

__global__ __launch_bounds__(512) void attend_fused(
    const float *q_raw, const float *k_raw, const float *v_raw, const float *qw, const float *kw,
    const float2 *cs, const int32_t *pos_p, int n_head, int n_head_kv, float eps, float scale,
    int max_kv, float *kc, float *vc, int8_t *oq, float *od, float *out, AttPrefetch pf) {
    constexpr int HD = ATT_HD, C = ATT_CHUNK, KS = ATT_KS;
    if (blockIdx.x >= n_head / 2) {
        // a prefetch workgroup: one piece of a later launch's weights into
        // this XCD's L2 (piece i of a region goes to the workgroup of this
        // launch that shares XCD i % 8 with the later launch's workgroup i),
        // read and dropped; no result depends on it
        const int i = blockIdx.x - n_head / 2;
        const bool r0 = i < pf.n0;
        const uint8_t *base = r0 ? pf.p0 + (size_t)i * pf.b0 : pf.p1 + (size_t)(i - pf.n0) * pf.b1;
        const unsigned pf_bytes = r0 ? pf.b0 : pf.b1;
        const uint4 *src = (const uint4 *)base;
        const unsigned n16 = pf_bytes / 16;
        uint32_t acc = 0;
        for (unsigned i = threadIdx.x; i < n16; i += 512) {
            const uint4 q = src[i];
            acc ^= q.x ^ q.y ^ q.z ^ q.w;
        }
        if (acc == 0x9E3779B9u && pf_bytes == 1u) od[0] = 0.0f;  // never (pf_bytes % 16 == 0): keeps the loads
        return;
    }
    extern __shared__ __align__(16) float dyn[];  // lg [2][max_kv] | K [nkv][C][KS] | V [nkv][C][HD]
    __shared__ __align__(16) float qs[2][HD], kn[2][HD], vn[2][HD];
    __shared__ __align__(16) float sq[2][2][HD], buf[2][2][HD];
    __shared__ __align__(16) float ov[256];
    __shared__ float red[2][4];
    __shared__ uint64_t tab[2][32];
    const int grp = threadIdx.x >> 8, tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
    const int h0 = blockIdx.x * 2, h = h0 + grp, group = n_head / n_head_kv;
    const int kvh = h / group, kv_dim = n_head_kv * HD, pos = pos_p[0], n_kv = pos + 1;
    const int nkv = group >= 2 ? 1 : 2;   // distinct kv heads of the two query heads
    const int slot = nkv == 1 ? 0 : grp;  // this head's K / V staging slot
    const int lgs = (max_kv + 3) & ~3;    // logits row stride (float4-aligned)
    float *lg = dyn + (size_t)grp * lgs;
    float *kst = dyn + (size_t)2 * lgs;
    float *vst = kst + (size_t)nkv * C * KS;
    const float2 *row = cs + (size_t)pos * (HD / 2);

    att_f4 sk[ATT_PER], sv[ATT_PER];
    if (pos > 0) {
        att_stage_load(sk, kc, 0, pos, nkv, h0, group, kv_dim);
        att_stage_load(sv, vc, 0, pos, nkv, h0, group, kv_dim);
    }
    if (wave == 0) {
        head_norm_rope(q_raw + (size_t)h * HD, qw, row, HD, eps, sq[grp][0], buf[grp][0], qs[grp]);
    } else if (wave == 1) {
        const float v0 = v_raw[(size_t)kvh * HD + lane], v1 = v_raw[(size_t)kvh * HD + WAVE + lane];
        head_norm_rope(k_raw + (size_t)kvh * HD, kw, row, HD, eps, sq[grp][1], buf[grp][1], kn[grp]);
        vn[grp][lane] = v0;
        vn[grp][WAVE + lane] = v1;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (h % group == 0)
            for (int d = lane; d < HD; d += WAVE) {
                kc[(size_t)pos * kv_dim + (size_t)kvh * HD + d] = kn[grp][d];
                vc[(size_t)pos * kv_dim + (size_t)kvh * HD + d] = vn[grp][d];
            }
    } else if (wave == 2) {
        expf_ref_tab_fill(tab[grp]);
    }
    if (pos > 0) {
        att_stage_store(sk, kst, KS, 0, pos, nkv);
        att_stage_store(sv, vst, HD, 0, pos, nkv);
    }
    __syncthreads();

    // logits: one thread per position, q . k in order from 0; 32 values of
    // q and of the row read from LDS per step, then their 32 ordered adds
    const auto qdot = [&](const float *kr) {
        float dot = 0.0f;
#pragma unroll
        for (int d0 = 0; d0 < HD; d0 += 32) {
            float4 k4[8], q4[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                k4[j] = *(const float4 *)(kr + d0 + 4 * j);
                q4[j] = *(const float4 *)(&qs[grp][d0 + 4 * j]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                dot = dot + q4[j].x * k4[j].x;
                dot = dot + q4[j].y * k4[j].y;
                dot = dot + q4[j].z * k4[j].z;
                dot = dot + q4[j].w * k4[j].w;
            }
        }
        return dot;
    };
    float mx = -INFINITY;
    for (int c0 = 0; c0 < n_kv; c0 += C) {
        if (c0 > 0) {
            // later chunks (long contexts): every thread stages, then folds
            if (c0 < pos) att_stage_load(sk, kc, c0, pos, nkv, h0, group, kv_dim);
            __syncthreads();
            if (c0 < pos) att_stage_store(sk, kst, KS, c0, pos, nkv);
            __syncthreads();
        }
        const int t = c0 + tid;
        if (tid < C && t < n_kv) {
            const float dot = t < pos ? qdot(kst + ((size_t)slot * C + tid) * KS) : qdot(kn[grp]);
            const float l = dot * scale;
            lg[t] = l;
            mx = fmaxf(mx, l);  // f32::max fold: NaN-ignoring, order-free
        }
    }
    mx = wave_reduce(mx, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    if (lane == 0) red[grp][wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[grp][0], red[grp][1]), fmaxf(red[grp][2], red[grp][3]));
    for (int t = tid; t < n_kv; t += 256) lg[t] = expf_ref_tab(lg[t] - mx, tab[grp]);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        int t = 0;
        for (; t + 32 <= n_kv; t += 32) {
            float4 e[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = *(const float4 *)(lg + t + 4 * j);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sum = sum + e[j].x;
                sum = sum + e[j].y;
                sum = sum + e[j].z;
                sum = sum + e[j].w;
            }
        }
        for (; t < n_kv; ++t) sum = sum + lg[t];
        red[grp][0] = __fdiv_rn(1.0f, sum);
    }
    __syncthreads();
    const float inv = red[grp][0];

    // the weighted V sum, one thread per dimension, in position order; the
    // first chunk was staged with K
    float acc = 0.0f;
    for (int c0 = 0; c0 < pos; c0 += C) {
        if (c0 > 0) {
            att_stage_load(sv, vc, c0, pos, nkv, h0, group, kv_dim);
            __syncthreads();
            att_stage_store(sv, vst, HD, c0, pos, nkv);
            __syncthreads();
        }
        if (tid < HD) {
            const int np = min(C, pos - c0);
            const float *vr = vst + (size_t)slot * C * HD + tid;
            int t = 0;
            for (; t + 8 <= np; t += 8) {
                // the 8 values and their 8 weights read together, then the
                // ordered adds (lg + c0 + t is 16-byte aligned)
                float vv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) vv[j] = vr[(size_t)(t + j) * HD];
                const float4 l0 = *(const float4 *)(lg + c0 + t), l1 = *(const float4 *)(lg + c0 + t + 4);
                const float ll[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float w = ll[j] * inv;
                    acc = acc + w * vv[j];
                }
            }
            for (; t < np; ++t) {
                const float w = lg[c0 + t] * inv;
                acc = acc + w * vr[(size_t)t * HD];
            }
        }
    }
    if (tid < HD) {
        const float w = lg[pos] * inv;
        acc = acc + w * vn[grp][tid];
        ov[grp * HD + tid] = acc;
        if (out) out[(size_t)h * HD + tid] = acc;
    }
    __syncthreads();
    if (threadIdx.x < WAVE) {
        const float4 v4 = *(const float4 *)(ov + 4 * lane);
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        quantize_wave(v, lane, oq + (size_t)blockIdx.x * QK_K, od + blockIdx.x, nullptr);
    }
}

// ---- attention over long contexts: logits spread over the GPU -------------
// attend_fused runs n_head / 2 workgroups and walks the positions 64 at a
// time, so its cost grows by ~50 ns per position and layer. Past a few
// hundred positions the same arithmetic runs in two launches instead (after
// qk_norm_rope_store has put the normed, rotated Q in place and K, V in the
// cache, and before the Q8_K of the output: q8k_quantize, or inside the O
// projection, q6k_mv_f32x):
//  - attend_logits: workgroup w keeps kv head w % n_head_kv and takes its
//    position blocks w / n_head_kv, + gridDim.x / n_head_kv, ...; the block's
//    K rows are staged in LDS (rows padded to 132 floats) and thread
//    (query head j of the group, position t) forms logit_t = (q . k_t, the
//    128 products added in order from 0) * scale into scores.
//  - attend_finish: AF_SL 1024-thread workgroups per head, each on
//    128 / AF_SL dimensions: max (order free), e_t = expf(logit_t - max),
//    their in-order sum by exact_sum_nonneg (the reference's bits from a
//    workgroup-wide certificate), inv = 1 / sum (every workgroup of the head
//    the same), then one thread per dimension adds (e_t * inv) * v_t[d] in
//    position order from V rows staged in LDS (half a row per position)
//    into the f32 output.
// The same operations in the same order as attend_fused (and the reference,
// attention.rs:73-125): the same bits.
constexpr int AL_KS = ATT_HD + 4;   // padded K row in LDS
constexpr int AL_MAX_GROUP = 16;    // query heads per kv head

__global__ __launch_bounds__(256) void attend_logits(const float *q, const float *kc,
                                                     const int32_t *pos_p, int n_head,
                                                     int n_head_kv, float scale, float *scores,
                                                     int max_kv) {
    constexpr int HD = ATT_HD;
    __shared__ __align__(16) float ks[64 * AL_KS];
    __shared__ __align__(16) float qs[AL_MAX_GROUP * HD];
    const int group = n_head / n_head_kv;
    const int ppi = min(64, 256 / group);  // positions per block
    const int g = blockIdx.x % n_head_kv;
    const int stride = gridDim.x / n_head_kv;
    const int kv_dim = n_head_kv * HD;
    const int n_kv = pos_p[0] + 1;
    const int nb = (n_kv + ppi - 1) / ppi;
    const int tid = threadIdx.x;
    if ((int)blockIdx.x / n_head_kv >= nb) return;
    for (int i = tid; i < group * HD / 4; i += 256)
        *(float4 *)(qs + 4 * i) = *(const float4 *)(q + (size_t)g * group * HD + 4 * i);
    const int hl = tid / ppi, tl = tid - hl * ppi;
    for (int pb = blockIdx.x / n_head_kv; pb < nb; pb += stride) {
        const int t0 = pb * ppi, np = min(ppi, n_kv - t0);
        __syncthreads();  // the previous block's rows are read
        for (int i = tid; i < np * (HD / 4); i += 256) {
            const int t = i / (HD / 4), d4 = i - t * (HD / 4);
            *(float4 *)(ks + t * AL_KS + 4 * d4) =
                *(const float4 *)(kc + (size_t)(t0 + t) * kv_dim + (size_t)g * HD + 4 * d4);
        }
        __syncthreads();
        if (hl < group && tl < np) {
            const float *kr = ks + tl * AL_KS, *qr = qs + hl * HD;
            float dot = 0.0f;
#pragma unroll
            for (int d0 = 0; d0 < HD; d0 += 32) {
                float4 k4[8], q4[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    k4[j] = *(const float4 *)(kr + d0 + 4 * j);
                    q4[j] = *(const float4 *)(qr + d0 + 4 * j);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dot = dot + q4[j].x * k4[j].x;
                    dot = dot + q4[j].y * k4[j].y;
                    dot = dot + q4[j].z * k4[j].z;
                    dot = dot + q4[j].w * k4[j].w;
                }
            }
            scores[(size_t)(g * group + hl) * max_kv + t0 + tl] = dot * scale;
        }
    }
}

constexpr int AF_PER = 8;  // float4s of one V chunk per thread
constexpr int AF_SL = 2;   // workgroups per head (dimension slices)
constexpr int AF_DS = ATT_HD / AF_SL;

__global__ __launch_bounds__(1024) void attend_finish(const float *scores, const float *vc,
                                                      const int32_t *pos_p, int n_head,
                                                      int n_head_kv, int max_kv, int chunk,
                                                      float *out) {
    constexpr int HD = ATT_HD, DS = AF_DS, DS4 = AF_DS / 4;
    // e_t [max_kv], then the V chunk [chunk][DS]
    extern __shared__ __align__(16) float lgs[];
    __shared__ ExactSumLds xl;
    __shared__ uint64_t tab[32];
    __shared__ float red[16];
    __shared__ float inv1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x, sd = blockIdx.y * DS;  // the head and the slice's first dimension
    const int kv_dim = n_head_kv * HD, kvh = h / (n_head / n_head_kv);
    const int n_kv = pos_p[0] + 1;
    if (wave == 0) expf_ref_tab_fill(tab);
    // the head's logits into LDS, and their max (f32::max fold: NaN
    // ignoring, order free)
    float mx = -INFINITY;
    for (int t = tid; t < n_kv; t += 1024) {
        const float l = scores[(size_t)h * max_kv + t];
        lgs[t] = l;
        mx = fmaxf(mx, l);
    }
    mx = wave_reduce(mx, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = -INFINITY;
    for (int w = 0; w < 16; ++w) mx = fmaxf(mx, red[w]);
    for (int t = tid; t < n_kv; t += 1024) lgs[t] = expf_ref_tab(lgs[t] - mx, tab);
    __syncthreads();
    // their sum in order from 0, by the workgroup
    {
        const int m = xsum_run(n_kv, 1024), j0 = tid * m;
        float v[XSUM_M];
#pragma unroll
        for (int k = 0; k < XSUM_M; ++k) v[k] = (k < m && j0 + k < n_kv) ? lgs[j0 + k] : 0.0f;
        const float *e = lgs;
        const float sum = exact_sum_nonneg(v, n_kv, 1024, xl, [e](int j) { return e[j]; });
        if (tid == 0) inv1 = __fdiv_rn(1.0f, sum);
    }
    __syncthreads();
    // the weighted V sum, one thread per dimension of this slice, in
    // position order, from V rows staged in LDS a chunk at a time: the next
    // chunk's loads (all threads, into registers) are in flight while this
    // one is folded
    float *vst = lgs + max_kv;                    // [chunk][DS]
    const int units = chunk * DS4;                // float4s per chunk
    att_f4 reg[AF_PER];
    // every load unconditional, at a clamped row (a conditional load makes
    // the compiler wait for each one before issuing the next); the extra
    // ones re-read a row of the chunk and are never stored
    const auto stage_load = [&](int c0) {
        const int last = min(chunk, n_kv - c0) - 1;
#pragma unroll
        for (int k = 0; k < AF_PER; ++k) {
            const int i = tid + 1024 * k;
            const int t = min(i / DS4, last), d4 = i % DS4;
            reg[k] = *(const att_f4 *)(vc + (size_t)(c0 + t) * kv_dim + (size_t)kvh * HD + sd + 4 * d4);
        }
    };
    const auto stage_store = [&](int c0) {
        const int np = min(chunk, n_kv - c0);
#pragma unroll
        for (int k = 0; k < AF_PER; ++k) {
            const int i = tid + 1024 * k;
            if (i < units && i / DS4 < np) *(att_f4 *)(vst + 4 * i) = reg[k];
        }
    };
    const bool folder = tid < DS;
    const float inv = inv1;
    float acc = 0.0f;
    stage_load(0);
    for (int c0 = 0; c0 < n_kv; c0 += chunk) {
        stage_store(c0);
        __syncthreads();
        if (c0 + chunk < n_kv) stage_load(c0 + chunk);
        if (folder) {
            const int np = min(chunk, n_kv - c0);
            const float *vr = vst + tid;
            int t = 0;
            for (; t + 8 <= np; t += 8) {
                // the 8 values and their 8 weights read together, then the
                // ordered adds (lgs + c0 + t is 16-byte aligned: c0 and t are
                // multiples of 8)
                float vv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) vv[j] = vr[(size_t)(t + j) * DS];
                const float4 e0 = *(const float4 *)(lgs + c0 + t), e1 = *(const float4 *)(lgs + c0 + t + 4);
                const float ee[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float w = ee[j] * inv;
                    acc = acc + w * vv[j];
                }
            }
            for (; t < np; ++t) {
                const float w = lgs[c0 + t] * inv;
                acc = acc + w * vr[(size_t)t * DS];
            }
        }
        __syncthreads();  // the chunk is read before the next one is stored
    }
    if (folder) out[(size_t)h * HD + sd + tid] = acc;
}

}  // namespace

int launch_embed_q6k(const void *table, const int32_t *tok, int blocks, float *out, hipStream_t st,
                     int nseq, int tok_stride, int tok_fixed) {
    if (blocks <= 0 || nseq <= 0) return -1;
    hipLaunchKernelGGL(embed_q6k, dim3(blocks, nseq), dim3(64), 0, st, (const uint8_t *)table, tok,
                       tok_stride, tok_fixed, blocks, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int attend_max_kv() { return ATT_MAX_KV; }

namespace {
size_t g_fused_lds = 0;  // the dynamic LDS attend_fused may use (raised by prepare)
}

namespace {
size_t fused_lds(int n_head, int n_head_kv, int max_kv) {
    const int nkv = n_head / n_head_kv >= 2 ? 1 : 2;
    return (size_t)2 * ((max_kv + 3) & ~3) * 4 + (size_t)nkv * ATT_CHUNK * (ATT_KS + ATT_HD) * 4;
}
}  // namespace

bool attend_fused_fits(int n_head, int n_head_kv, int hd, int max_kv) {
    if (hd != ATT_HD || n_head_kv <= 0 || n_head % n_head_kv || n_head % 2 || max_kv <= 0) return false;
    return fused_lds(n_head, n_head_kv, max_kv) + 24 * 1024 <= 160 * 1024;
}

int attend_fused_prepare(int n_head, int n_head_kv, int hd, int max_kv) {
    if (!attend_fused_fits(n_head, n_head_kv, hd, max_kv)) return -1;
    const size_t lds = fused_lds(n_head, n_head_kv, max_kv);
    if (lds <= g_fused_lds) return 0;
    if (hipFuncSetAttribute((const void *)attend_fused, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
        return -1;
    g_fused_lds = lds;
    return 0;
}

int launch_attend_fused(const float *q, const float *k, const float *v, const float *qw,
                        const float *kw, const float2 *cs, const int32_t *pos, int n_head,
                        int n_head_kv, int hd, float eps, float scale, int max_kv, float *kc,
                        float *vc, int8_t *oq, float *od, float *out, hipStream_t st,
                        const void *pf0, size_t b0, int n0, const void *pf1, size_t b1, int n1) {
    if (!attend_fused_fits(n_head, n_head_kv, hd, max_kv)) return -1;
    const size_t lds = fused_lds(n_head, n_head_kv, max_kv);
    if (lds > g_fused_lds) return -1;  // attend_fused_prepare first
    // the pieces of region 1 start on XCD 0 again: region 0 is padded to a
    // multiple of 8 workgroups
    AttPrefetch pf{(const uint8_t *)pf0, (const uint8_t *)pf1, (unsigned)b0, (unsigned)b1, n0, n1};
    if (!pf0 || b0 % 16 || b0 > (1u << 30) || n0 < 0 || (n_head / 2) % 8) pf.n0 = 0;
    if (!pf1 || b1 % 16 || b1 > (1u << 30) || n1 < 0 || pf.n0 % 8 || (n_head / 2) % 8) pf.n1 = 0;
    hipLaunchKernelGGL(attend_fused, dim3(n_head / 2 + pf.n0 + pf.n1), dim3(512), lds, st, q, k, v,
                       qw, kw, cs, pos, n_head, n_head_kv, eps, scale, max_kv, kc, vc, oq, od, out,
                       pf);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

namespace {
size_t g_split_lds = 0;  // the dynamic LDS attend_finish may use (raised by prepare)

// V positions per LDS chunk: what the e_t rows leave of 152 KB, at most
// AF_PER float4s per thread, a multiple of 16 (0: does not fit)
int split_chunk(int n_head, int n_head_kv, int max_kv) {
    (void)n_head;
    (void)n_head_kv;
    const long room = 152L * 1024 - (long)max_kv * 4 - 8 * 1024;
    long c = room / (AF_DS * 4);
    c = std::min<long>(c, (long)AF_PER * 1024 / (AF_DS / 4));
    c -= c % 16;
    return c >= 16 ? (int)c : 0;
}
size_t split_lds(int n_head, int n_head_kv, int max_kv) {
    return (size_t)max_kv * 4 + (size_t)split_chunk(n_head, n_head_kv, max_kv) * AF_DS * 4;
}
}  // namespace

bool attend_split_fits(int n_head, int n_head_kv, int hd, int max_kv) {
    if (hd != ATT_HD || n_head_kv <= 0 || n_head % n_head_kv || n_head % 2 || max_kv <= 0) return false;
    const int group = n_head / n_head_kv;
    return group <= AL_MAX_GROUP && split_chunk(n_head, n_head_kv, max_kv) > 0;
}

int attend_split_prepare(int n_head, int n_head_kv, int hd, int max_kv) {
    if (!attend_split_fits(n_head, n_head_kv, hd, max_kv)) return -1;
    const size_t lds = split_lds(n_head, n_head_kv, max_kv);
    if (lds <= g_split_lds) return 0;
    if (hipFuncSetAttribute((const void *)attend_finish, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
        return -1;
    g_split_lds = lds;
    return 0;
}

int launch_attend_split(const float *q, const float *kc, const float *vc, const int32_t *pos,
                        int n_head, int n_head_kv, int hd, float scale, int max_kv, float *scores,
                        int8_t *oq, float *od, float *out, hipStream_t st) {
    if (!attend_split_fits(n_head, n_head_kv, hd, max_kv) || !out) return -1;
    const size_t lds = split_lds(n_head, n_head_kv, max_kv);
    if (lds > g_split_lds) return -1;  // attend_split_prepare first
    const int chunk = split_chunk(n_head, n_head_kv, max_kv);
    // 256 workgroups (a multiple of n_head_kv), each fixed to one kv head
    const int grid = (256 / n_head_kv) * n_head_kv;
    if (grid <= 0) return -1;
    hipLaunchKernelGGL(attend_logits, dim3(grid), dim3(256), 0, st, q, kc, pos, n_head, n_head_kv,
                       scale, scores, max_kv);
    hipLaunchKernelGGL(attend_finish, dim3(n_head, AF_SL), dim3(1024), lds, st, scores, vc, pos,
                       n_head, n_head_kv, max_kv, chunk, out);
    if (hipGetLastError() != hipSuccess) return -1;
    // oq null: the caller takes the f32 output (launch_q6k_mv_f32x)
    return oq ? launch_q8k_quantize(out, oq, od, nullptr, n_head / 2, st) : 0;
}

int launch_attend_decode(const float *q, const float *kc, const float *vc, const int32_t *pos,
                         int n_head, int n_head_kv, int hd, float scale, float *out,
                         hipStream_t st, int nseq, int n_kv_fixed, int pos_stride,
                         size_t cache_seq_stride) {
    if (hd <= 0 || hd % 4 || hd > 256 || n_head_kv <= 0 || n_head % n_head_kv || nseq <= 0)
        return -1;
    hipLaunchKernelGGL(attend_decode, dim3(n_head, nseq), dim3(256), 0, st, q, kc, vc, pos, n_head,
                       n_head_kv, hd, scale, out, n_kv_fixed, pos_stride, cache_seq_stride);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
