// decode.hip -- the pieces of a whole-token decode step around the
// quantized matvecs: embedding row and attention over the KV cache (QK-norm,
// RoPE and the cache store are in norm.hip, beside the norms they fuse with). Each reproduces the reference CPU path's f32
// operations in its order, so a step is bit-identical to
// crates/llamd-runtime/src/layer.rs:forward (single token, single sequence).
//
// The token and position are read from device memory (not kernel
// arguments), so a step's launches do not change from token to token.
#include "common.hpp"
#include "expf_ref.h"
#include "launch.hpp"

namespace llamd {
namespace {

// One row of a ggml-layout Q6_K table, dequantized as dequantize_q6_k
// (crates/llamd-quant/src/lib.rs:181-226): y = (f16(d) * sc) * (q - 32), all
// products exact in f32. get_rows of the dequantized table
// (crates/llamd-cpu/src/lib.rs:211-224). One wave per 256-value block; lane
// (half h, l) writes elements l, l+32, l+64, l+96 of half h.
__global__ __launch_bounds__(64) void embed_q6k(const uint8_t *table, const int32_t *tok,
                                                int blocks, float *out) {
    const int b = blockIdx.x, lane = threadIdx.x;
    const uint8_t *blk = table + ((size_t)tok[0] * blocks + b) * 210;
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
__global__ __launch_bounds__(256) void attend_decode(const float *q, const float *kc,
                                                     const float *vc, const int32_t *pos_p,
                                                     int n_head, int n_head_kv, int hd, float scale,
                                                     float *out) {
    __shared__ float lg[ATT_MAX_KV];
    __shared__ float qs[256];
    __shared__ float red[4];
    __shared__ uint64_t tab[32];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_kv = pos_p[0] + 1;
    const int kv_dim = n_head_kv * hd, kvh = h / (n_head / n_head_kv);
    if (wave == 0) expf_ref_tab_fill(tab);
    for (int d = tid; d < hd; d += blockDim.x) qs[d] = q[h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (int t = tid; t < n_kv; t += blockDim.x) {
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
    for (int t = tid; t < n_kv; t += blockDim.x) lg[t] = expf_ref_tab(lg[t] - mx, tab);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t < n_kv; ++t) sum = sum + lg[t];
        red[0] = __fdiv_rn(1.0f, sum);
    }
    __syncthreads();
    const float inv = red[0];
    for (int d = tid; d < hd; d += blockDim.x) {
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

}  // namespace

int launch_embed_q6k(const void *table, const int32_t *tok, int blocks, float *out, hipStream_t st) {
    if (blocks <= 0) return -1;
    hipLaunchKernelGGL(embed_q6k, dim3(blocks), dim3(64), 0, st, (const uint8_t *)table, tok, blocks,
                       out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int attend_max_kv() { return ATT_MAX_KV; }

int launch_attend_decode(const float *q, const float *kc, const float *vc, const int32_t *pos,
                         int n_head, int n_head_kv, int hd, float scale, float *out,
                         hipStream_t st) {
    if (hd <= 0 || hd % 4 || hd > 256 || n_head_kv <= 0 || n_head % n_head_kv) return -1;
    hipLaunchKernelGGL(attend_decode, dim3(n_head), dim3(256), 0, st, q, kc, vc, pos, n_head,
                       n_head_kv, hd, scale, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
