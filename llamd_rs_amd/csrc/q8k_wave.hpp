// q8k_wave.hpp -- one wave quantizes one 256-element block to Q8_K,
// bit-exactly as quantize_q8_k (crates/llamd-quant/src/dot.rs:89-128); see
// q8k.hip for the derivation. Shared by the quantize kernels and the fused
// router kernel.
#pragma once

#include "common.hpp"
#include "expf_ref.h"

namespace llamd {

// qs: natural order (the reference's BlockQ8K.qs). qs_cm (optional): the same
// quants in class-major order, byte 32 * (e % 8) + e / 8 for element e, which
// is what the batched kernel's MFMA operand loads want.
__device__ __forceinline__ void quantize_wave(const float v[4], int lane, int8_t *qs, int8_t *qs_cm,
                                              float *d, int16_t *bsums) {
    float amax = 0.0f, mx = 0.0f;
    int idx = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        if (a > amax) { amax = a; mx = v[i]; idx = 4 * lane + i; }
    }
    // (|x|, index) arg-max over the wave; the sign comes from the winning lane
    int win = idx;
    float best = amax;
    wave_argmax(best, win, -1.0f);
    amax = best;
    mx = win == 0x7FFFFFFF ? 0.0f
                           : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), win >> 2));
    int q[4];
    float dv;
    if (amax == 0.0f) {
        q[0] = q[1] = q[2] = q[3] = 0;
        dv = 0.0f;
    } else {
        const float iscale = -127.0f / mx;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = (int)__builtin_rintf(iscale * v[i]);
            q[i] = r < 127 ? r : 127;
        }
        dv = 1.0f / iscale;
    }
    const uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                            ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    if (qs) *(uint32_t *)(qs + 4 * lane) = packed;
    if (qs_cm) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            qs_cm[32 * (e & 7) + (e >> 3)] = (int8_t)q[i];
        }
    }
    int gs = q[0] + q[1] + q[2] + q[3];
    gs += dpp<DPP_XOR1>(0, gs);
    gs += dpp<DPP_XOR2>(0, gs);
    if (bsums && (lane & 3) == 0) bsums[lane >> 2] = (int16_t)gs;
    if (lane == 0) *d = dv;
}


// silu(v) = v / (1 + exp(-v)) with the reference's f32 expf (model.rs silu).
__device__ __forceinline__ float silu_ref(float v, const uint64_t *tab) {
    return v / (1.0f + expf_ref_tab(-v, tab));
}

__device__ __forceinline__ void quantize_block_wave(const float v[4], int lane, int8_t *qs, float *d) {
    quantize_wave(v, lane, qs, nullptr, d, nullptr);
}

}  // namespace llamd
