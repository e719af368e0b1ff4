// q8k_wave.hpp -- one wave quantizes one 256-element block to Q8_K,
// bit-exactly as quantize_q8_k (crates/llamd-quant/src/dot.rs:89-128); see
// q8k.hip for the derivation. Shared by the quantize kernels and the fused
// router kernel, with writers for the reference's layout and for the
// token-chunked layout of the batched matvec.
#pragma once

#include "common.hpp"
#include "expf_ref.h"

namespace llamd {

// Q8_K of the wave's 256 values (4 per lane, elements 4*lane .. 4*lane+3):
// this lane's 4 quants and the block scale d (on every lane).
__device__ __forceinline__ void quantize_wave_q(const float v[4], int lane, int q[4], float &dv) {
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
}

// The reference's BlockQ8K arrays: qs in natural order, d, bsums (optional).
__device__ __forceinline__ void store_q8k(const int q[4], float dv, int lane, int8_t *qs, float *d,
                                          int16_t *bsums) {
    const uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                            ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    if (qs) *(uint32_t *)(qs + 4 * lane) = packed;
    int gs = q[0] + q[1] + q[2] + q[3];
    gs += dpp<DPP_XOR1>(0, gs);
    gs += dpp<DPP_XOR2>(0, gs);
    if (bsums && (lane & 3) == 0) bsums[lane >> 2] = (int16_t)gs;
    if (lane == 0) *d = dv;
}

__device__ __forceinline__ void quantize_wave(const float v[4], int lane, int8_t *qs, float *d,
                                              int16_t *bsums) {
    int q[4];
    float dv;
    quantize_wave_q(v, lane, q, dv);
    store_q8k(q, dv, lane, qs, d, bsums);
}

// ---- token-chunked activations (the batched matvec's operand layout) -----
// 16 token slots form a chunk; block b of chunk k occupies 4 KiB at
// (k * blocks + b) * 4096, holding class plane c (weights e with e % 8 == c)
// at c * 512, token n of the chunk at n * 32 within it, and weight 8 m + c
// at byte m. One MFMA operand load of a class is then one contiguous 512-B
// read for the whole wave. The scales sit at d[(k * blocks + b) * 16 + n].
constexpr int CHUNK_TOKENS = 16;
constexpr int CHUNK_BLOCK_BYTES = 8 * 512;

// The wave's quants regrouped for the chunked layout: lane L ends up with
// the 4 bytes of class plane L / 8 at bytes 4 (L % 8) .. +3 of the token's
// 32 -- elements 8k + L / 8 for k = 4 (L % 8) .. +3 -- gathered from the
// lanes that hold them (lane e / 4 holds element e), so each lane then
// stores one dword per destination instead of four scattered bytes.
__device__ __forceinline__ uint32_t chunk_dword(const int q[4], int lane) {
    const uint32_t own = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                         ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    const int c = lane >> 3, k0 = 4 * (lane & 7);
    uint32_t out = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t v = (uint32_t)__shfl((int)own, 2 * (k0 + t) + (c >> 2), WAVE);
        out |= ((v >> (8 * (c & 3))) & 0xFFu) << (8 * t);
    }
    return out;
}

__device__ __forceinline__ void store_chunk(uint32_t dword, float dv, int lane, int8_t *cq,
                                            float *cd, int slot, int b, int blocks) {
    if (slot < 0) return;  // a pair with no expert (out-of-range id)
    const size_t base = ((size_t)(slot / CHUNK_TOKENS) * blocks + b);
    int8_t *dst = cq + base * CHUNK_BLOCK_BYTES + (slot % CHUNK_TOKENS) * 32;
    *(uint32_t *)(dst + (lane >> 3) * 512 + 4 * (lane & 7)) = dword;
    if (lane == 0) cd[base * CHUNK_TOKENS + slot % CHUNK_TOKENS] = dv;
}

// silu(v) = v / (1 + exp(-v)) with the reference's f32 expf (model.rs silu).
__device__ __forceinline__ float silu_ref(float v, const uint64_t *tab) {
    return v / (1.0f + expf_ref_tab(-v, tab));
}

__device__ __forceinline__ void quantize_block_wave(const float v[4], int lane, int8_t *qs, float *d) {
    quantize_wave(v, lane, qs, d, nullptr);
}

}  // namespace llamd
