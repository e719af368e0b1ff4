// row_scale.hpp -- RMSNorm's scale for a short row by one wave, the sum of
// squares in the reference's order (crates/llamd-cpu/src/lib.rs:55-66):
// all lanes form the rounded squares, one lane adds them in order. Used for
// the per-head QK norm (128 values), where one lane's chain is short.
#pragma once
#include "common.hpp"

namespace llamd {

// The sequential sum of squares of src[0..n) by lane 0 of the calling wave,
// from squares parked in sq[] (all of the wave's lanes write them first).
// Returns scale on every lane of the wave.
__device__ inline float row_scale_wave(const float *src, int n, float eps, float *sq) {
    const int lane = threadIdx.x & 63;
    // every load of the row in flight before the first square is stored (a
    // loop of dependent load -> store would pay one memory latency per step)
    if ((n & 3) == 0 && ((uintptr_t)src & 15) == 0) {
        for (int base = 0; base < n; base += 8 * 4 * WAVE) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + 4 * (j * WAVE + lane);
                if (i < n) v[j] = *(const float4 *)(src + i);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + 4 * (j * WAVE + lane);
                if (i < n)
                    *(float4 *)(sq + i) = make_float4(v[j].x * v[j].x, v[j].y * v[j].y,
                                                       v[j].z * v[j].z, v[j].w * v[j].w);
            }
        }
    } else {
        for (int base = 0; base < n; base += 8 * WAVE) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + j * WAVE + lane;
                if (i < n) v[j] = src[i];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + j * WAVE + lane;
                if (i < n) sq[i] = v[j] * v[j];
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float scale = 0.0f;
    if (lane == 0) {
        float sum = 0.0f;
        int i = 0;
        for (; i + 32 <= n; i += 32) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = *(const float4 *)(sq + i + 4 * j);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sum = sum + v[j].x;
                sum = sum + v[j].y;
                sum = sum + v[j].z;
                sum = sum + v[j].w;
            }
        }
        for (; i < n; ++i) sum = sum + sq[i];
        const float mean = __fdiv_rn(sum, (float)n);
        scale = __fdiv_rn(1.0f, sqrt_rn(mean + eps));
    }
    return __shfl(scale, 0, WAVE);
}

}  // namespace llamd
