// q8k.hip -- bit-exact Q8_K activation quantization on the device.
//
// Restates quantize_q8_k (crates/llamd-quant/src/dot.rs:89-128) for one wave
// per 256-element block, 4 elements per lane:
//   - max = the SIGNED value of largest magnitude, earliest index on ties
//     (the reference's `if a > amax` scan keeps the first); a wave reduction
//     on (|x|, index) with "larger, or equal and lower index" is the same
//     selection in any order;
//   - all-zero block -> d = 0 and zero quants;
//   - iscale = -127 / max, q = min(round_half_even(iscale * x), 127)
//     (v_rndne_f32 is round-half-even), d = 1 / iscale, both IEEE divisions;
//   - bsums[g] = sum of the 16 quants of group g.
// The fused SwiGLU variant first forms act = silu(g) * u exactly as
// CpuBackend::silu and ::mul do (crates/llamd-cpu/src/lib.rs:103-113):
// v / (1 + exp(-v)) with glibc-identical expf, then * u.
#include "common.hpp"
#include "expf_ref.h"
#include "launch.hpp"

namespace llamd {
namespace {

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
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float oa = shfl_xor_f(amax, m);
        const float om = shfl_xor_f(mx, m);
        const int oi = shfl_xor_i(idx, m);
        if (oa > amax || (oa == amax && oi < idx)) { amax = oa; mx = om; idx = oi; }
    }
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
    gs += shfl_xor_i(gs, 1);
    gs += shfl_xor_i(gs, 2);
    if (bsums && (lane & 3) == 0) bsums[lane >> 2] = (int16_t)gs;
    if (lane == 0) *d = dv;
}

__global__ __launch_bounds__(256) void q8k_quantize(const float *x, int8_t *qs, int8_t *qs_cm,
                                                    float *d, int16_t *bsums, int nblocks) {
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const float4 xv = *(const float4 *)(x + (size_t)blk * QK_K + 4 * lane);
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    quantize_wave(v, lane, qs ? qs + (size_t)blk * QK_K : nullptr,
                  qs_cm ? qs_cm + (size_t)blk * QK_K : nullptr, d + blk,
                  bsums ? bsums + (size_t)blk * 16 : nullptr);
}

__device__ __forceinline__ float silu_ref(float v) { return v / (1.0f + expf_ref(-v)); }

// act[i] = silu(gate[i]) * up[i], then Q8_K of act. Optionally stores act.
__global__ __launch_bounds__(256) void swiglu_q8k(const float *gate, const float *up, float *act_out,
                                                  int8_t *qs, int8_t *qs_cm, float *d,
                                                  int16_t *bsums, int nblocks) {
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const size_t o = (size_t)blk * QK_K + 4 * lane;
    const float4 gv = *(const float4 *)(gate + o);
    const float4 uv = *(const float4 *)(up + o);
    float v[4];
    v[0] = silu_ref(gv.x) * uv.x;
    v[1] = silu_ref(gv.y) * uv.y;
    v[2] = silu_ref(gv.z) * uv.z;
    v[3] = silu_ref(gv.w) * uv.w;
    if (act_out) *(float4 *)(act_out + o) = make_float4(v[0], v[1], v[2], v[3]);
    quantize_wave(v, lane, qs ? qs + (size_t)blk * QK_K : nullptr,
                  qs_cm ? qs_cm + (size_t)blk * QK_K : nullptr, d + blk,
                  bsums ? bsums + (size_t)blk * 16 : nullptr);
}

__global__ void silu_mul_f32(const float *gate, const float *up, float *out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_ref(gate[i]) * up[i];
}

}  // namespace

int launch_q8k_quantize(const float *x, int8_t *qs, int8_t *qs_cm, float *d, int16_t *bsums,
                        int nblocks, hipStream_t st) {
    if (nblocks <= 0) return 0;
    hipLaunchKernelGGL(q8k_quantize, dim3((nblocks + 3) / 4), dim3(256), 0, st, x, qs, qs_cm, d,
                       bsums, nblocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_swiglu_q8k(const float *gate, const float *up, float *act_out, int8_t *qs,
                      int8_t *qs_cm, float *d, int16_t *bsums, int nblocks, hipStream_t st) {
    if (nblocks <= 0) return 0;
    hipLaunchKernelGGL(swiglu_q8k, dim3((nblocks + 3) / 4), dim3(256), 0, st, gate, up, act_out,
                       qs, qs_cm, d, bsums, nblocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_silu_mul(const float *gate, const float *up, float *out, int n, hipStream_t st) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(silu_mul_f32, dim3((n + 255) / 256), dim3(256), 0, st, gate, up, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
