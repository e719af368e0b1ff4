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
#include "q8k_wave.hpp"

namespace llamd {
namespace {

__global__ __launch_bounds__(256) void q8k_quantize(const float *x, int8_t *qs, float *d,
                                                    int16_t *bsums, int nblocks) {
    asm volatile("" ::"s"(x), "s"(qs), "s"(d), "s"(bsums), "s"(nblocks));
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const float4 xv = *(const float4 *)(x + (size_t)blk * QK_K + 4 * lane);
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    quantize_wave(v, lane, qs + (size_t)blk * QK_K, d + blk, bsums ? bsums + (size_t)blk * 16 : nullptr);
}

// Row r of x ([rows][blocks*256]) to the token-chunked layout, once for each
// of its `fan` slots: slot_of[r * fan + k], or slot r when slot_of is null.
__global__ __launch_bounds__(256) void q8k_quantize_chunks(const float *x, int rows, int blocks,
                                                           const int32_t *slot_of, int fan,
                                                           int8_t *cq, float *cd, int8_t *nq,
                                                           float *nd) {
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= rows * blocks) return;
    const int r = item / blocks, b = item - r * blocks;
    const float4 xv = *(const float4 *)(x + (size_t)item * QK_K + 4 * lane);
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    // lane k < fan holds the k-th slot, loaded beside x (one round trip,
    // not one per slot)
    const int my_slot = slot_of ? (lane < fan ? slot_of[(size_t)r * fan + lane] : -1) : r;
    int q[4];
    float dv;
    quantize_wave_q(v, lane, q, dv);
    // optionally the reference's natural layout too, row r at nq[r][blocks*256]
    if (nq) store_q8k(q, dv, lane, nq + (size_t)item * QK_K, nd + item, nullptr);
    const uint32_t dw = chunk_dword(q, lane);
    for (int k = 0; k < fan; ++k)
        store_chunk(dw, dv, lane, cq, cd, slot_of ? __builtin_amdgcn_readlane(my_slot, k) : r, b, blocks);
}

// act[i] = silu(gate[i]) * up[i], then Q8_K of act. Optionally stores act.
__global__ __launch_bounds__(256) void swiglu_q8k(const float *gate, const float *up, float *act_out,
                                                  int8_t *qs, float *d, int16_t *bsums, int nblocks) {
    __shared__ uint64_t tab[32];
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const size_t o = (size_t)blk * QK_K + 4 * lane;
    const float4 gv = *(const float4 *)(gate + o);
    const float4 uv = *(const float4 *)(up + o);
    expf_ref_tab_fill(tab);
    float v[4];
    v[0] = silu_ref(gv.x, tab) * uv.x;
    v[1] = silu_ref(gv.y, tab) * uv.y;
    v[2] = silu_ref(gv.z, tab) * uv.z;
    v[3] = silu_ref(gv.w, tab) * uv.w;
    if (act_out) *(float4 *)(act_out + o) = make_float4(v[0], v[1], v[2], v[3]);
    quantize_wave(v, lane, qs + (size_t)blk * QK_K, d + blk, bsums ? bsums + (size_t)blk * 16 : nullptr);
}

// The same for rows of pairs, written to the token-chunked layout at
// slot_of[row] (the expert-sorted position of each pair).
__global__ __launch_bounds__(256) void swiglu_q8k_chunks(const float *gate, const float *up,
                                                         int rows, int blocks,
                                                         const int32_t *slot_of, int8_t *cq,
                                                         float *cd) {
    __shared__ uint64_t tab[32];
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= rows * blocks) return;
    const int r = item / blocks, b = item - r * blocks;
    const size_t o = (size_t)item * QK_K + 4 * lane;
    const int slot = slot_of[r];  // loaded with the operands, not after the math
    const float4 gv = *(const float4 *)(gate + o);
    const float4 uv = *(const float4 *)(up + o);
    expf_ref_tab_fill(tab);
    const float v[4] = {silu_ref(gv.x, tab) * uv.x, silu_ref(gv.y, tab) * uv.y,
                        silu_ref(gv.z, tab) * uv.z, silu_ref(gv.w, tab) * uv.w};
    int q[4];
    float dv;
    quantize_wave_q(v, lane, q, dv);
    store_chunk(chunk_dword(q, lane), dv, lane, cq, cd, slot, b, blocks);
}

__global__ __launch_bounds__(256) void silu_mul_f32(const float *gate, const float *up, float *out, int n) {
    __shared__ uint64_t tab[32];
    const int i = blockIdx.x * 256 + threadIdx.x;
    expf_ref_tab_fill(tab);
    if (i < n) out[i] = silu_ref(gate[i], tab) * up[i];
}

// Plain grid-stride copy (16-byte vectors), the calibration kernel for the
// HBM traffic counters: it reads and writes exactly n16 * 16 bytes.
__global__ __launch_bounds__(256) void copy_calibration(uint4 *dst, const uint4 *src, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// Read-only pass over n16 16-byte words (four independent loads in flight
// per thread), the launch-cost reference for short kernels: with n16 = 0 it
// is an empty kernel. The sink store never happens in practice; it keeps the
// loads.
__global__ __launch_bounds__(256) void read_calibration(const uint4 *src, size_t n16, uint32_t *sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        acc ^= a.x ^ b.y ^ c.z ^ d.w ^ a.w ^ b.x ^ c.y ^ d.z;
    }
    for (; i < n16; i += stride) acc ^= src[i].x ^ src[i].w;
    if (acc == 0x9E3779B9u && sink) sink[0] = acc;
}

}  // namespace

int launch_read_calibration(const void *src, size_t bytes, int grid, hipStream_t st) {
    if (bytes % 16 || grid < 1) return -1;
    hipLaunchKernelGGL(read_calibration, dim3(grid), dim3(256), 0, st, (const uint4 *)src, bytes / 16,
                       nullptr);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_copy_calibration(void *dst, const void *src, size_t bytes, hipStream_t st) {
    if (bytes % 16) return -1;
    hipLaunchKernelGGL(copy_calibration, dim3(4096), dim3(256), 0, st, (uint4 *)dst,
                       (const uint4 *)src, bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q8k_quantize(const float *x, int8_t *qs, float *d, int16_t *bsums, int nblocks,
                        hipStream_t st) {
    if (nblocks <= 0) return 0;
    hipLaunchKernelGGL(q8k_quantize, dim3((nblocks + 3) / 4), dim3(256), 0, st, x, qs, d, bsums,
                       nblocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q8k_quantize_chunks(const float *x, int rows, int blocks, const int32_t *slot_of,
                               int fan, int8_t *cq, float *cd, hipStream_t st, int8_t *nq,
                               float *nd) {
    if (rows <= 0 || blocks <= 0) return 0;
    if (fan < 1 || fan > WAVE || (!nq) != (!nd)) return -1;
    hipLaunchKernelGGL(q8k_quantize_chunks, dim3((rows * blocks + 3) / 4), dim3(256), 0, st, x,
                       rows, blocks, slot_of, fan, cq, cd, nq, nd);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_swiglu_q8k(const float *gate, const float *up, float *act_out, int8_t *qs, float *d,
                      int16_t *bsums, int nblocks, hipStream_t st) {
    if (nblocks <= 0) return 0;
    hipLaunchKernelGGL(swiglu_q8k, dim3((nblocks + 3) / 4), dim3(256), 0, st, gate, up, act_out,
                       qs, d, bsums, nblocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_swiglu_q8k_chunks(const float *gate, const float *up, int rows, int blocks,
                             const int32_t *slot_of, int8_t *cq, float *cd, hipStream_t st) {
    if (rows <= 0 || blocks <= 0) return 0;
    hipLaunchKernelGGL(swiglu_q8k_chunks, dim3((rows * blocks + 3) / 4), dim3(256), 0, st, gate,
                       up, rows, blocks, slot_of, cq, cd);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_silu_mul(const float *gate, const float *up, float *out, int n, hipStream_t st) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(silu_mul_f32, dim3((n + 255) / 256), dim3(256), 0, st, gate, up, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
