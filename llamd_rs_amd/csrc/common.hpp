// common.hpp -- shared constants and device helpers for the gfx950 kernels.
//
// Everything here is compiled with -ffp-contract=off: the reference path is
// Rust, which never fuses a*b+c, and the kernels reproduce its float
// operations one for one where bit-exactness is claimed. Where an FMA is
// wanted (it never is on a bit-exact path) it is written as fmaf explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace llamd {

constexpr int QK_K = 256;              // k-quant super-block (ggml QK_K)
constexpr int QK8_0 = 32;              // Q8_0 block
constexpr int Q6K_BLOCK_BYTES = 210;   // block_q6_K
constexpr int Q8_0_BLOCK_BYTES = 34;   // block_q8_0
constexpr int WAVE = 64;               // CDNA wavefront
constexpr int TILE_ROWS = 16;          // rows per MFMA tile
// One (16-row tile, 256-weight block) segment of the tiled Q6_K layout:
// 16 rows x 210 bytes, re-ordered so each of the 64 lanes owns 48 contiguous
// bytes of 6-bit codes plus its scales (see host/layout.cpp).
constexpr int SEG_BYTES = TILE_ROWS * Q6K_BLOCK_BYTES;  // 3360
constexpr int SEG_PART = 1024;                          // 64 lanes x 16 B
constexpr int SEG_SC = 3 * SEG_PART;                    // 3072
constexpr int SEG_D = SEG_SC + 256;                     // 3328
constexpr float WEIGHT_SUM_FLOOR = 6.103515625e-5f;     // 2^-14, moe.rs:50

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    // v_cvt_f32_f16 is exact for every binary16 code (f16 denormals are kept).
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ int shfl_xor_i(int v, int mask) { return __shfl_xor(v, mask, WAVE); }
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, WAVE); }
__device__ __forceinline__ double shfl_xor_d(double v, int mask) { return __shfl_xor(v, mask, WAVE); }

// Wave-wide sum in double (order-free enough for a bound; never used where a
// bit-exact float result is claimed).
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_d(v, m);
    return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
    return v;
}

}  // namespace llamd
