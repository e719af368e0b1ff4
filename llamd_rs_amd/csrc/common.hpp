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

// Correctly rounded f32 square root (what Rust's f32::sqrt returns). The
// hardware estimate is within an ulp or so; the result is then moved to the
// neighbour whose rounding interval holds sqrt(t), decided exactly in double:
// a midpoint between two floats has at most 25 significant bits, so its
// square is exact in double and t < m^2 is an exact comparison (t is never
// equal to the square of such a midpoint).
__device__ __forceinline__ float sqrt_rn(float t) {
    float s = __builtin_sqrtf(t);
    if (!(t > 0.0f) || __builtin_isinf(t)) return s;  // 0, -0, NaN, negatives, +inf
    const double td = (double)t;
    for (int k = 0; k < 4; ++k) {
        const float dn = __uint_as_float(__float_as_uint(s) - 1u);
        const double lo = ((double)s + (double)dn) * 0.5;
        if (s > 0.0f && td < lo * lo) { s = dn; continue; }
        const float up = __uint_as_float(__float_as_uint(s) + 1u);
        const double hi = ((double)s + (double)up) * 0.5;
        if (td > hi * hi) { s = up; continue; }
        break;
    }
    return s;
}

__device__ __forceinline__ int shfl_xor_i(int v, int mask) { return __shfl_xor(v, mask, WAVE); }
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, WAVE); }
__device__ __forceinline__ double shfl_xor_d(double v, int mask) { return __shfl_xor(v, mask, WAVE); }

// ---- DPP wave reductions -------------------------------------------------
// __shfl_xor is a ds_bpermute through the LDS crossbar (~100+ cycles each);
// these use the gfx9 DPP lane patterns instead, which are ordinary VALU ops:
// xor 1 and xor 2 inside quads, half-row and row mirrors, then row_bcast:15
// and row_bcast:31 carry rows 0 and 2 into rows 1 and 3 and rows 0-1 into
// rows 2-3. Lane 63 ends with the reduction of all 64 lanes; readlane(63)
// broadcasts it. The combining op must be associative and commutative, and
// disabled lanes see the identity `idn`.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
constexpr int DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118;
constexpr int DPP_WAVE_SHR1 = 0x138;

template <int CTRL, int ROWS = 0xF, bool BOUND = false>
__device__ __forceinline__ int dpp(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, BOUND);
}
template <int CTRL, int ROWS = 0xF, bool BOUND = false>
__device__ __forceinline__ float dpp(float old, float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, BOUND));
}
template <int CTRL, int ROWS = 0xF, bool BOUND = false>
__device__ __forceinline__ double dpp(double old, double v) {
    const long long o = __double_as_longlong(old), x = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp((int)o, (int)x, CTRL, ROWS, 0xF, BOUND);
    const int hi = __builtin_amdgcn_update_dpp((int)(o >> 32), (int)(x >> 32), CTRL, ROWS, 0xF, BOUND);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ int readlane63(int v) { return __builtin_amdgcn_readlane(v, 63); }
__device__ __forceinline__ float readlane63(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ double readlane63(double v) {
    const long long x = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)x, 63), hi = __builtin_amdgcn_readlane((int)(x >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Reduce with op over the wave; every lane gets the result.
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, T idn, Op op) {
    v = op(v, dpp<DPP_XOR1>(idn, v));
    v = op(v, dpp<DPP_XOR2>(idn, v));
    v = op(v, dpp<DPP_HALF_MIRROR>(idn, v));
    v = op(v, dpp<DPP_MIRROR>(idn, v));
    v = op(v, dpp<DPP_BCAST15, 0xA>(idn, v));
    v = op(v, dpp<DPP_BCAST31, 0xC>(idn, v));
    return readlane63(v);
}

// Wave-wide (value, index) arg-max: larger value, ties to the lower index.
// Branch-free steps (selects, no exec-mask juggling).
template <class T>
__device__ __forceinline__ void argmax_step(T &v, int &i, T ov, int oi) {
    const bool take = (ov > v) | ((ov == v) & (oi < i));
    v = take ? ov : v;
    i = take ? oi : i;
}

template <class T>
__device__ __forceinline__ void wave_argmax(T &v, int &i, T vidn) {
    argmax_step(v, i, dpp<DPP_XOR1>(vidn, v), dpp<DPP_XOR1>(0x7FFFFFFF, i));
    argmax_step(v, i, dpp<DPP_XOR2>(vidn, v), dpp<DPP_XOR2>(0x7FFFFFFF, i));
    argmax_step(v, i, dpp<DPP_HALF_MIRROR>(vidn, v), dpp<DPP_HALF_MIRROR>(0x7FFFFFFF, i));
    argmax_step(v, i, dpp<DPP_MIRROR>(vidn, v), dpp<DPP_MIRROR>(0x7FFFFFFF, i));
    argmax_step(v, i, dpp<DPP_BCAST15, 0xA>(vidn, v), dpp<DPP_BCAST15, 0xA>(0x7FFFFFFF, i));
    argmax_step(v, i, dpp<DPP_BCAST31, 0xC>(vidn, v), dpp<DPP_BCAST31, 0xC>(0x7FFFFFFF, i));
    v = readlane63(v);
    i = readlane63(i);
}

// Inclusive prefix sum over the wave (lane order).
__device__ __forceinline__ double wave_inclusive_sum(double v) {
    v += dpp<DPP_ROW_SHR1, 0xF, true>(0.0, v);
    v += dpp<DPP_ROW_SHR2, 0xF, true>(0.0, v);
    v += dpp<DPP_ROW_SHR4, 0xF, true>(0.0, v);
    v += dpp<DPP_ROW_SHR8, 0xF, true>(0.0, v);
    v += dpp<DPP_BCAST15, 0xA>(0.0, v);
    v += dpp<DPP_BCAST31, 0xC>(0.0, v);
    return v;
}

// Inclusive prefix sum of ints over the wave (lane order).
__device__ __forceinline__ int wave_incl_sum_i(int v) {
    v += dpp<DPP_ROW_SHR1, 0xF, true>(0, v);
    v += dpp<DPP_ROW_SHR2, 0xF, true>(0, v);
    v += dpp<DPP_ROW_SHR4, 0xF, true>(0, v);
    v += dpp<DPP_ROW_SHR8, 0xF, true>(0, v);
    v += dpp<DPP_BCAST15, 0xA>(0, v);
    v += dpp<DPP_BCAST31, 0xC>(0, v);
    return v;
}

// Wave-wide sum in double (order-free enough for a bound; never used where a
// bit-exact float result is claimed).
__device__ __forceinline__ double wave_sum_d(double v) {
    return wave_reduce(v, 0.0, [](double a, double b) { return a + b; });
}

__device__ __forceinline__ float wave_sum_f(float v) {
    return wave_reduce(v, 0.0f, [](float a, float b) { return a + b; });
}

}  // namespace llamd
