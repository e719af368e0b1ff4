// q6k_tile.hpp -- the per-block building blocks of the Q6_K x Q8_K kernels
// (q6k_mv.hip explains the scheme): operand unpacking from the tiled layout,
// the masked-activation MFMAs of one 256-weight block and its ordered float
// terms (dot.rs:190-193), and the register loads of one block.
#pragma once

#include "common.hpp"

namespace llamd {

constexpr long NEG32_BYTES = (long)0xE0E0E0E0E0E0E0E0ull;  // int8 -32 in every byte


// 6-bit codes of class c for this lane's 8 weights (B operand, K = 8s..8s+7)
// from the nibble words and high-bit words of the tiled layout.
__device__ __forceinline__ long unpack_codes(const uint32_t nib[8], const uint32_t hb[4], int c) {
    const uint32_t N = nib[c];
    const uint32_t H = hb[c >> 1];
    uint32_t b0, b1;
    if ((c & 1) == 0) {
        b0 = (N & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
        b1 = ((N >> 4) & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
    } else {
        b0 = (N & 0x0F0F0F0Fu) | (H & 0x30303030u);
        b1 = ((N >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
    }
    return (long)((uint64_t)b0 | ((uint64_t)b1 << 32));
}

// The A operand (activation mask) of lane L = n + 16 s for class c holds, if
// s == n / 4 (the lane carries group j = n), the pair (a[16j + c],
// a[16j + c + 8]) in bytes 2 (j % 4) and 2 (j % 4) + 1 of its 8 bytes, and
// zeros otherwise. v_perm_b32 builds each dword in one instruction: the pair
// sits in byte (c & 3) of g[c >> 2] and of g[2 + (c >> 2)]; selector byte
// values 0..3 pick from the second operand, 4..7 from the first, 0x0C gives 0.
struct MaskSel {
    uint32_t s0, s1;   // selectors for A dword 0 / dword 1 with c & 3 == 0
    uint32_t inc0, inc1;  // added (c & 3) times for the other classes
};

__device__ __forceinline__ MaskSel mask_selectors(int n, bool valid) {
    // the pair lands in bytes 2 (j % 4) and 2 (j % 4) + 1 of the 8-byte operand
    const uint32_t pair = 0x0400u;              // (lo: sel 0, hi: sel 4)
    const uint32_t shift = 16u * (n & 1);
    const uint32_t placed = (pair << shift) | (0x0C0C0C0Cu & ~(0xFFFFu << shift));
    const uint32_t inc = 0x0101u << shift;
    MaskSel m;
    const bool lo = valid && !(n & 2), hi = valid && (n & 2);
    m.s0 = lo ? placed : 0x0C0C0C0Cu;
    m.s1 = hi ? placed : 0x0C0C0C0Cu;
    m.inc0 = lo ? inc : 0u;
    m.inc1 = hi ? inc : 0u;
    return m;
}

__device__ __forceinline__ long amask_perm(const uint32_t g[4], int c, const MaskSel &m) {
    const uint32_t lo = g[c >> 2], hi = g[2 + (c >> 2)];
    const uint32_t a0 = __builtin_amdgcn_perm(hi, lo, m.s0 + (uint32_t)(c & 3) * m.inc0);
    const uint32_t a1 = __builtin_amdgcn_perm(hi, lo, m.s1 + (uint32_t)(c & 3) * m.inc1);
    return (long)((uint64_t)a0 | ((uint64_t)a1 << 32));
}

struct BlockRegs {
    uint4 q0, q1, q2;
    uint32_t scw;
    uint16_t dh;
    uint4 g;
    float ad;
};

__device__ __forceinline__ void load_block(BlockRegs &r, const uint8_t *seg, const int8_t *aq,
                                           const float *ad, int b, int lane, int n) {
    r.q0 = *(const uint4 *)(seg + 16 * lane);
    r.q1 = *(const uint4 *)(seg + SEG_PART + 16 * lane);
    r.q2 = *(const uint4 *)(seg + 2 * SEG_PART + 16 * lane);
    r.scw = *(const uint32_t *)(seg + SEG_SC + 4 * lane);
    r.dh = *(const uint16_t *)(seg + SEG_D + 2 * n);
    r.g = *(const uint4 *)(aq + (size_t)b * QK_K + 16 * n);
    r.ad = ad[b];
}

// Butterfly over the 4 lanes of a row (n, n+16, n+32, n+48) with gfx950's
// half-wave swaps. permlane32_swap(a, b) leaves a = [a_lo, b_lo] and
// b = [a_hi, b_hi] (halves of 32 lanes), so a + b sums class c over lanes L,
// L^32 in the low half and class c+4 in the high half; permlane16_swap does
// the same between 16-lane rows. After both steps lane (n, s) holds the full
// aux32 of classes 2s and 2s+1.
__device__ __forceinline__ void reduce_classes(const int acc[8], int &c_even, int &c_odd) {
    int r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const auto sw = __builtin_amdgcn_permlane32_swap(acc[k], acc[k + 4], false, false);
        r[k] = (int)sw[0] + (int)sw[1];  // low half: class k, high half: class k + 4
    }
    const auto s0 = __builtin_amdgcn_permlane16_swap(r[0], r[2], false, false);
    const auto s1 = __builtin_amdgcn_permlane16_swap(r[1], r[3], false, false);
    c_even = (int)s0[0] + (int)s0[1];  // rows 0..3: classes 0, 2, 4, 6
    c_odd = (int)s1[0] + (int)s1[1];   // rows 0..3: classes 1, 3, 5, 7
}

// Per-block float terms (f16(d) * a.d) * aux32[c] for this lane's row and its
// two classes 2s, 2s+1: exactly the products the reference adds into
// sums[c] (dot.rs:190-193).
__device__ __forceinline__ void block_terms(const BlockRegs &r, const MaskSel &ms, float &t_even,
                                            float &t_odd) {
    const uint32_t nib[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t hb[4] = {r.q2.x, r.q2.y, r.q2.z, r.q2.w};
    const uint32_t g[4] = {r.g.x, r.g.y, r.g.z, r.g.w};
    const v4i zero = {0, 0, 0, 0};
    long am[8];
    v4i kc[8], d[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        am[c] = amask_perm(g, c, ms);
        kc[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(am[c], NEG32_BYTES, zero, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c)
        d[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(am[c], unpack_codes(nib, hb, c), kc[c], 0, 0, 0);
    // int8 scales of the lane's 4 groups; 24-bit multiplies run at full rate
    const int sc0 = __builtin_amdgcn_sbfe(r.scw, 0, 8), sc1 = __builtin_amdgcn_sbfe(r.scw, 8, 8);
    const int sc2 = __builtin_amdgcn_sbfe(r.scw, 16, 8), sc3 = __builtin_amdgcn_sbfe(r.scw, 24, 8);
    int acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        int v = __mul24(sc0, d[c][0]);
        v = __mul24(sc1, d[c][1]) + v;
        v = __mul24(sc2, d[c][2]) + v;
        acc[c] = __mul24(sc3, d[c][3]) + v;
    }
    int ae, ao;
    reduce_classes(acc, ae, ao);
    const float dd = f16_bits_to_f32(r.dh) * r.ad;
    t_even = dd * (float)ae;
    t_odd = dd * (float)ao;
}

template <int KS>
__device__ __forceinline__ void consume_terms(int b, float te, float to, float &se, float &so,
                                              float (*terms)[TILE_ROWS][8], int n, int s) {
    if constexpr (KS == 1) {
        se = se + te;
        so = so + to;
    } else {
        if (b < 16) {
            terms[b][n][2 * s] = te;
            terms[b][n][2 * s + 1] = to;
        }
    }
}

constexpr int DOWN_ACT_BLOCKS = 8;  // f32 activations quantized in LDS: n_ff <= 2048

__device__ __forceinline__ void load_weights(BlockRegs &r, const uint8_t *seg, int lane, int n) {
    r.q0 = *(const uint4 *)(seg + 16 * lane);
    r.q1 = *(const uint4 *)(seg + SEG_PART + 16 * lane);
    r.q2 = *(const uint4 *)(seg + 2 * SEG_PART + 16 * lane);
    r.scw = *(const uint32_t *)(seg + SEG_SC + 4 * lane);
    r.dh = *(const uint16_t *)(seg + SEG_D + 2 * n);
}

}  // namespace llamd
