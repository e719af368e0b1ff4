// q6k_mv.hip -- Q6_K x Q8_K matrix-vector kernels for gfx950 (CDNA4, wave64).
//
// WHAT IS COMPUTED. For every row r, exactly the reference's
// dot_q6k_q8k (crates/llamd-quant/src/dot.rs:138-196): per 256-weight block
// the eight integer lane sums
//     aux32[c] = sum over groups j of sc[j] * sum_{e in j, e mod 8 == c} (q_e - 32) * a_e
// then the ordered float epilogue sums[c] += (f16(d) * a.d) * aux32[c]
// (no FMA), block after block, and finally sums[0] + ... + sums[7] in order.
// The integer part is exact whatever the association, and the float part is
// performed in the reference's order, so the result is BIT-IDENTICAL to the
// CPU path, not merely within REDUCTION.
//
// HOW, ON CDNA4. The integer part runs on the matrix cores. One wave owns a
// 16-row tile; per block and per class c it issues
//     D = v_mfma_i32_16x16x32_i8(A_c, B_c, K_c)
// with
//   B_c[k][n] = code of weight e = 8k + c of row n   (K = the 32 class-c weights,
//               unpacked in registers from the tiled layout, host/layout.cpp)
//   A_c[j][k] = a_e if k / 2 == j else 0             (M = the 16 scale groups:
//               weight e = 8k + c lies in group e / 16 = k / 2)
//   K_c       = A_c x (-32)                           (the code offset, from a
//               second MFMA against a constant, once per block and class)
// so D[j][n] = sum_{e in group j, class c} (q_e - 32) a_e for all 16 groups at
// once. Each lane then holds 4 groups of one row and applies their int8 scales
// with 4 integer multiply-adds; a cross-lane add over the 4 lanes of a row
// gives aux32[c]. HBM traffic is the 210 bytes per 256 weights of the format
// plus the activation, read with three coalesced 16-byte loads per lane per
// block; the 16x redundancy of the masked MFMA costs nothing because the
// matrix cores are >50x faster than HBM can feed this op.
#include "common.hpp"
#include "launch.hpp"

namespace llamd {
namespace {

constexpr long NEG32_BYTES = (long)0xE0E0E0E0E0E0E0E0ull;  // int8 -32 in every byte

struct MvParams {
    const uint8_t *w;         // tiled Q6_K base
    size_t expert_stride;     // bytes between experts' tiled matrices
    const int32_t *ids;       // slot -> expert (nullptr: slot -> expert 0)
    const int8_t *aq;         // Q8_K quants, [n_act][blocks*256]
    const float *ad;          // Q8_K scales, [n_act][blocks]
    float *y;                 // [n_slots][rows]
    int rows, tiles, blocks, n_slots;
    int act_per_slot;         // 1: slot i uses activation i; 0: all use activation 0
};

__device__ __forceinline__ long make_amask(const uint32_t g[4], int c, int n, bool valid) {
    const uint32_t lo = (g[c >> 2] >> (8 * (c & 3))) & 0xFFu;
    const uint32_t hi = (g[2 + (c >> 2)] >> (8 * (c & 3))) & 0xFFu;
    const uint32_t placed = (lo | (hi << 8)) << (16 * (n & 1));
    const uint32_t a0 = (valid && !(n & 2)) ? placed : 0u;
    const uint32_t a1 = (valid && (n & 2)) ? placed : 0u;
    return (long)((uint64_t)a0 | ((uint64_t)a1 << 32));
}

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

// One wave = one (slot, tile) item. 4 waves per workgroup.
__global__ __launch_bounds__(256) void q6k_mv_b1(MvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int item = blockIdx.x * 4 + wave;
    if (item >= p.n_slots * p.tiles) return;  // whole wave exits together
    const int slot = item / p.tiles;
    const int t = item - slot * p.tiles;
    const int n = lane & 15;
    const int s = lane >> 4;
    const bool valid = (n >> 2) == s;  // this lane carries the mask of group n

    const int expert = p.ids ? p.ids[slot] : 0;
    const uint8_t *seg = p.w + (size_t)expert * p.expert_stride + (size_t)t * p.blocks * SEG_BYTES;
    const int act = p.act_per_slot ? slot : 0;
    const int8_t *aq = p.aq + (size_t)act * p.blocks * QK_K;
    const float *ad = p.ad + (size_t)act * p.blocks;

    float sums[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) sums[c] = 0.0f;

    for (int b = 0; b < p.blocks; ++b, seg += SEG_BYTES) {
        const uint4 q0 = *(const uint4 *)(seg + 16 * lane);
        const uint4 q1 = *(const uint4 *)(seg + SEG_PART + 16 * lane);
        const uint4 q2 = *(const uint4 *)(seg + 2 * SEG_PART + 16 * lane);
        const uint32_t scw = *(const uint32_t *)(seg + SEG_SC + 4 * lane);
        const uint16_t dh = *(const uint16_t *)(seg + SEG_D + 2 * n);
        const uint4 gv = *(const uint4 *)(aq + (size_t)b * QK_K + 16 * n);
        const float adb = ad[b];

        const uint32_t nib[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[4] = {q2.x, q2.y, q2.z, q2.w};
        const uint32_t g[4] = {gv.x, gv.y, gv.z, gv.w};
        const int sc0 = (int8_t)(scw & 0xFF), sc1 = (int8_t)((scw >> 8) & 0xFF);
        const int sc2 = (int8_t)((scw >> 16) & 0xFF), sc3 = (int8_t)(scw >> 24);

        int acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const long am = make_amask(g, c, n, valid);
            const v4i zero = {0, 0, 0, 0};
            const v4i kc = __builtin_amdgcn_mfma_i32_16x16x32_i8(am, NEG32_BYTES, zero, 0, 0, 0);
            const long bw = unpack_codes(nib, hb, c);
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(am, bw, kc, 0, 0, 0);
            acc[c] = sc0 * d[0] + sc1 * d[1] + sc2 * d[2] + sc3 * d[3];
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            acc[c] += shfl_xor_i(acc[c], 16);
            acc[c] += shfl_xor_i(acc[c], 32);
        }
        const float dd = f16_bits_to_f32(dh) * adb;
#pragma unroll
        for (int c = 0; c < 8; ++c) sums[c] = sums[c] + dd * (float)acc[c];
    }

    if (s == 0) {
        const int row = t * TILE_ROWS + n;
        if (row < p.rows) {
            float tot = -0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) tot = tot + sums[c];
            p.y[(size_t)slot * p.rows + row] = tot;
        }
    }
}

// Device dequantization of the tiled layout back to f32, element order of
// crates/llamd-quant/src/lib.rs:181-226 (d * sc first, then * (q - 32)).
// One wave per segment; out is [rows][blocks*256].
__global__ __launch_bounds__(256) void q6k_dequant_tiled(const uint8_t *w, int rows, int tiles,
                                                         int blocks, float *out) {
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= tiles * blocks) return;
    const int t = item / blocks, b = item - t * blocks;
    const uint8_t *seg = w + (size_t)item * SEG_BYTES;
    const int n = lane & 15, s = lane >> 4;
    const int row = t * TILE_ROWS + n;
    const uint4 q0 = *(const uint4 *)(seg + 16 * lane);
    const uint4 q1 = *(const uint4 *)(seg + SEG_PART + 16 * lane);
    const uint4 q2 = *(const uint4 *)(seg + 2 * SEG_PART + 16 * lane);
    const uint32_t scw = *(const uint32_t *)(seg + SEG_SC + 4 * lane);
    const float d = f16_bits_to_f32(*(const uint16_t *)(seg + SEG_D + 2 * n));
    const uint32_t nib[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const uint32_t hb[4] = {q2.x, q2.y, q2.z, q2.w};
    if (row >= rows) return;
    float *o = out + (size_t)row * blocks * QK_K + (size_t)b * QK_K;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint64_t codes = (uint64_t)unpack_codes(nib, hb, c);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int m = 8 * s + k;           // class element index
            const int e = 8 * m + c;           // weight index in the block
            const int grp = e >> 4;            // = 4 s + k / 2
            const int sc = (int8_t)((scw >> (8 * (grp - 4 * s))) & 0xFF);
            const int q = (int)((codes >> (8 * k)) & 0x3F) - 32;
            o[e] = d * (float)sc * (float)q;
        }
    }
}


// ---- batched / expert-grouped: up to 16 tokens per MFMA ---------------------
//
// For many tokens against one weight tile, the scale is folded into the
// weights instead of into the masked activation: per class c,
//     w'_k = sc[group(k)] * (q_k - 32)  in [-4064, 4096]
// is split into two int8 digits w' = 64 * hi + lo (lo = w' & 63, hi = w' >> 6)
// and two MFMAs against the 16 tokens' class-c activations give
//     aux32[c] = 64 * (A_hi x B) + (A_lo x B)
// exactly, for 16 rows x 16 tokens at once. The float epilogue per (row,
// token) is the reference's, so every output is again bit-identical to
// dot_q6k_q8k on that token's activation.
//
// Work: one wave per (group g, 16-token sub-tile st, 16-row tile t). A group
// is one expert and a list of (activation index, output index) pairs; the LM
// head at batch 16 is one group of 16 tokens. Activations are read in the
// class-major order written by the quantize kernels (byte 32 c + m of each
// block holds weight 8 m + c).
struct BatchParams {
    const uint8_t *w;
    size_t expert_stride;
    const int32_t *grp_expert;   // [n_groups]
    const int32_t *grp_start;    // first pair of the group
    const int32_t *grp_count;    // pairs in the group
    const int32_t *sub_start;    // prefix sum of ceil(count/16) over groups
    const int32_t *pair_act;     // activation index of each pair (nullptr: identity)
    const int32_t *pair_out;     // output row of each pair (nullptr: identity)
    const int8_t *aq_cm;         // class-major Q8_K quants [n_act][blocks*256]
    const float *ad;             // [n_act][blocks]
    float *y;                    // y[pair_out * ldy + row]
    int ldy, rows, tiles, blocks, n_groups;
    int single_count;            // grp_expert == nullptr: one group, expert 0, this many pairs
};

__device__ __forceinline__ void fold_digits(uint64_t codes, uint32_t scw, long &lo8, long &hi8) {
    uint64_t lo = 0, hi = 0;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        const int q = (int)((codes >> (8 * kk)) & 0x3F) - 32;
        const int sc = (int8_t)((scw >> (8 * (kk >> 1))) & 0xFF);
        const int v = sc * q;
        lo |= (uint64_t)(v & 63) << (8 * kk);
        hi |= (uint64_t)((v >> 6) & 0xFF) << (8 * kk);
    }
    lo8 = (long)lo;
    hi8 = (long)hi;
}

__global__ __launch_bounds__(256) void q6k_mv_batched(BatchParams p) {
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int t = item % p.tiles;
    const int sub = item / p.tiles;
    int g = 0, st = sub, cnt, start = 0, expert = 0;
    if (p.grp_expert) {
        // find the group whose sub-tile range holds `sub` (sub_start has
        // n_groups + 1 entries)
        if (sub >= p.sub_start[p.n_groups]) return;
        int lo = 0, hi = p.n_groups;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (p.sub_start[mid] <= sub) lo = mid; else hi = mid;
        }
        g = lo;
        st = sub - p.sub_start[g];
        cnt = p.grp_count[g];
        start = p.grp_start[g];
        expert = p.grp_expert[g];
    } else {
        cnt = p.single_count;
        if (sub >= (cnt + 15) / 16) return;
    }
    const int n = lane & 15, s = lane >> 4;
    const int tok = 16 * st + n;               // this lane's token (B operand / output column)
    const bool tok_ok = tok < cnt;
    const int pair = start + (tok_ok ? tok : 0);
    const int act = p.pair_act ? p.pair_act[pair] : pair;
    const uint8_t *seg = p.w + (size_t)expert * p.expert_stride + (size_t)t * p.blocks * SEG_BYTES;
    const int8_t *aq = p.aq_cm + (size_t)act * p.blocks * QK_K;
    const float *ad = p.ad + (size_t)act * p.blocks;

    float sums[8][4];
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) sums[c][v] = 0.0f;

    for (int b = 0; b < p.blocks; ++b, seg += SEG_BYTES) {
        const uint4 q0 = *(const uint4 *)(seg + 16 * lane);
        const uint4 q1 = *(const uint4 *)(seg + SEG_PART + 16 * lane);
        const uint4 q2 = *(const uint4 *)(seg + 2 * SEG_PART + 16 * lane);
        const uint32_t scw = *(const uint32_t *)(seg + SEG_SC + 4 * lane);
        const uint32_t nib[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[4] = {q2.x, q2.y, q2.z, q2.w};
        // d of rows 4s..4s+3 (the D layout rows this lane holds) times this
        // lane's token scale
        const float adb = tok_ok ? ad[b] : 0.0f;
        float dd[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
            dd[v] = f16_bits_to_f32(*(const uint16_t *)(seg + SEG_D + 2 * (4 * s + v))) * adb;
        const int8_t *ab = aq + (size_t)b * QK_K + 8 * s;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const long bw = unpack_codes(nib, hb, c);
            long a_lo, a_hi;
            fold_digits((uint64_t)bw, scw, a_lo, a_hi);
            const long bact = tok_ok ? *(const long *)(ab + 32 * c) : 0;
            const v4i zero = {0, 0, 0, 0};
            const v4i dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, bact, zero, 0, 0, 0);
            const v4i dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, bact, zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int aux = dh[v] * 64 + dl[v];
                sums[c][v] = sums[c][v] + dd[v] * (float)aux;
            }
        }
    }
    if (tok_ok) {
        const int orow = p.pair_out ? p.pair_out[pair] : pair;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = t * TILE_ROWS + 4 * s + v;
            if (row < p.rows) {
                float tot = -0.0f;
#pragma unroll
                for (int c = 0; c < 8; ++c) tot = tot + sums[c][v];
                p.y[(size_t)orow * p.ldy + row] = tot;
            }
        }
    }
}

}  // namespace

int launch_q6k_mv_b1(const void *w, size_t expert_stride, const int32_t *ids, const int8_t *aq,
                     const float *ad, float *y, int rows, int blocks, int n_slots, int act_per_slot,
                     hipStream_t st) {
    MvParams p;
    p.w = (const uint8_t *)w;
    p.expert_stride = expert_stride;
    p.ids = ids;
    p.aq = aq;
    p.ad = ad;
    p.y = y;
    p.rows = rows;
    p.tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    p.blocks = blocks;
    p.n_slots = n_slots;
    p.act_per_slot = act_per_slot;
    const int items = p.tiles * n_slots;
    hipLaunchKernelGGL(q6k_mv_b1, dim3((items + 3) / 4), dim3(256), 0, st, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q6k_mv_batched(const void *w, size_t expert_stride, const int32_t *grp_expert,
                          const int32_t *grp_start, const int32_t *grp_count,
                          const int32_t *sub_start, const int32_t *pair_act,
                          const int32_t *pair_out, const int8_t *aq_cm, const float *ad, float *y,
                          int ldy, int rows, int blocks, int n_groups, int max_subtiles,
                          hipStream_t st) {
    BatchParams p;
    p.single_count = n_groups;  // only read when grp_expert == nullptr
    p.w = (const uint8_t *)w;
    p.expert_stride = expert_stride;
    p.grp_expert = grp_expert;
    p.grp_start = grp_start;
    p.grp_count = grp_count;
    p.sub_start = sub_start;
    p.pair_act = pair_act;
    p.pair_out = pair_out;
    p.aq_cm = aq_cm;
    p.ad = ad;
    p.y = y;
    p.ldy = ldy;
    p.rows = rows;
    p.tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    p.blocks = blocks;
    p.n_groups = n_groups;
    const long items = (long)p.tiles * max_subtiles;
    if (items <= 0) return 0;
    hipLaunchKernelGGL(q6k_mv_batched, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q6k_dequant(const void *w, int rows, int blocks, float *out, hipStream_t st) {
    const int tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    const int items = tiles * blocks;
    hipLaunchKernelGGL(q6k_dequant_tiled, dim3((items + 3) / 4), dim3(256), 0, st,
                       (const uint8_t *)w, rows, tiles, blocks, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
