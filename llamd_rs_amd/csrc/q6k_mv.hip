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
#include "expf_ref.h"
#include "launch.hpp"
#include "q6k_tile.hpp"
#include "q8k_wave.hpp"
#include "route.hpp"

namespace llamd {
namespace {

// Up to three weight matrices ("segments") share one launch and one
// activation set: gate and up of the same experts, or Q, K and V. Items are
// numbered segment by segment; within a segment, item = slot * tiles + tile.
struct MvSeg {
    const uint8_t *w;         // tiled Q6_K base (expert 0)
    float *y;                 // [n_slots][rows]
    int rows, tiles, first;   // first: index of the segment's first item
};

// The fields every launch reads come first and together, so the kernel's
// prologue fetches them from the kernarg segment in one go before the first
// weight load; the other segments, the routing prologue's and the arg-max
// fields follow.
struct MvParams {
    MvSeg seg0;               // 32 B
    const int8_t *aq;         // Q8_K quants, [n_act][blocks*256]
    const float *ad;          // Q8_K scales, [n_act][blocks]
    const int32_t *ids;       // slot -> expert (nullptr: slot -> expert 0)
    size_t expert_stride;     // bytes between experts' tiled matrices
    int items, blocks;        // items over all segments; 256-blocks per row
    int n_slots, act_per_slot;  // > 0: slot i uses activation i / act_per_slot; 0: activation 0
    MvSeg seg1, seg2;
    int n_seg;
    // routing prologue (ROUTE): wave 0 of every workgroup routes on the exact
    // router logits and takes slot -> expert from its own selection;
    // workgroup 0 publishes ids / weights for the kernels after it
    const float *route_l;     // [n_expert]
    int n_expert, n_used;
    int32_t *ids_out;
    float *w_out;
    int *stats;               // [2] calls (+1 each, both counters)
    // optional per-tile arg-max candidates (one segment): [n_slots][tiles]
    float *amax_v;
    int *amax_i;
    // optional in-kernel clock (llamd_hip_kernel_clock): the launch's record
    unsigned long long *clk;
};

// In-kernel clock: wave w (flat index over the grid) stores its start at
// clk[w] and its end at clk[CLOCK_WAVES + w], s_memrealtime ticks, with plain
// vector stores (one writer per word: no contention, no atomics). The start
// is read first thing and both are stored on every exit of the kernel, so
// the record's pointer is not needed before the kernel's first loads.
constexpr int CLOCK_WAVES = 1024;
template <int WAVES_PER_WG>
struct ClockEnd {
    unsigned long long *r;  // the launch's record (null: no clock)
    unsigned long long t0;
    __device__ ~ClockEnd() {
        const int w = (int)(blockIdx.x * WAVES_PER_WG + (threadIdx.x >> 6));
        if (r && w < CLOCK_WAVES && (threadIdx.x & 63) == 0) {
            r[w] = t0;
            r[CLOCK_WAVES + w] = __builtin_amdgcn_s_memrealtime();
        }
    }
};

// One (slot, 16-row tile) item per KS waves of a 4-wave (KS = 8: 8-wave) workgroup; wave kc of
// the item takes blocks [kc*bpc, (kc+1)*bpc) with the next block's loads in
// flight while the current one is computed. With KS > 1 the per-block terms
// meet in LDS and are folded in block order -- the same additions in the same
// order as a single wave walking every block, so splitting K changes the
// latency, never the bits.
//
// The fields the first loads depend on come as leading scalar arguments,
// which gfx950 preloads into SGPRs at dispatch (kernarg preload): the first
// weight and activation loads issue without waiting for the kernarg segment.
//
// PX is MvParams, or MvLite for the plain matvec (one segment, no routing
// prologue, no arg-max): a 40-byte block instead of 216 bytes, since the
// size of the kernarg segment shows in the launch cost of a small matvec.
struct MvLite {
    float *y;
    size_t expert_stride;
    unsigned long long *clk;
    int rows, n_slots;
};
__device__ __forceinline__ MvParams expand_params(const MvParams &p) { return p; }
__device__ __forceinline__ MvParams expand_params(const MvLite &l) {
    MvParams p = {};
    p.seg0.y = l.y;
    p.seg0.rows = l.rows;
    p.expert_stride = l.expert_stride;
    p.clk = l.clk;
    p.n_slots = l.n_slots;
    p.n_seg = 1;
    return p;
}

template <int KS, bool ROUTE = false, int NSEG = 1, bool AMAX = false, class PX = MvParams>
__global__ __launch_bounds__(KS > 4 ? 64 * KS : 256) void q6k_mv_b1(
    const uint8_t *w0, const int8_t *aq0, const float *ad0, const int32_t *ids0, int blocks0,
    int tiles0, int items0, int act_per_slot0, PX px) {
    const unsigned long long t_start = __builtin_amdgcn_s_memrealtime();
    MvParams p = expand_params(px);
    p.seg0.w = w0;
    p.aq = aq0;
    p.ad = ad0;
    p.ids = ids0;
    p.blocks = blocks0;
    p.seg0.tiles = tiles0;
    p.items = items0;
    p.act_per_slot = act_per_slot0;
    constexpr int IPW = KS >= 4 ? 1 : 4 / KS;   // items per workgroup
    constexpr int MAXB = 16;                    // blocks per row held in LDS (KS > 1)
    __shared__ float terms[KS > 1 ? IPW : 1][KS > 1 ? MAXB : 1][TILE_ROWS][8];
    const int lane = threadIdx.x & 63;
    // the parameter block's fields that the item's segment and the weight
    // address need, fetched in one batch up front (not one dependent scalar
    // load after another)
    if constexpr (NSEG > 1)
        asm volatile("" ::"s"(p.seg1.w), "s"(p.seg1.first), "s"(p.seg1.tiles), "s"(p.seg2.w),
                     "s"(p.seg2.first), "s"(p.seg2.tiles), "s"(p.expert_stride), "s"(p.seg0.y),
                     "s"(p.seg0.rows));
    else
        asm volatile("" ::"s"(p.expert_stride), "s"(p.seg0.y), "s"(p.seg0.rows));
    const ClockEnd<(KS > 4 ? KS : 4)> clock_end{p.clk, t_start};
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int kc = wave % KS;
    const int local = wave / KS;
    const int item = blockIdx.x * IPW + local;
    const bool live = item < p.items;
    // the item's segment, chosen with scalar selects (no indexed kernarg load)
    // field by field (a whole-struct select becomes an indexed stack copy)
    MvSeg sgm = p.seg0;
    sgm.first = 0;  // segment 0 always starts the item numbering
    if constexpr (NSEG > 1) {
        const bool in1 = item >= px.seg1.first;
        const bool in2 = NSEG > 2 && item >= px.seg2.first;
        sgm.w = in2 ? px.seg2.w : in1 ? px.seg1.w : sgm.w;
        sgm.y = in2 ? px.seg2.y : in1 ? px.seg1.y : sgm.y;
        sgm.rows = in2 ? px.seg2.rows : in1 ? px.seg1.rows : sgm.rows;
        sgm.tiles = in2 ? px.seg2.tiles : in1 ? px.seg1.tiles : sgm.tiles;
        sgm.first = in2 ? px.seg2.first : in1 ? px.seg1.first : 0;
    }
    const int pos = item - sgm.first;
    const int slot = live ? pos / sgm.tiles : 0;
    const int t = live ? pos - slot * sgm.tiles : 0;
    const int n = lane & 15;
    const int s = lane >> 4;
    const MaskSel msel = mask_selectors(n, (n >> 2) == s);  // lane carries group n's mask

    int expert;
    if constexpr (ROUTE) {
        // wave 0 routes; the workgroup's other waves wait for its choice
        __shared__ RouteLds rsh;
        if (wave == 0) {
            float l[RW];
#pragma unroll
            for (int j = 0; j < RW; ++j) {
                const int i = lane + WAVE * j;
                l[j] = i < p.n_expert ? p.route_l[i] : 0.0f;
            }
            const bool writer = blockIdx.x == 0;
            route_finish(l, p.n_expert, p.n_used, true, rsh, writer ? p.ids_out : nullptr,
                         writer ? p.w_out : nullptr, nullptr);
            if (writer && lane == 0 && p.stats) {
                p.stats[0] += 1;
                p.stats[1] += 1;
            }
        }
        __syncthreads();
        expert = live ? rsh.sorted[slot] : 0;
    } else {
        expert = (live && p.ids) ? p.ids[slot] : 0;
    }
    const int act = p.act_per_slot ? slot / p.act_per_slot : 0;
    const int8_t *aq = p.aq + (size_t)act * p.blocks * QK_K;
    const float *ad = p.ad + (size_t)act * p.blocks;
    // (without ids, expert 0: no kernarg-segment field on the way to the first load)
    const uint8_t *wexp = (ROUTE || p.ids) ? sgm.w + (size_t)expert * p.expert_stride : sgm.w;
    const uint8_t *seg0 = wexp + (size_t)t * p.blocks * SEG_BYTES;

    const int bpc = (p.blocks + KS - 1) / KS;
    const int b0 = kc * bpc;
    const int b1 = min(p.blocks, b0 + bpc);

    float se = 0.0f, so = 0.0f;  // classes 2s and 2s+1 of row n
    if (live && b0 < b1) {
        // two register sets in ping-pong: the next block's loads are in
        // flight while the current block is computed, with no copies
        BlockRegs ra, rb;
        auto load = [&](BlockRegs &r, int bb) {
            load_block(r, seg0 + (size_t)bb * SEG_BYTES, aq, ad, bb, lane, n);
        };
        auto terms_of = [&](const BlockRegs &r, float &te, float &to) {
            block_terms(r, msel, te, to);
        };
        load(ra, b0);
        for (int b = b0; b < b1; b += 2) {
            if (b + 1 < b1) load(rb, b + 1);
            float te, to;
            terms_of(ra, te, to);
            consume_terms<KS>(b, te, to, se, so, terms[local], n, s);
            if (b + 1 >= b1) break;
            if (b + 2 < b1) load(ra, b + 2);
            terms_of(rb, te, to);
            consume_terms<KS>(b + 1, te, to, se, so, terms[local], n, s);
        }
    }
    if constexpr (KS > 1) {
        __syncthreads();
        if (!live || kc != 0) return;
        // fold in block order, classes 2s and 2s+1 on lane (n, s)
        for (int b = 0; b < p.blocks; ++b) {
            se = se + terms[local][b][n][2 * s];
            so = so + terms[local][b][n][2 * s + 1];
        }
    } else {
        if (!live) return;
    }
    // lane (n, 0) adds the eight class sums in class order (dot.rs:195)
    float cls[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        cls[2 * q] = __shfl(se, n + 16 * q, WAVE);
        cls[2 * q + 1] = __shfl(so, n + 16 * q, WAVE);
    }
    const int row = t * TILE_ROWS + n;
    float tot = -0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) tot = tot + cls[c];
    if (s == 0 && row < sgm.rows) sgm.y[(size_t)slot * sgm.rows + row] = tot;
    if constexpr (AMAX) {
        // this tile's arg-max candidate for the LM head (argmax_final reduces
        // the tiles): the largest non-NaN logit, lowest row on ties
        const bool ok = s == 0 && row < sgm.rows && !isnan(tot);
        float bv = ok ? tot : -INFINITY;
        int bi = ok ? row : 0x7FFFFFFF;
        argmax_step(bv, bi, dpp<DPP_XOR1>(-INFINITY, bv), dpp<DPP_XOR1>(0x7FFFFFFF, bi));
        argmax_step(bv, bi, dpp<DPP_XOR2>(-INFINITY, bv), dpp<DPP_XOR2>(0x7FFFFFFF, bi));
        argmax_step(bv, bi, dpp<DPP_HALF_MIRROR>(-INFINITY, bv), dpp<DPP_HALF_MIRROR>(0x7FFFFFFF, bi));
        argmax_step(bv, bi, dpp<DPP_MIRROR>(-INFINITY, bv), dpp<DPP_MIRROR>(0x7FFFFFFF, bi));
        if (lane == 0) {
            p.amax_v[(size_t)slot * sgm.tiles + t] = bv;
            p.amax_i[(size_t)slot * sgm.tiles + t] = bi;
        }
    }
}

// Down projection and expert combine in one workgroup per 16-row tile: wave e
// computes the tile for routed expert ids[e] on activation e (all of its
// blocks, next block's loads in flight), then wave 0 adds the experts in
// routing order, out = res + (((0 + w0*y0) + w1*y1) + ...) (layer.rs:245-258,
// 281-287). No cross-workgroup traffic: the combine reads LDS.
struct DownParams {
    const uint8_t *w;
    size_t expert_stride;
    const int32_t *ids;
    const int8_t *aq;     // [n_slots][blocks*256]  (act == nullptr)
    const float *ad;      // [n_slots][blocks]
    const float *weights; // [n_slots] routing weights
    const float *res;     // [rows] or nullptr
    float *out;           // [rows]
    int rows, tiles, blocks, n_slots;
};

__global__ __launch_bounds__(1024) void q6k_down_combine(DownParams p) {
    asm volatile("" ::"s"(p.w), "s"(p.expert_stride), "s"(p.ids), "s"(p.aq), "s"(p.ad),
                 "s"(p.weights), "s"(p.res), "s"(p.out), "s"(p.rows), "s"(p.blocks), "s"(p.n_slots));
    __shared__ float ys[16][TILE_ROWS];
    const int lane = threadIdx.x & 63;
    const int e = threadIdx.x >> 6;
    const int t = blockIdx.x;
    const int n = lane & 15, s = lane >> 4;
    const MaskSel msel = mask_selectors(n, (n >> 2) == s);
    float se = 0.0f, so = 0.0f;
    BlockRegs ra, rb;
    {
        const uint8_t *seg0 = p.w + (size_t)p.ids[e] * p.expert_stride + (size_t)t * p.blocks * SEG_BYTES;
        const int8_t *aq = p.aq + (size_t)e * p.blocks * QK_K;
        const float *ad = p.ad + (size_t)e * p.blocks;
        load_block(ra, seg0, aq, ad, 0, lane, n);
        for (int b = 0; b < p.blocks; b += 2) {
            if (b + 1 < p.blocks) load_block(rb, seg0 + (size_t)(b + 1) * SEG_BYTES, aq, ad, b + 1, lane, n);
            float te, to;
            block_terms(ra, msel, te, to);
            se = se + te;
            so = so + to;
            if (b + 1 >= p.blocks) break;
            if (b + 2 < p.blocks) load_block(ra, seg0 + (size_t)(b + 2) * SEG_BYTES, aq, ad, b + 2, lane, n);
            block_terms(rb, msel, te, to);
            se = se + te;
            so = so + to;
        }
    }
    float cls[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        cls[2 * q] = __shfl(se, n + 16 * q, WAVE);
        cls[2 * q + 1] = __shfl(so, n + 16 * q, WAVE);
    }
    if (s == 0) {
        float tot = -0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) tot = tot + cls[c];
        ys[e][n] = tot;
    }
    __syncthreads();
    if (e == 0 && lane < TILE_ROWS) {
        const int row = t * TILE_ROWS + lane;
        if (row < p.rows) {
            float acc = 0.0f;
            for (int q = 0; q < p.n_slots; ++q) {
                const float prod = p.weights[q] * ys[q][lane];
                acc = acc + prod;
            }
            p.out[row] = p.res ? p.res[row] + acc : acc;
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
    const int32_t *pair_out;     // output row of each sorted pair (nullptr: identity)
    const int8_t *act_q;         // token-chunked Q8_K quants (q8k_wave.hpp)
    const float *act_d;          // their scales
    float *y;                    // y[pair_out * ldy + row]
    float *amax_v;               // optional per-(token, tile) arg-max candidates
    int *amax_i;                 //   [token][tiles] (single group only)
    int ldy, rows, tiles, blocks, n_groups;
    int single_count;            // grp_expert == nullptr: one group, expert 0, this many tokens
    const GroupItem *sub_info;   // optional: each chunk's / twin's record
    const GroupItem *twin_info;  //   (launch_moe_group), else a binary search
    // optional second matrix of the same shape on the same activations (gate
    // and up in one launch): items from items_per_mat on use w2 / y2
    const uint8_t *w2;
    float *y2;
    int items_per_mat;
    // n_segs > 0 (single group only): up to three matrices of their own row
    // counts on the same activations in one launch (Q, K and V of a batch);
    // segment i's items start at item segs[i].first
    int n_segs;
    struct Seg {
        const uint8_t *w;
        float *y;
        int rows, tiles, first, items;
    } segs[3];
};

// The work item of this wave and the parameters it runs with: the second
// matrix's items are the first's, offset by items_per_mat.
__device__ __forceinline__ int batch_item(const BatchParams &p, BatchParams &q) {
    int item = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
    q = p;
    if (p.n_segs > 0) {
        // the item's segment, chosen with scalar selects
        BatchParams::Seg sg = p.segs[0];
        if (p.n_segs > 1 && item >= p.segs[1].first) sg = p.segs[1];
        if (p.n_segs > 2 && item >= p.segs[2].first) sg = p.segs[2];
        q.w = sg.w;
        q.y = sg.y;
        q.rows = q.ldy = sg.rows;
        q.tiles = sg.tiles;
        q.items_per_mat = sg.items;
        return item - sg.first;
    }
    if (p.w2 && item >= p.items_per_mat) {
        item -= p.items_per_mat;
        q.w = p.w2;
        q.y = p.y2;
    }
    return item;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ s16x2 as_s16x2(uint32_t v) { return __builtin_bit_cast(s16x2, v); }
__device__ __forceinline__ uint32_t as_u32(s16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Per-block constants of the fold: this lane's 4 scales as int16 pairs, and
// 128 - 32 * scale likewise (so sc * (q - 32) + 128 is one packed multiply-add).
struct FoldScales {
    s16x2 sc[4], off[4];
};

__device__ __forceinline__ FoldScales fold_scales(uint32_t scw) {
    FoldScales f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const short v = (short)(int8_t)((scw >> (8 * j)) & 0xFF);
        f.sc[j] = s16x2{v, v};
        f.off[j] = s16x2{(short)(128 - 32 * v), (short)(128 - 32 * v)};
    }
    return f;
}

// w' = sc * (q - 32) for the lane's 8 class-c weights (codes: one byte each,
// weight kk uses scale kk / 2), split into int8 digits w' = 256 * hi + lo with
// lo in [-128, 127] and hi in [-16, 16]. One packed 16-bit multiply-add per
// two weights gives v = w' + 128 in [-3936, 4224]; the high byte of v is hi
// (arithmetic: floor(v / 256)) and its low byte, minus 128, is lo -- as a
// byte, the low byte with its top bit flipped. Byte permutes gather the
// 8-byte MFMA operands straight from the 16-bit lanes.
__device__ __forceinline__ void fold_digits(uint64_t codes, const FoldScales &f, long &lo8,
                                            long &hi8) {
    const uint32_t c0 = (uint32_t)codes, c1 = (uint32_t)(codes >> 32);
    const uint32_t w[4] = {__builtin_amdgcn_perm(0u, c0, 0x0C010C00u),
                           __builtin_amdgcn_perm(0u, c0, 0x0C030C02u),
                           __builtin_amdgcn_perm(0u, c1, 0x0C010C00u),
                           __builtin_amdgcn_perm(0u, c1, 0x0C030C02u)};
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = as_u32(as_s16x2(w[j]) * f.sc[j] + f.off[j]);
    lo8 = (long)((uint64_t)(__builtin_amdgcn_perm(v[1], v[0], 0x06040200u) ^ 0x80808080u) |
                 ((uint64_t)(__builtin_amdgcn_perm(v[3], v[2], 0x06040200u) ^ 0x80808080u) << 32));
    hi8 = (long)((uint64_t)__builtin_amdgcn_perm(v[1], v[0], 0x07050301u) |
                 ((uint64_t)__builtin_amdgcn_perm(v[3], v[2], 0x07050301u) << 32));
}


// The work of one wave on one 16-row tile t of expert `expert`'s weights
// against NC consecutive 16-token chunks sub0.. of the token-chunked
// activations (local chunk numbers st0.. inside the group of `cnt` pairs
// starting at sorted position `start`). The weight codes are unpacked and
// folded once per class and feed the MFMAs of all NC chunks, so a second
// chunk costs only its MFMAs and its float epilogue. Each chunk's class plane
// of a block is one contiguous 512-byte load for the wave.
template <int NC, bool PF = false>
__device__ __forceinline__ void batched_tile(const BatchParams &p, int lane, int t, int sub0,
                                             int st0, int cnt, int start, int expert) {
    const int n = lane & 15, s = lane >> 4;
    const uint8_t *seg = p.w + (size_t)expert * p.expert_stride + (size_t)t * p.blocks * SEG_BYTES;
    const size_t chunk_q = (size_t)p.blocks * CHUNK_BLOCK_BYTES, chunk_d = (size_t)p.blocks * CHUNK_TOKENS;
    const int8_t *aq = p.act_q + (size_t)sub0 * chunk_q + n * 32 + 8 * s;
    const float *ad = p.act_d + (size_t)sub0 * chunk_d + n;

    float sums[NC][8][4];
#pragma unroll
    for (int u = 0; u < NC; ++u)
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int v = 0; v < 4; ++v) sums[u][c][v] = 0.0f;

    // one block's operands: the lane's weight words and its chunks' class
    // planes and scales
    struct Regs {
        uint4 q0, q1, q2;
        uint32_t scw;
        uint2 dw;
        float adb[NC];
    };
    auto load = [&](Regs &r, int b) {
        const uint8_t *sg = seg + (size_t)b * SEG_BYTES;
        r.q0 = *(const uint4 *)(sg + 16 * lane);
        r.q1 = *(const uint4 *)(sg + SEG_PART + 16 * lane);
        r.q2 = *(const uint4 *)(sg + 2 * SEG_PART + 16 * lane);
        r.scw = *(const uint32_t *)(sg + SEG_SC + 4 * lane);
        r.dw = *(const uint2 *)(sg + SEG_D + 8 * s);  // f16 d of rows 4s..4s+3
#pragma unroll
        for (int u = 0; u < NC; ++u) {
            r.adb[u] = ad[u * chunk_d + (size_t)b * CHUNK_TOKENS];
        }
    };
    // the class planes run BQ classes ahead of their MFMAs, across block
    // boundaries (8 % BQ == 0, so a class keeps its ring slot); past the
    // last block the loads re-read it, unused
    constexpr int BQ = 2;
    const int last = p.blocks - 1;
    long act[BQ][NC];
    auto aload = [&](int b, int c) {
#pragma unroll
        for (int u = 0; u < NC; ++u)
            act[c % BQ][u] = *(const long *)(aq + u * chunk_q + (size_t)min(b, last) * CHUNK_BLOCK_BYTES + 512 * c);
    };
    auto compute = [&](const Regs &r, int b) {
        const uint32_t nib[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t hb[4] = {r.q2.x, r.q2.y, r.q2.z, r.q2.w};
        const FoldScales fs = fold_scales(r.scw);
        // f16(d) of the lane's 4 rows (D rows 4s..4s+3) times the token's scale
        const float d4[4] = {f16_bits_to_f32((uint16_t)(r.dw.x & 0xFFFF)),
                             f16_bits_to_f32((uint16_t)(r.dw.x >> 16)),
                             f16_bits_to_f32((uint16_t)(r.dw.y & 0xFFFF)),
                             f16_bits_to_f32((uint16_t)(r.dw.y >> 16))};
        float dd[NC][4];
#pragma unroll
        for (int u = 0; u < NC; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) dd[u][v] = d4[v] * r.adb[u];
        const v4i zero = {0, 0, 0, 0};
        // software-pipelined by one class: the MFMAs of class c+1 are issued
        // before the epilogue of class c reads its results
        v4i dh[2][NC], dl[2][NC];
        {
            long a_lo, a_hi;
            fold_digits((uint64_t)unpack_codes(nib, hb, 0), fs, a_lo, a_hi);
#pragma unroll
            for (int u = 0; u < NC; ++u) {
                dh[0][u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, act[0][u], zero, 0, 0, 0);
                dl[0][u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, act[0][u], zero, 0, 0, 0);
            }
            aload(BQ < 8 ? b : b + 1, BQ % 8);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (c + 1 < 8) {
                long a_lo, a_hi;
                fold_digits((uint64_t)unpack_codes(nib, hb, c + 1), fs, a_lo, a_hi);
#pragma unroll
                for (int u = 0; u < NC; ++u) {
                    dh[(c + 1) & 1][u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, act[(c + 1) % BQ][u], zero, 0, 0, 0);
                    dl[(c + 1) & 1][u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, act[(c + 1) % BQ][u], zero, 0, 0, 0);
                }
                aload(c + 1 + BQ < 8 ? b : b + 1, (c + 1 + BQ) % 8);
            }
#pragma unroll
            for (int u = 0; u < NC; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int aux = dh[c & 1][u][v] * 256 + dl[c & 1][u][v];
                    sums[u][c][v] = sums[u][c][v] + dd[u][v] * (float)aux;
                }
        }
    };
    if constexpr (PF) {
        // two register sets in ping-pong: the next block's loads are in
        // flight while the current block is computed. The loads are
        // unconditional (past the last block they re-read it, unused), so
        // the compiler waits for each block's own loads only.
        Regs ra, rb;
        load(ra, 0);
#pragma unroll
        for (int c = 0; c < BQ; ++c) aload(0, c);
        for (int b = 0; b < p.blocks; b += 2) {
            load(rb, min(b + 1, last));
            compute(ra, b);
            if (b + 1 >= p.blocks) break;
            load(ra, min(b + 2, last));
            compute(rb, b + 1);
        }
    } else {
#pragma unroll
        for (int c = 0; c < BQ; ++c) aload(0, c);
        for (int b = 0; b < p.blocks; ++b) {
            Regs r;
            load(r, b);
            compute(r, b);
        }
    }
#pragma unroll
    for (int u = 0; u < NC; ++u) {
        const int tok = 16 * (st0 + u) + n;  // this lane's token (B operand / output column)
        const bool tok_ok = tok < cnt;       // slots past the last token hold no data;
                                             // their columns are never stored
        float bv = -INFINITY;  // arg-max candidate of this lane's rows (lowest row on ties)
        int bi = 0x7FFFFFFF;
        if (tok_ok) {
            const int pos = start + tok;
            const int orow = p.pair_out ? p.pair_out[pos] : pos;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = t * TILE_ROWS + 4 * s + v;
                if (row < p.rows) {
                    float tot = -0.0f;
#pragma unroll
                    for (int c = 0; c < 8; ++c) tot = tot + sums[u][c][v];
                    p.y[(size_t)orow * p.ldy + row] = tot;
                    if (!isnan(tot)) argmax_step(bv, bi, tot, row);
                }
            }
        }
        if (p.amax_v) {
            // combine the 4 lanes (s = 0..3) of each token: lanes n, n+16, n+32, n+48
            argmax_step(bv, bi, __shfl_xor(bv, 16, WAVE), __shfl_xor(bi, 16, WAVE));
            argmax_step(bv, bi, __shfl_xor(bv, 32, WAVE), __shfl_xor(bi, 32, WAVE));
            if (s == 0 && tok_ok) {
                p.amax_v[(size_t)tok * p.tiles + t] = bv;
                p.amax_i[(size_t)tok * p.tiles + t] = bi;
            }
        }
    }
}

// One wave per (group, 16-token chunk, 16-row tile). The chunk index is the
// global sub-tile number, which is also where the activations of its 16
// tokens sit in the token-chunked layout.
__global__ __launch_bounds__(256) void q6k_mv_batched(BatchParams pk) {
    const int lane = threadIdx.x & 63;
    BatchParams p;
    const int item = batch_item(pk, p);
    if (item >= p.items_per_mat) return;  // the grid's rounding to whole workgroups
    const int t = item % p.tiles;
    const int sub = item / p.tiles;
    int st = sub, cnt, start = 0, expert = 0;
    if (p.grp_expert) {
        // find the group whose chunk range holds `sub` (sub_start has
        // n_groups + 1 entries)
        if (p.sub_info) {
            const GroupItem it = p.sub_info[sub];  // expert -1: a spare item
            if (it.expert < 0) return;
            st = it.st;
            cnt = it.count;
            start = it.start;
            expert = it.expert;
        } else {
            if (sub >= p.sub_start[p.n_groups]) return;
            int lo = 0, hi = p.n_groups;
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (p.sub_start[mid] <= sub) lo = mid; else hi = mid;
            }
            st = sub - p.sub_start[lo];
            cnt = p.grp_count[lo];
            start = p.grp_start[lo];
            expert = p.grp_expert[lo];
        }
    } else {
        cnt = p.single_count;
        if (sub >= (cnt + 15) / 16) return;
    }
    batched_tile<1, true>(p, lane, t, sub, st, cnt, start, expert);
}

// One wave per (group, twin, 16-row tile): a twin is two consecutive chunks
// of one group (the group's last twin holds one chunk when its chunk count is
// odd). twin_start = sub_start + n_groups + 1 is the prefix sum of
// ceil(chunks/2) over the groups. The shared fold takes the VALU work of a
// twin from 2 x 325 to 460 instructions per block; the register budget is
// capped at 3 waves per SIMD (168 VGPRs, a few spilled), which measured 20%
// faster than the uncapped 178 VGPRs at 2 waves and 5% faster than one chunk
// per wave.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void q6k_mv_batched_twin(BatchParams pk) {
    const int lane = threadIdx.x & 63;
    BatchParams p;
    const int item = batch_item(pk, p);
    if (item >= p.items_per_mat) return;  // the grid's rounding to whole workgroups
    const int t = item % p.tiles;
    const int tw = item / p.tiles;
    const int32_t *twin_start = p.sub_start + p.n_groups + 1;
    int st, sub, cnt, start, expert;
    bool two;
    if (p.twin_info) {
        const GroupItem it = p.twin_info[tw];  // expert -1: a spare item
        if (it.expert < 0) return;
        st = it.st;
        sub = it.sub;
        cnt = it.count;
        start = it.start;
        expert = it.expert;
        two = it.twin2 != 0;
    } else {
        if (tw >= twin_start[p.n_groups]) return;
        int lo = 0, hi = p.n_groups;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (twin_start[mid] <= tw) lo = mid; else hi = mid;
        }
        st = 2 * (tw - twin_start[lo]);
        sub = p.sub_start[lo] + st;
        cnt = p.grp_count[lo];
        start = p.grp_start[lo];
        expert = p.grp_expert[lo];
        two = sub + 1 < p.sub_start[lo + 1];
    }
    if (two)
        batched_tile<2>(p, lane, t, sub, st, cnt, start, expert);
    else
        batched_tile<1>(p, lane, t, sub, st, cnt, start, expert);
}

// ---- REDUCTION-tolerance batched kernels (LLAMD_HIP_REDUCTION) ----------------
//
// The same operands, digits and MFMAs as batched_tile, but the MFMAs of all 8
// classes of a block accumulate into one pair of digit accumulators: the
// block's integer dot sum_c aux32[c] is exact in int32 (|.| < 2^27), and the
// float epilogue is one convert and one fused multiply-add per (row, token,
// block) instead of the reference's eight ordered class sums. Only the float
// rounding differs from dot_q6k_q8k (nb products and additions per row
// instead of 8 nb and the 8-term class sum), so outputs are within REDUCTION,
// not bit-identical. Because the partial sums may now be added in any order,
// K is split over KS waves of one workgroup (a shorter dependent chain of
// block loads per wave, KS times the waves in flight), met in LDS.

// The lane's partial sums (4 rows x NC chunks) over blocks [b0, b1) of tile t.
// The dynamic LDS of the LDSA kernels below.
extern __shared__ uint4 g_act_lds[];

// Activation planes in LDS are stored with a swizzle: in each 512-byte plane
// (16 tokens x 32 bytes), the two 16-byte halves of token n's row are swapped
// when bit 2 of n is set. The MFMA lane (token n, quarter s) reads 8 bytes at
// 32 n + 8 s; without the swap, tokens n and n + 4 hit the same banks and a
// plane read has 4-way bank conflicts, with it 2-way at most (the 16-byte
// unit of the global-to-LDS copies allows no finer move).
__device__ __forceinline__ int act_lds_byte(int n, int s) {
    return 32 * n + 16 * ((s >> 1) ^ ((n >> 2) & 1)) + 8 * (s & 1);
}
// The global 16-byte unit (offset within the chunk's block) that LDS unit
// `slot` of the same block holds: the swap is its own inverse.
__device__ __forceinline__ int act_lds_src(int slot) {
    const int n = (slot >> 1) & 15;
    return 16 * (slot ^ ((n >> 2) & 1));
}

// LDSA: the chunk's quants are read from g_act_lds (same layout).
template <int NC, bool LDSA = false>
__device__ __forceinline__ void fast_tile_range(const BatchParams &p, int lane, int t, int sub0,
                                                int expert, int b0, int b1, float acc[2][4]) {
    const int n = lane & 15, s = lane >> 4;
    const uint8_t *seg = p.w + (size_t)expert * p.expert_stride + (size_t)t * p.blocks * SEG_BYTES;
    const size_t chunk_q = (size_t)p.blocks * CHUNK_BLOCK_BYTES, chunk_d = (size_t)p.blocks * CHUNK_TOKENS;
    const int8_t *aq = LDSA ? (const int8_t *)g_act_lds + act_lds_byte(n, s)
                            : p.act_q + (size_t)sub0 * chunk_q + n * 32 + 8 * s;
    const float *ad = p.act_d + (size_t)sub0 * chunk_d + n;
    // class planes two classes ahead of their MFMAs, across blocks (past the
    // range's last block the loads re-read it, unused)
    constexpr int BQ = 2;
    const int last = b1 - 1;
    long act[BQ][NC];
    auto aload = [&](int b, int c) {
#pragma unroll
        for (int u = 0; u < NC; ++u)
            act[c % BQ][u] = *(const long *)(aq + u * chunk_q + (size_t)min(b, last) * CHUNK_BLOCK_BYTES + 512 * c);
    };
#pragma unroll
    for (int c = 0; c < BQ; ++c) aload(b0, c);
    struct W {
        uint4 q0, q1, q2;
        uint32_t scw;
        uint2 dw;
        float adb[NC];
    };
    auto wload = [&](W &r, int b) {
        const uint8_t *sg = seg + (size_t)b * SEG_BYTES;
        r.q0 = *(const uint4 *)(sg + 16 * lane);
        r.q1 = *(const uint4 *)(sg + SEG_PART + 16 * lane);
        r.q2 = *(const uint4 *)(sg + 2 * SEG_PART + 16 * lane);
        r.scw = *(const uint32_t *)(sg + SEG_SC + 4 * lane);
        r.dw = *(const uint2 *)(sg + SEG_D + 8 * s);  // f16 d of rows 4s..4s+3
#pragma unroll
        for (int u = 0; u < NC; ++u) r.adb[u] = ad[u * chunk_d + (size_t)b * CHUNK_TOKENS];
    };
    auto compute = [&](const W &r, int b) {
        const uint32_t nib[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t hb[4] = {r.q2.x, r.q2.y, r.q2.z, r.q2.w};
        const FoldScales fs = fold_scales(r.scw);
        const v4i zero = {0, 0, 0, 0};
        v4i ah[NC], al[NC];
#pragma unroll
        for (int u = 0; u < NC; ++u) ah[u] = al[u] = zero;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            long a_lo, a_hi;
            fold_digits((uint64_t)unpack_codes(nib, hb, c), fs, a_lo, a_hi);
#pragma unroll
            for (int u = 0; u < NC; ++u) {
                ah[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, act[c % BQ][u], ah[u], 0, 0, 0);
                al[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, act[c % BQ][u], al[u], 0, 0, 0);
            }
            aload(c + BQ < 8 ? b : b + 1, (c + BQ) % 8);
        }
        const float d4[4] = {f16_bits_to_f32((uint16_t)(r.dw.x & 0xFFFF)), f16_bits_to_f32((uint16_t)(r.dw.x >> 16)),
                             f16_bits_to_f32((uint16_t)(r.dw.y & 0xFFFF)), f16_bits_to_f32((uint16_t)(r.dw.y >> 16))};
#pragma unroll
        for (int u = 0; u < NC; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int aux = ah[u][v] * 256 + al[u][v];
                acc[u][v] = __builtin_fmaf(d4[v] * r.adb[u], (float)aux, acc[u][v]);
            }
    };
    if constexpr (LDSA) {
        // the class planes come from LDS (lgkmcnt), so the next block's
        // weights can be in flight a whole block ahead without a class-plane
        // wait also waiting for them; the scheduling barriers keep the
        // compiler from sinking those loads back to their first use
        W ra, rb;
        wload(ra, b0);
        for (int b = b0; b < b1; b += 2) {
            wload(rb, min(b + 1, last));
            __builtin_amdgcn_sched_barrier(0);
            compute(ra, b);
            if (b + 1 >= b1) break;
            wload(ra, min(b + 2, last));
            __builtin_amdgcn_sched_barrier(0);
            compute(rb, b + 1);
        }
    } else {
        for (int b = b0; b < b1; ++b) {
            const uint8_t *sg = seg + (size_t)b * SEG_BYTES;
            const uint4 q0 = *(const uint4 *)(sg + 16 * lane);
            const uint4 q1 = *(const uint4 *)(sg + SEG_PART + 16 * lane);
            const uint4 q2 = *(const uint4 *)(sg + 2 * SEG_PART + 16 * lane);
            const uint32_t scw = *(const uint32_t *)(sg + SEG_SC + 4 * lane);
            const uint2 dw = *(const uint2 *)(sg + SEG_D + 8 * s);
            float adb[NC];
#pragma unroll
            for (int u = 0; u < NC; ++u) adb[u] = ad[u * chunk_d + (size_t)b * CHUNK_TOKENS];
            const uint32_t nib[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            const uint32_t hb[4] = {q2.x, q2.y, q2.z, q2.w};
            const FoldScales fs = fold_scales(scw);
            const v4i zero = {0, 0, 0, 0};
            v4i ah[NC], al[NC];
#pragma unroll
            for (int u = 0; u < NC; ++u) ah[u] = al[u] = zero;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                long a_lo, a_hi;
                fold_digits((uint64_t)unpack_codes(nib, hb, c), fs, a_lo, a_hi);
#pragma unroll
                for (int u = 0; u < NC; ++u) {
                    ah[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, act[c % BQ][u], ah[u], 0, 0, 0);
                    al[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, act[c % BQ][u], al[u], 0, 0, 0);
                }
                aload(c + BQ < 8 ? b : b + 1, (c + BQ) % 8);
            }
            const float d4[4] = {f16_bits_to_f32((uint16_t)(dw.x & 0xFFFF)), f16_bits_to_f32((uint16_t)(dw.x >> 16)),
                                 f16_bits_to_f32((uint16_t)(dw.y & 0xFFFF)), f16_bits_to_f32((uint16_t)(dw.y >> 16))};
#pragma unroll
            for (int u = 0; u < NC; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int aux = ah[u][v] * 256 + al[u][v];
                    acc[u][v] = __builtin_fmaf(d4[v] * adb[u], (float)aux, acc[u][v]);
                }
        }
    }
}

// KS waves per work item (4 / KS items per workgroup). TWIN: the items are
// twins (moe_group's twin records), else 16-token chunks (chunk records, or
// the single group of grp_expert == nullptr).
// LDSA: one 16-token chunk for the whole grid (the LM head at batch <= 16):
// each workgroup first copies the chunk's quants (blocks x 4 KiB, dynamic
// LDS) once, so the class-plane loads of every block read LDS instead of
// going through the vector memory path (they outnumber the weight loads).
template <int KS, bool TWIN, bool LDSA = false>
__global__ __launch_bounds__(256) void q6k_mv_batched_fast(BatchParams pk) {
    constexpr int IPW = 4 / KS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kc = wave % KS;
    const int n = lane & 15, s = lane >> 4;
    int item = (int)blockIdx.x * IPW + wave / KS;
    BatchParams p = pk;
    if (p.w2 && item >= p.items_per_mat) {
        item -= p.items_per_mat;
        p.w = p.w2;
        p.y = p.y2;
    }
    bool live = item < p.items_per_mat;  // the grid's rounding to whole workgroups
    int t = 0, sub = 0, st = 0, cnt = 0, start = 0, expert = 0, nc = 1;
    if (live) {
        t = item % p.tiles;
        const int unit = item / p.tiles;
        if (p.grp_expert) {
            const GroupItem it = TWIN ? p.twin_info[unit] : p.sub_info[unit];  // expert -1: spare
            live = it.expert >= 0;
            st = it.st;
            sub = it.sub;
            cnt = it.count;
            start = it.start;
            expert = it.expert;
            nc = TWIN && it.twin2 ? 2 : 1;
        } else {
            cnt = p.single_count;
            sub = st = unit;
            live = unit < (cnt + 15) / 16;
        }
    }
    const int bpc = (p.blocks + KS - 1) / KS;
    const int b0 = kc * bpc, b1 = min(p.blocks, b0 + bpc);
    float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    if constexpr (LDSA) {
        const int n16 = p.blocks * CHUNK_BLOCK_BYTES / 16;
        const uint4 *src = (const uint4 *)p.act_q;
        for (int i = threadIdx.x; i < n16; i += blockDim.x) g_act_lds[i] = src[act_lds_src(i) / 16];
        __syncthreads();
        if (live && b0 < b1) fast_tile_range<1, true>(p, lane, t, 0, expert, b0, b1, acc);
    } else if (live && b0 < b1) {
        if (nc == 2) fast_tile_range<2>(p, lane, t, sub, expert, b0, b1, acc);
        else fast_tile_range<1>(p, lane, t, sub, expert, b0, b1, acc);
    }
    if constexpr (KS > 1) {
        // every wave reaches the barrier (no early return above)
        __shared__ float part[4][2][4][WAVE];
        if (kc != 0) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) part[wave][u][v][lane] = acc[u][v];
        }
        __syncthreads();
        if (kc != 0) return;
#pragma unroll
        for (int k = 1; k < KS; ++k)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] += part[wave + k][u][v][lane];
    }
    if (!live) return;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        if (u >= nc) break;
        const int tok = 16 * (st + u) + n;  // this lane's token
        const bool tok_ok = tok < cnt;
        float bv = -INFINITY;  // arg-max candidate of this lane's rows (lowest row on ties)
        int bi = 0x7FFFFFFF;
        int nan_row = 0;       // a NaN logit in the tile voids the tile's certificate
        if (tok_ok) {
            const int pos = start + tok;
            const int orow = p.pair_out ? p.pair_out[pos] : pos;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = t * TILE_ROWS + 4 * s + v;
                if (row < p.rows) {
                    p.y[(size_t)orow * p.ldy + row] = acc[u][v];
                    if (!isnan(acc[u][v])) argmax_step(bv, bi, acc[u][v], row);
                    else nan_row = 1;
                }
            }
        }
        if (p.amax_v) {
            // the 4 lanes (s = 0..3) of each token: lanes n, n+16, n+32, n+48
            argmax_step(bv, bi, __shfl_xor(bv, 16, WAVE), __shfl_xor(bi, 16, WAVE));
            argmax_step(bv, bi, __shfl_xor(bv, 32, WAVE), __shfl_xor(bi, 32, WAVE));
            nan_row |= __shfl_xor(nan_row, 16, WAVE);
            nan_row |= __shfl_xor(nan_row, 32, WAVE);
            if (s == 0 && tok_ok) {
                p.amax_v[(size_t)tok * p.tiles + t] = bv;
                p.amax_i[(size_t)tok * p.tiles + t] = nan_row ? -1 : bi;
            }
        }
    }
}



// The grouped kernel with the activations staged in LDS. A workgroup's 4
// waves are 4 tiles of one unit (tiles % 4 == 0), so they read the same
// chunks: per block, the unit's NC x 4 KiB of class planes are copied once
// into LDS by direct global-to-LDS loads (1 KiB per wave instruction, no
// registers), double-buffered, and every wave reads its planes from LDS. The
// next block's planes and weights are in flight while the current block is
// computed; one barrier per block hands the buffer over.
using lds_ptr = __attribute__((address_space(3))) void *;

template <int NC>
__device__ __forceinline__ void fast_tile_staged(const BatchParams &p, int lane, int wave, int t,
                                                 int sub0, int expert, float acc[2][4]) {
    const int n = lane & 15, s = lane >> 4;
    const uint8_t *seg = p.w + (size_t)expert * p.expert_stride + (size_t)t * p.blocks * SEG_BYTES;
    const size_t chunk_q = (size_t)p.blocks * CHUNK_BLOCK_BYTES, chunk_d = (size_t)p.blocks * CHUNK_TOKENS;
    const int8_t *gq = p.act_q + (size_t)sub0 * chunk_q;
    const float *ad = p.act_d + (size_t)sub0 * chunk_d + n;
    int8_t *lds = (int8_t *)g_act_lds;  // [2][NC][4096]
    constexpr int BUF = NC * CHUNK_BLOCK_BYTES;
    // this wave's share of a block's planes: NC KiB, one 16-byte piece per lane
    auto stage = [&](int b) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int off = (wave * NC + i) * 1024;  // within the NC x 4 KiB
            const int u = off / CHUNK_BLOCK_BYTES, o = off % CHUNK_BLOCK_BYTES;
            __builtin_amdgcn_global_load_lds(
                (const void *)(gq + u * chunk_q + (size_t)b * CHUNK_BLOCK_BYTES + act_lds_src(o / 16 + lane)),
                (lds_ptr)(lds + (b & 1) * BUF + off), 16, 0, 0);
        }
    };
    struct W {
        uint4 q0, q1, q2;
        uint32_t scw;
        uint2 dw;
        float adb[NC];
    };
    auto wload = [&](W &r, int b) {
        const uint8_t *sg = seg + (size_t)b * SEG_BYTES;
        r.q0 = *(const uint4 *)(sg + 16 * lane);
        r.q1 = *(const uint4 *)(sg + SEG_PART + 16 * lane);
        r.q2 = *(const uint4 *)(sg + 2 * SEG_PART + 16 * lane);
        r.scw = *(const uint32_t *)(sg + SEG_SC + 4 * lane);
        r.dw = *(const uint2 *)(sg + SEG_D + 8 * s);
#pragma unroll
        for (int u = 0; u < NC; ++u) r.adb[u] = ad[u * chunk_d + (size_t)b * CHUNK_TOKENS];
    };
    auto compute = [&](const W &r, int b) {
        const int8_t *aq = lds + (b & 1) * BUF + act_lds_byte(n, s);
        const uint32_t nib[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t hb[4] = {r.q2.x, r.q2.y, r.q2.z, r.q2.w};
        const FoldScales fs = fold_scales(r.scw);
        const v4i zero = {0, 0, 0, 0};
        v4i ah[NC], al[NC];
#pragma unroll
        for (int u = 0; u < NC; ++u) ah[u] = al[u] = zero;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            long a_lo, a_hi;
            fold_digits((uint64_t)unpack_codes(nib, hb, c), fs, a_lo, a_hi);
#pragma unroll
            for (int u = 0; u < NC; ++u) {
                const long av = *(const long *)(aq + u * CHUNK_BLOCK_BYTES + 512 * c);
                ah[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, av, ah[u], 0, 0, 0);
                al[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, av, al[u], 0, 0, 0);
            }
        }
        const float d4[4] = {f16_bits_to_f32((uint16_t)(r.dw.x & 0xFFFF)), f16_bits_to_f32((uint16_t)(r.dw.x >> 16)),
                             f16_bits_to_f32((uint16_t)(r.dw.y & 0xFFFF)), f16_bits_to_f32((uint16_t)(r.dw.y >> 16))};
#pragma unroll
        for (int u = 0; u < NC; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int aux = ah[u][v] * 256 + al[u][v];
                acc[u][v] = __builtin_fmaf(d4[v] * r.adb[u], (float)aux, acc[u][v]);
            }
    };
    // the block's planes must be in LDS (this wave's pieces landed, every
    // wave past the barrier) before any wave reads them; the barrier also
    // keeps a buffer from being refilled while a wave still reads it
    auto handover = [&]() {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    const int last = p.blocks - 1;
    W ra, rb;
    stage(0);
    wload(ra, 0);
    handover();
    for (int b = 0; b < p.blocks; b += 2) {
        if (b + 1 <= last) stage(b + 1);
        wload(rb, min(b + 1, last));
        __builtin_amdgcn_sched_barrier(0);
        compute(ra, b);
        handover();
        if (b + 1 > last) break;
        if (b + 2 <= last) stage(b + 2);
        wload(ra, min(b + 2, last));
        __builtin_amdgcn_sched_barrier(0);
        compute(rb, b + 1);
        handover();
    }
}

// One wave per (unit, tile), 4 tiles of one unit per workgroup; TWIN as in
// q6k_mv_batched_fast. Dynamic LDS: 2 x (TWIN ? 2 : 1) x 4 KiB.
template <bool TWIN>
__global__ __launch_bounds__(256) void q6k_mv_batched_fast_staged(BatchParams pk) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, s = lane >> 4;
    int item = (int)blockIdx.x * 4 + wave;
    BatchParams p = pk;
    if (p.w2 && item >= p.items_per_mat) {
        item -= p.items_per_mat;
        p.w = p.w2;
        p.y = p.y2;
    }
    // the workgroup's 4 items share their unit (tiles % 4 == 0), so these
    // exits are uniform over the workgroup and no barrier below is skipped
    // by some waves only
    if (item >= p.items_per_mat) return;
    const int t = item % p.tiles;
    const GroupItem it = TWIN ? p.twin_info[item / p.tiles] : p.sub_info[item / p.tiles];
    if (it.expert < 0) return;
    const int nc = TWIN && it.twin2 ? 2 : 1;
    float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    if (nc == 2) fast_tile_staged<2>(p, lane, wave, t, it.sub, it.expert, acc);
    else fast_tile_staged<1>(p, lane, wave, t, it.sub, it.expert, acc);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        if (u >= nc) break;
        const int tok = 16 * (it.st + u) + n;
        if (tok >= it.count) continue;
        const int pos = it.start + tok;
        const int orow = p.pair_out ? p.pair_out[pos] : pos;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = t * TILE_ROWS + 4 * s + v;
            if (row < p.rows) p.y[(size_t)orow * p.ldy + row] = acc[u][v];
        }
    }
}

// ---- LM head: certified arg-max over REDUCTION-tolerance logits -------------
//
// The fast batched kernel's logit F_r of row r and the reference's E_r are two
// roundings of the same real value T_r = sum_b dd_b * sum_c aux_b[c] (dd_b =
// f16(d_b) * a.d_b, the same float in both; aux integers exact in both):
//   |E_r - T_r| <= gamma_{nb+10} S_r  (8 class sums of nb rounded products,
//                                     then the 8-term class sum)
//   |F_r - T_r| <= gamma_{nb+1} S_r   (nb fused multiply-adds)
// with S_r = sum_b |dd_b| sum_c |aux_b[c]| <= 127 (1 + u) sum_b |a.d_b|
// |f16(d_b)| sum_e |sc(e)(q_e - 32)| <= 127 (1 + u) D_a M_r, since every Q8_K
// quant is at most 127 in magnitude; D_a = max_b |a.d_b| of the token and M_r
// the weights' own sum, bounded per tile by q6k_tile_bound. So
// |F_r - E_r| <= delta_t = 2 (2 nb + 12) u 127 D_a M_t (+ 2^-20 |F|, covering
// the bound's own float rounding) for every row r of tile t (u = 2^-24).
// Every row whose E_r could be the maximum then lies in a tile with
// F_t + delta_t >= L = max_t (F_t - delta_t), F_t the tile's largest F.

// One wave per tile.
__global__ __launch_bounds__(256) void q6k_tile_bound(const uint8_t *w, int tiles, int blocks,
                                                      float *mt) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tiles) return;
    const int n = lane & 15;
    float m = 0.0f;
    for (int b = 0; b < blocks; ++b) {
        const uint8_t *sg = w + ((size_t)t * blocks + b) * SEG_BYTES;
        const uint4 q0 = *(const uint4 *)(sg + 16 * lane);
        const uint4 q1 = *(const uint4 *)(sg + SEG_PART + 16 * lane);
        const uint4 q2 = *(const uint4 *)(sg + 2 * SEG_PART + 16 * lane);
        const uint32_t scw = *(const uint32_t *)(sg + SEG_SC + 4 * lane);
        const uint16_t dh = *(const uint16_t *)(sg + SEG_D + 2 * n);
        const uint32_t nib[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[4] = {q2.x, q2.y, q2.z, q2.w};
        // the lane's 64 weights of row n: class c, byte kk = weight 8 (8 s + kk) + c,
        // scale group 4 s + kk / 2 (byte kk / 2 of scw)
        int acc = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint64_t codes = (uint64_t)unpack_codes(nib, hb, c);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const int q = (int)((codes >> (8 * kk)) & 0xFF) - 32;
                const int sc = __builtin_amdgcn_sbfe(scw, 8 * (kk >> 1), 8);
                acc += abs(sc * q);
            }
        }
        acc += __shfl_xor(acc, 16, WAVE);
        acc += __shfl_xor(acc, 32, WAVE);
        m += fabsf(f16_bits_to_f32(dh)) * (float)acc;  // acc <= 2^20: exact
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, WAVE));
    if (lane == 0) mt[t] = m;
}

struct CertifyParams {
    const uint8_t *w;      // tiled Q6_K [rows x blocks]
    const int8_t *nq;      // [nseq][blocks * 256] natural Q8_K
    const float *nd;       // [nseq][blocks]
    const float *pv;       // [nseq][tiles] the fast kernel's tile candidates
    const int *pi;         //   (row, or -1: a NaN logit in the tile)
    const float *mt;       // [tiles] q6k_tile_bound
    float *logits;         // [nseq][rows]
    int32_t *ids;          // [nseq]
    int rows, tiles, blocks;
};

// One 1024-thread workgroup per token. Its tiles' candidates are read once
// (CERT_PT per thread kept in registers), the candidate tiles gathered in LDS,
// and their exact recomputation spread over the 16 waves by (tile, block):
// each wave computes one block's eight class terms of one tile into LDS (a
// single round trip to memory for up to 16 / blocks tiles), then one wave per
// tile folds them in block order, as dot_q6k_q8k does (the q6k_mv_b1 split-K
// fold).
constexpr int CERT_PT = 16;     // tiles per thread held in registers (beyond: re-read)
constexpr int CERT_CAP = 1024;  // candidate list; more (no certificate) -> every tile
constexpr int CERT_MAXB = 32;   // blocks per row (k <= 8192)

__global__ __launch_bounds__(1024) void lmhead_certify(CertifyParams p) {
    const int u = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, s = lane >> 4;
    const float *F = p.pv + (size_t)u * p.tiles;
    const int *FI = p.pi + (size_t)u * p.tiles;
    const float *ad = p.nd + (size_t)u * p.blocks;
    const int8_t *aq = p.nq + (size_t)u * p.blocks * QK_K;
    __shared__ float s_lo[16];
    __shared__ int s_bad[16];
    __shared__ int s_cand[CERT_CAP];
    __shared__ int s_ncand;
    // per round: entry e = (tile e / blocks, block e % blocks), CERT_MAXB / blocks tiles
    __shared__ float s_terms[CERT_MAXB][TILE_ROWS][8];
    if (tid == 0) s_ncand = 0;
    // 1. the certified lower bound L of the largest exact logit
    float fv[CERT_PT], dv[CERT_PT];
    float lo = -INFINITY;
    int bad = 0;
    float da, cst;
    {
        // all of the thread's loads in flight at once: unconditional, at a
        // clamped index, the out-of-range ones discarded afterwards
        int fi[CERT_PT];
        float mv[CERT_PT];
#pragma unroll
        for (int i = 0; i < CERT_PT; ++i) {
            const int t = min(tid + i * (int)blockDim.x, p.tiles - 1);
            fv[i] = F[t];
            mv[i] = p.mt[t];
            fi[i] = FI[t];
        }
        // D_a = max_b |a.d_b|: one load per lane (blocks <= 32), a wave max
        da = lane < p.blocks ? fabsf(ad[lane]) : 0.0f;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) da = fmaxf(da, __shfl_xor(da, o, WAVE));
        cst = 2.0f * (float)(2 * p.blocks + 12) * 0x1p-24f * 127.0f * da;
#pragma unroll
        for (int i = 0; i < CERT_PT; ++i) {
            if (tid + i * (int)blockDim.x >= p.tiles) continue;
            dv[i] = cst * mv[i] + 0x1p-20f * fabsf(fv[i]);
            if (!isfinite(fv[i]) || !isfinite(dv[i]) || fi[i] < 0) bad = 1;
            else lo = fmaxf(lo, fv[i] - dv[i]);
        }
    }
    for (int t = tid + CERT_PT * (int)blockDim.x; t < p.tiles; t += blockDim.x) {
        const float f = F[t], d = cst * p.mt[t] + 0x1p-20f * fabsf(f);
        if (!isfinite(f) || !isfinite(d) || FI[t] < 0) bad = 1;
        else lo = fmaxf(lo, f - d);
    }
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        lo = fmaxf(lo, __shfl_xor(lo, o, WAVE));
        bad |= __shfl_xor(bad, o, WAVE);
    }
    if (lane == 0) { s_lo[wave] = lo; s_bad[wave] = bad; }
    __syncthreads();
    for (int w = 0; w < 16; ++w) { lo = fmaxf(lo, s_lo[w]); bad |= s_bad[w]; }
    // 2. the candidate tiles (tile 0 always: the reference's incumbent is row 0)
    if (!bad) {
        auto keep = [&](int t, float f, float d) {
            if (t == 0 || f + d >= lo) {
                const int at = atomicAdd(&s_ncand, 1);
                if (at < CERT_CAP) s_cand[at] = t;
            }
        };
#pragma unroll
        for (int i = 0; i < CERT_PT; ++i) {
            const int t = tid + i * (int)blockDim.x;
            if (t < p.tiles) keep(t, fv[i], dv[i]);
        }
        for (int t = tid + CERT_PT * (int)blockDim.x; t < p.tiles; t += blockDim.x)
            keep(t, F[t], cst * p.mt[t] + 0x1p-20f * fabsf(F[t]));
    }
    __syncthreads();
    const bool all = bad || s_ncand > CERT_CAP;
    const int total = all ? p.tiles : s_ncand;
    // 3. exact recomputation, (tile, block) pairs over the waves: up to
    // CERT_MAXB pairs per round, two per wave with both pairs' loads in
    // flight together (a round is one memory round trip)
    // tiles per round: a wave folds each (blocks <= CERT_MAXB, checked at launch)
    const int per = min(16, CERT_MAXB / p.blocks);
    const int pairs = per * p.blocks;
    const MaskSel msel = mask_selectors(n, (n >> 2) == s);
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    int nan0 = 0;
    for (int r0 = 0; r0 < total; r0 += per) {
        float se = 0.0f, so = 0.0f;
        for (int e0 = wave; e0 < pairs; e0 += 32) {
            BlockRegs r[2];
            bool ok[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int e = e0 + 16 * h;
                const int ci = r0 + e / p.blocks, b = e % p.blocks;
                ok[h] = e < pairs && ci < total;
                if (ok[h]) {
                    const int tt = all ? ci : s_cand[ci];
                    load_block(r[h], p.w + ((size_t)tt * p.blocks + b) * SEG_BYTES, aq, ad, b, lane, n);
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (!ok[h]) continue;
                const int e = e0 + 16 * h;
                float te, to;
                block_terms(r[h], msel, te, to);
                const int slot = e;
                s_terms[slot][n][2 * s] = te;
                s_terms[slot][n][2 * s + 1] = to;
            }
        }
        __syncthreads();
        if (wave < per && r0 + wave < total) {
            const int tt = all ? r0 + wave : s_cand[r0 + wave];
            const int base = wave * p.blocks;
            for (int b = 0; b < p.blocks; ++b) {
                se = se + s_terms[base + b][n][2 * s];
                so = so + s_terms[base + b][n][2 * s + 1];
            }
            float cls[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                cls[2 * q] = __shfl(se, n + 16 * q, WAVE);
                cls[2 * q + 1] = __shfl(so, n + 16 * q, WAVE);
            }
            float tot = -0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) tot = tot + cls[c];
            const int row = tt * TILE_ROWS + n;
            if (s == 0 && row < p.rows) {
                p.logits[(size_t)u * p.rows + row] = tot;
                if (!isnan(tot)) argmax_step(bv, bi, tot, row);
                if (row == 0 && isnan(tot)) nan0 = 1;
            }
        }
        __syncthreads();
    }
    wave_argmax(bv, bi, -INFINITY);
    nan0 = __ballot(nan0 != 0) != 0 ? 1 : 0;
    __shared__ float s_bv[16];
    __shared__ int s_bi[16], s_nan[16];
    if (lane == 0) { s_bv[wave] = bv; s_bi[wave] = bi; s_nan[wave] = nan0; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w) {
            argmax_step(bv, bi, s_bv[w], s_bi[w]);
            nan0 |= s_nan[w];
        }
        p.ids[u] = (nan0 || bi == 0x7FFFFFFF) ? 0 : bi;
    }
}

// y = W . Q8_K(x) with x in f32 (the long-context decode step's O
// projection, whose activation comes from the attention as f32): the bits of
// launch_q8k_quantize + q6k_mv_b1<8> in one launch. One 16-row tile per
// 8-wave workgroup; wave k quantizes the blocks it multiplies, [bpc k,
// bpc k + bpc), with quantize_wave into its own LDS rows while its weight
// loads are in flight; the per-block terms are folded in block order.
constexpr int F32X_MAX_BLOCKS = 16;

__global__ __launch_bounds__(512) void q6k_mv_f32x(const uint8_t *w, const float *x, float *y,
                                                   int rows, int blocks) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, s = lane >> 4;
    const int t = blockIdx.x;
    const int bpc = (blocks + 7) / 8;  // at most 2
    const int b0 = wave * bpc, b1 = min(blocks, b0 + bpc);
    __shared__ float terms[F32X_MAX_BLOCKS][TILE_ROWS][8];
    __shared__ __align__(16) int8_t lq[F32X_MAX_BLOCKS * QK_K];
    __shared__ float ld[F32X_MAX_BLOCKS];
    const uint8_t *seg = w + (size_t)t * blocks * SEG_BYTES;
    BlockRegs r[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (i < bpc) load_weights(r[i], seg + (size_t)min(b0 + i, blocks - 1) * SEG_BYTES, lane, n);
    float4 xv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (i < bpc) xv[i] = *(const float4 *)(x + (size_t)min(b0 + i, blocks - 1) * QK_K + 4 * lane);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (i < bpc && b0 + i < b1) {
            const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
            quantize_wave(v, lane, lq + (b0 + i) * QK_K, ld + b0 + i, nullptr);
        }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const MaskSel msel = mask_selectors(n, (n >> 2) == s);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (i < bpc && b0 + i < b1) {
            r[i].g = *(const uint4 *)(lq + (b0 + i) * QK_K + 16 * n);
            r[i].ad = ld[b0 + i];
            float te, to;
            block_terms(r[i], msel, te, to);
            terms[b0 + i][n][2 * s] = te;
            terms[b0 + i][n][2 * s + 1] = to;
        }
    __syncthreads();
    if (wave != 0) return;
    float se = 0.0f, so = 0.0f;
    for (int b = 0; b < blocks; ++b) {
        se = se + terms[b][n][2 * s];
        so = so + terms[b][n][2 * s + 1];
    }
    float cls[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        cls[2 * q] = __shfl(se, n + 16 * q, WAVE);
        cls[2 * q + 1] = __shfl(so, n + 16 * q, WAVE);
    }
    const int row = t * TILE_ROWS + n;
    float tot = -0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) tot = tot + cls[c];
    if (s == 0 && row < rows) y[row] = tot;
}

}  // namespace

int g_tune_mv_ks = 0;
int g_tune_batched_twin = 1;
int g_tune_fast_ks = 0;
int g_tune_fast_lds = 1;

namespace {

// Fills the segment table for n matrices sharing `rows`-independent shapes.
void set_segments(MvParams &p, int n, const void *const *w, float *const *y, const int *rows,
                  int n_slots) {
    MvSeg *seg[3] = {&p.seg0, &p.seg1, &p.seg2};
    int first = 0;
    p.n_seg = n;
    for (int i = 0; i < n; ++i) {
        seg[i]->w = (const uint8_t *)w[i];
        seg[i]->y = y[i];
        seg[i]->rows = rows[i];
        seg[i]->tiles = (rows[i] + TILE_ROWS - 1) / TILE_ROWS;
        seg[i]->first = first;
        first += seg[i]->tiles * n_slots;
    }
    for (int i = n; i < 3; ++i) *seg[i] = p.seg0;
    p.items = first;
    p.n_slots = n_slots;
}

// q6k_mv_b1's preloaded leading arguments, then the whole parameter block
#define B1_ARGS(p) (p).seg0.w, (p).aq, (p).ad, (p).ids, (p).blocks, (p).seg0.tiles, (p).items, \
                   (p).act_per_slot, (p)
// ... or, for the plain matvec, the compact one
#define B1_LITE(p) (p).seg0.w, (p).aq, (p).ad, (p).ids, (p).blocks, (p).seg0.tiles, (p).items, \
                   (p).act_per_slot, MvLite{(p).seg0.y, (p).expert_stride, (p).clk, (p).seg0.rows, (p).n_slots}

template <int NSEG, bool AMAX = false>
void launch_b1_n(const MvParams &p, hipStream_t st) {
    const int items = p.items;
    // Measured on MI355X: eight waves per tile (one block each at k = 2048)
    // win while the grid is small -- 768 x 2048: 3.46 -> 3.17 us, 4096 x
    // 2048: 4.14 -> 3.82 us -- and lose from ~1000 tiles on (LM head 41 ->
    // 52 us), where four waves already fill the machine.
    // Short rows (at most 4 blocks, down's k = 768) in a large grid go the
    // other way: one wave per tile walks all of its blocks. 128 down
    // matrices [2048 x 768] in one grouped launch: 44.0 -> 29.9 us with one
    // wave per tile; 8 of them (1024 tiles): 3.80 -> 3.48 us; below ~1000
    // tiles four waves stay ahead (512 tiles: 2.98 vs 3.12 us).
    const int ks = g_tune_mv_ks ? g_tune_mv_ks
                                : (p.blocks > 4 && items <= 384 ? 8 : (p.blocks <= 4 && items >= 1024 ? 1 : 0));
    constexpr bool LITE = NSEG == 1 && !AMAX;
    if (p.blocks <= 16 && (ks == 4 || ks == 8 || ks == 0)) {
        if (ks == 8) {
            if constexpr (LITE)
                hipLaunchKernelGGL((q6k_mv_b1<8, false, 1, false, MvLite>), dim3(items), dim3(512), 0, st, B1_LITE(p));
            else
                hipLaunchKernelGGL((q6k_mv_b1<8, false, NSEG, AMAX>), dim3(items), dim3(512), 0, st, B1_ARGS(p));
        } else {
            // Measured on MI355X (gate/up/down/q_proj/LM-head shapes): four
            // waves per tile, each on a quarter of the row, beat one wave per
            // tile -- more loads in flight per tile and shorter per-wave
            // chains -- except for short rows in large grids (above).
            if constexpr (LITE)
                hipLaunchKernelGGL((q6k_mv_b1<4, false, 1, false, MvLite>), dim3(items), dim3(256), 0, st, B1_LITE(p));
            else
                hipLaunchKernelGGL((q6k_mv_b1<4, false, NSEG, AMAX>), dim3(items), dim3(256), 0, st, B1_ARGS(p));
        }
    } else {
        if constexpr (LITE)
            hipLaunchKernelGGL((q6k_mv_b1<1, false, 1, false, MvLite>), dim3((items + 3) / 4), dim3(256), 0, st, B1_LITE(p));
        else
            hipLaunchKernelGGL((q6k_mv_b1<1, false, NSEG, AMAX>), dim3((items + 3) / 4), dim3(256), 0, st, B1_ARGS(p));
    }
}

// llamd_hip_kernel_clock: slots [n][2] for the q6k_mv_b1 launches, in turn
unsigned long long *g_clk_slots = nullptr;
int g_clk_n = 0, g_clk_next = 0;

int launch_b1(const MvParams &pin, hipStream_t st) {
    MvParams p = pin;
    if (g_clk_slots) {
        p.clk = g_clk_slots + 2 * (size_t)CLOCK_WAVES * g_clk_next;
        g_clk_next = (g_clk_next + 1) % g_clk_n;
    }
    if (p.amax_v) launch_b1_n<1, true>(p, st);  // LM head: one segment, one slot
    else if (p.n_seg == 1) launch_b1_n<1>(p, st);
    else if (p.n_seg == 2) launch_b1_n<2>(p, st);
    else launch_b1_n<3>(p, st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_q6k_mv_b1(const void *w, size_t expert_stride, const int32_t *ids, const int8_t *aq,
                     const float *ad, float *y, int rows, int blocks, int n_slots, int act_per_slot,
                     hipStream_t st, const void *w_b, float *amax_v, int *amax_i) {
    if (amax_v && w_b) return -1;
    MvParams p = {};
    p.amax_v = amax_v;
    p.amax_i = amax_i;
    // with a second weight, its outputs follow the first's: y = [w | w_b]
    const void *ws[2] = {w, w_b};
    float *ys[2] = {y, y + (size_t)n_slots * rows};
    const int rs[2] = {rows, rows};
    set_segments(p, w_b ? 2 : 1, ws, ys, rs, n_slots);
    p.expert_stride = expert_stride;
    p.ids = ids;
    p.aq = aq;
    p.ad = ad;
    p.blocks = blocks;
    p.act_per_slot = act_per_slot;
    return launch_b1(p, st);
}

int launch_q6k_mv_x3(const void *const w[3], float *const y[3], const int rows[3], int n_mat,
                     const int8_t *aq, const float *ad, int blocks, hipStream_t st) {
    if (n_mat < 1 || n_mat > 3) return -1;
    MvParams p = {};
    set_segments(p, n_mat, w, y, rows, 1);
    p.aq = aq;
    p.ad = ad;
    p.blocks = blocks;
    return launch_b1(p, st);
}

int launch_q6k_mv_grouped_x2(const void *wa, const void *wb, size_t expert_stride,
                             const int32_t *ids, const int8_t *aq, const float *ad, float *oa,
                             float *ob, int rows, int blocks, int n_used, hipStream_t st,
                             int act_per_slot) {
    MvParams p = {};
    const void *ws[2] = {wa, wb};
    float *ys[2] = {oa, ob};
    const int rs[2] = {rows, rows};
    set_segments(p, 2, ws, ys, rs, n_used);
    p.expert_stride = expert_stride;
    p.ids = ids;
    p.aq = aq;
    p.ad = ad;
    p.blocks = blocks;
    p.act_per_slot = act_per_slot;
    return launch_b1(p, st);
}

int launch_q6k_mv_routed(const void *w, const void *w_b, size_t expert_stride,
                         const float *logits, int n_expert, int n_used, int32_t *ids_out,
                         float *w_out, int *stats, const int8_t *aq, const float *ad, float *y,
                         int rows, int blocks, hipStream_t st) {
    if (blocks > 16 || n_expert > ROUTE_MAX_EXPERTS || n_used > ROUTE_MAX_USED) return -1;
    MvParams p = {};
    const void *ws[2] = {w, w_b};
    float *ys[2] = {y, y + (size_t)n_used * rows};
    const int rs[2] = {rows, rows};
    set_segments(p, 2, ws, ys, rs, n_used);
    p.expert_stride = expert_stride;
    p.aq = aq;
    p.ad = ad;
    p.blocks = blocks;
    p.route_l = logits;
    p.n_expert = n_expert;
    p.n_used = n_used;
    p.ids_out = ids_out;
    p.w_out = w_out;
    p.stats = stats;
    hipLaunchKernelGGL((q6k_mv_b1<4, true, 2>), dim3(p.items), dim3(256), 0, st, B1_ARGS(p));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q6k_mv_batched(const void *w, size_t expert_stride, const int32_t *grp_expert,
                          const int32_t *grp_start, const int32_t *grp_count,
                          const int32_t *sub_start, const int32_t *pair_out, const int8_t *act_q,
                          const float *act_d, float *y, int ldy, int rows, int blocks,
                          int n_groups, int max_chunks, hipStream_t st, float *amax_v,
                          int *amax_i, bool group_tables, const void *w2, float *y2, bool fast) {
    if (amax_v && grp_expert) return -1;
    // every item of the grids below indexes a record below max_chunks when
    // max_chunks >= n_groups (twins: ceil((max_chunks + n_groups) / 2) items)
    if (group_tables && (!grp_expert || max_chunks < n_groups || max_chunks <= 0)) return -1;
    BatchParams p;
    p.n_segs = 0;
    if (w2 && (!y2 || amax_v)) return -1;
    p.w2 = (const uint8_t *)w2;
    p.y2 = y2;
    p.sub_info = group_tables ? (const GroupItem *)(sub_start + group_items_offset(n_groups)) : nullptr;
    p.twin_info = group_tables ? p.sub_info + max_chunks : nullptr;
    p.single_count = n_groups;  // only read when grp_expert == nullptr
    p.w = (const uint8_t *)w;
    p.expert_stride = expert_stride;
    p.grp_expert = grp_expert;
    p.grp_start = grp_start;
    p.grp_count = grp_count;
    p.sub_start = sub_start;
    p.pair_out = pair_out;
    p.act_q = act_q;
    p.act_d = act_d;
    p.y = y;
    p.amax_v = amax_v;
    p.amax_i = amax_i;
    p.ldy = ldy;
    p.rows = rows;
    p.tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    p.blocks = blocks;
    p.n_groups = n_groups;
    if (fast) {
        // K split over ks waves (tune key fast_ks): one measured best on
        // MI355X for both the prefill and the LM head shapes
        const int ks = g_tune_fast_ks ? g_tune_fast_ks : 1;
        const bool twin = grp_expert && g_tune_batched_twin;
        if (grp_expert && !group_tables) return -1;
        const long units = twin ? (max_chunks + n_groups + 1) / 2 : max_chunks;
        const long items = (long)p.tiles * units;
        if (items <= 0) return 0;
        p.items_per_mat = (int)items;
        const long all = w2 ? 2 * items : items;
        const unsigned grid = (unsigned)((all * ks + 3) / 4);
        const size_t lds = (size_t)blocks * CHUNK_BLOCK_BYTES;
        if (grp_expert && ks == 1 && p.tiles % 4 == 0 && g_tune_fast_lds) {
            const size_t slds = (size_t)2 * (twin ? 2 : 1) * CHUNK_BLOCK_BYTES;
            if (twin) hipLaunchKernelGGL(q6k_mv_batched_fast_staged<true>, dim3(grid), dim3(256), slds, st, p);
            else hipLaunchKernelGGL(q6k_mv_batched_fast_staged<false>, dim3(grid), dim3(256), slds, st, p);
        } else if (!grp_expert && n_groups <= CHUNK_TOKENS && lds <= 65536 && g_tune_fast_lds) {
            if (ks == 4) hipLaunchKernelGGL((q6k_mv_batched_fast<4, false, true>), dim3(grid), dim3(256), lds, st, p);
            else if (ks == 2) hipLaunchKernelGGL((q6k_mv_batched_fast<2, false, true>), dim3(grid), dim3(256), lds, st, p);
            else hipLaunchKernelGGL((q6k_mv_batched_fast<1, false, true>), dim3(grid), dim3(256), lds, st, p);
        } else if (ks == 4 && twin) hipLaunchKernelGGL((q6k_mv_batched_fast<4, true>), dim3(grid), dim3(256), 0, st, p);
        else if (ks == 4) hipLaunchKernelGGL((q6k_mv_batched_fast<4, false>), dim3(grid), dim3(256), 0, st, p);
        else if (ks == 2 && twin) hipLaunchKernelGGL((q6k_mv_batched_fast<2, true>), dim3(grid), dim3(256), 0, st, p);
        else if (ks == 2) hipLaunchKernelGGL((q6k_mv_batched_fast<2, false>), dim3(grid), dim3(256), 0, st, p);
        else if (twin) hipLaunchKernelGGL((q6k_mv_batched_fast<1, true>), dim3(grid), dim3(256), 0, st, p);
        else hipLaunchKernelGGL((q6k_mv_batched_fast<1, false>), dim3(grid), dim3(256), 0, st, p);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (grp_expert && g_tune_batched_twin) {
        // twins: sum of ceil(ch/2) <= (sum of ch + n_groups) / 2
        const long items = (long)p.tiles * ((max_chunks + n_groups + 1) / 2);
        if (items <= 0) return 0;
        p.items_per_mat = (int)items;
        const long all = w2 ? 2 * items : items;
        hipLaunchKernelGGL(q6k_mv_batched_twin, dim3((unsigned)((all + 3) / 4)), dim3(256), 0, st, p);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    const long items = (long)p.tiles * max_chunks;
    if (items <= 0) return 0;
    p.items_per_mat = (int)items;
    const long all = w2 ? 2 * items : items;
    hipLaunchKernelGGL(q6k_mv_batched, dim3((unsigned)((all + 3) / 4)), dim3(256), 0, st, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q6k_mv_batched_x3(const void *const w[3], float *const y[3], const int rows[3], int n_mat,
                             const int8_t *act_q, const float *act_d, int blocks, int nseq,
                             hipStream_t st) {
    if (n_mat < 1 || n_mat > 3 || nseq <= 0 || blocks <= 0) return -1;
    BatchParams p = {};
    const int chunks = (nseq + CHUNK_TOKENS - 1) / CHUNK_TOKENS;
    int first = 0;
    p.n_segs = n_mat;
    for (int i = 0; i < n_mat; ++i) {
        auto &sg = p.segs[i];
        sg.w = (const uint8_t *)w[i];
        sg.y = y[i];
        sg.rows = rows[i];
        sg.tiles = (rows[i] + TILE_ROWS - 1) / TILE_ROWS;
        sg.first = first;
        sg.items = sg.tiles * chunks;
        first += sg.items;
    }
    p.w = p.segs[0].w;
    p.y = p.segs[0].y;
    p.rows = p.ldy = rows[0];
    p.tiles = p.segs[0].tiles;
    p.items_per_mat = p.segs[0].items;
    p.act_q = act_q;
    p.act_d = act_d;
    p.blocks = blocks;
    p.single_count = nseq;  // one group (expert 0) of nseq tokens
    hipLaunchKernelGGL(q6k_mv_batched, dim3((unsigned)((first + 3) / 4)), dim3(256), 0, st, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q6k_down_combine(const void *w, size_t expert_stride, const int32_t *ids,
                            const int8_t *aq, const float *ad, const float *weights,
                            const float *res, float *out, int rows, int blocks, int n_slots,
                            hipStream_t st) {
    if (n_slots <= 0 || n_slots > 16) return -1;
    DownParams p;
    p.w = (const uint8_t *)w;
    p.expert_stride = expert_stride;
    p.ids = ids;
    p.aq = aq;
    p.ad = ad;
    p.weights = weights;
    p.res = res;
    p.out = out;
    p.rows = rows;
    p.tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    p.blocks = blocks;
    p.n_slots = n_slots;
    hipLaunchKernelGGL(q6k_down_combine, dim3(p.tiles), dim3(64 * n_slots), 0, st, p);
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

namespace llamd {

int launch_q6k_tile_bound(const void *w, int rows, int blocks, float *mt, hipStream_t st) {
    const int tiles = (rows + TILE_ROWS - 1) / TILE_ROWS;
    if (tiles <= 0 || blocks <= 0) return -1;
    hipLaunchKernelGGL(q6k_tile_bound, dim3((tiles + 3) / 4), dim3(256), 0, st, (const uint8_t *)w,
                       tiles, blocks, mt);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q6k_mv_f32x(const void *w, const float *x, float *y, int rows, int blocks,
                       hipStream_t st) {
    if (!w || !x || !y || rows <= 0 || blocks <= 0 || blocks > F32X_MAX_BLOCKS) return -1;
    hipLaunchKernelGGL(q6k_mv_f32x, dim3((rows + TILE_ROWS - 1) / TILE_ROWS), dim3(512), 0, st,
                       (const uint8_t *)w, x, y, rows, blocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_lmhead_certify(const void *w, int rows, int blocks, int nseq, const int8_t *nq,
                          const float *nd, const float *pv, const int *pi, const float *mt,
                          float *logits, int32_t *ids, hipStream_t st) {
    if (rows <= 0 || blocks <= 0 || blocks > CERT_MAXB || nseq <= 0) return -1;
    CertifyParams p{(const uint8_t *)w, nq, nd, pv, pi, mt, logits, ids, rows,
                    (rows + TILE_ROWS - 1) / TILE_ROWS, blocks};
    hipLaunchKernelGGL(lmhead_certify, dim3(nseq), dim3(1024), 0, st, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd

extern "C" int llamd_hip_kernel_clock(unsigned long long *d_slots, int n_slots) {
    if (d_slots && n_slots <= 0) return -1;
    llamd::g_clk_slots = d_slots;
    llamd::g_clk_n = d_slots ? n_slots : 0;
    llamd::g_clk_next = 0;
    return 0;
}
