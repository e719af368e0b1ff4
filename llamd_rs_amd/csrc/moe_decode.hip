// moe_decode.hip -- one MoE decode layer in TWO launches, bit-identical to
// the reference's CPU path: router logits (moe.rs:73-80), softmax / top-k /
// renormalise (moe.rs:82-113), gate, up, SwiGLU (layer.rs:230-244), down and
// the weighted combine + residual (layer.rs:245-258, 281-287).
//
// WHY. The reference's router logit is a 2048-long sequential f32 fold:
// about 7 us on one lane, and in stream order (router; gate/up; down) the
// expert matvecs wait for it. Here gate/up runs WHILE the folds run:
//
//   launch 1, workgroups [0, n_chain): four experts each. Products to LDS;
//     waves 0-3 run the exact folds while waves 4-7 publish an estimate T
//     and a bound E with |logit - T| <= E (fold_estimate).
//   launch 1, workgroups [n_chain, ...): one (routed slot, 16-row tile) of
//     gate and up each. Wave 0 takes the n_used largest estimates; when every
//     chosen [T - E] lies above every other [T + E] (with a margin that keeps
//     the softmax from tying them) the exact top-k SET is certain and the
//     experts are used in the estimate's order. Otherwise it waits for the
//     exact logits and routes exactly. act = silu(g) * u.
//   launch 1, last workgroup (per sequence): waits for the exact logits and
//     routes them (route_finish) -- ids and weights in the reference's
//     order -- while the gate/up tiles are still streaming.
//   launch 2, one workgroup per 16-row tile of down: wave e computes the
//     tile for act row e, and the rows are combined in the exact routing's
//     order with its weights. No result depends on the estimate; it only
//     decides how early gate/up may start.
//
// HAND-OFF WITHOUT CACHE-WIDE FENCES. Inside launch 1, values cross
// workgroups in 64-bit words (value, ready mark) written with relaxed
// agent-scope atomic stores and polled with relaxed agent-scope atomic loads
// (route.hpp). A workgroup only waits for workgroups with lower indices,
// which the dispatcher places first, and every wait is bounded. Launch 2
// empties the words for the next call. (Measured on MI355X: putting the down
// projection in the same launch, with one more hand-off for act, is slower --
// 30 us per token instead of 25: each cross-XCD hand-off costs microseconds,
// more than the launch boundary it replaces.)
#include "common.hpp"
#include "exact_sum.hpp"
#include "expf_ref.h"
#include "launch.hpp"
#include "q6k_tile.hpp"
#include "q8k_wave.hpp"
#include "route.hpp"

namespace llamd {
namespace {

constexpr int CHAIN_EXPERTS = 4;   // experts per chain workgroup (waves 0-3)
constexpr int KMAX = 2048;         // router row length held in LDS
constexpr int MAX_USED = 16;
constexpr int GU_MAX_BLOCKS = 16;  // n_embd <= 4096 for the gate/up activation in LDS

struct DecodeParams {
    const uint8_t *w_gate, *w_up, *w_down;
    const float *rw, *x, *res;   // router [n_expert][k], x [k], residual [k] or null
    float *out, *logits;         // [k], [n_expert]
    double *est;                 // [2][n_expert] diagnostic copy of T, E
    unsigned long long *slots;   // [2][n_expert]: (T, E) floats, then (logit, 0)
    float *act;                  // [n_used][n_ff]
    int32_t *spec_ids;           // [n_used] expert of each act row
    int32_t *ids_out;
    float *w_out;
    int *stats;                  // [4] calls, exact calls, certified calls, timed out
    size_t gu_stride, down_stride;
    int k, n_expert, n_used, n_ff, gu_tiles, bf, down_tiles, n_chain, n_gu, nseq;
    const float *norm_a, *norm_b, *norm_w;  // fused FFN norm (norm_w null: x is given)
    float norm_eps;
    float *norm_sum;
    int polls;  // bound of every wait on another workgroup (slots_wait)
};

// The parameters of sequence `seq` of a batch: every per-token array offset
// to that sequence's row (x, res, out [nseq][k]; logits [nseq][n_expert];
// est, slots [nseq][2][n_expert]; act [nseq][n_used][n_ff]; spec_ids, ids_out,
// w_out [nseq][n_used]).
__device__ __forceinline__ DecodeParams for_seq(const DecodeParams &p, int seq) {
    DecodeParams q = p;
    q.x += (size_t)seq * p.k;
    if (q.res) q.res += (size_t)seq * p.k;
    q.out += (size_t)seq * p.k;
    q.logits += (size_t)seq * p.n_expert;
    q.est += (size_t)seq * 2 * p.n_expert;
    q.slots += (size_t)seq * 2 * p.n_expert;
    q.act += (size_t)seq * p.n_used * p.n_ff;
    q.spec_ids += (size_t)seq * p.n_used;
    q.ids_out += (size_t)seq * p.n_used;
    q.w_out += (size_t)seq * p.n_used;
    return q;
}

union DecodeLds {
    float4 prod[CHAIN_EXPERTS][KMAX / 4];
    struct {
        float terms[2][16][TILE_ROWS][8];
        float gu[2][TILE_ROWS];
        RouteLds rsh;
        int given[MAX_USED];
        uint64_t tab[32];
        int8_t lq[GU_MAX_BLOCKS * QK_K];
        float ld[GU_MAX_BLOCKS];
    } g;
};

// Exact logits of the lane's experts, waiting for each (whole wave). A wait
// that gives up (the producing chain workgroup was not placed in time)
// computes that logit here: the same rounded products folded in the same
// order from -0.0 (moe.rs:73-80), so the routing never depends on timing.
__device__ void wait_logits(const DecodeParams &p, float l[RW], bool &late) {
    const int lane = threadIdx.x & 63;
    bool lt = false;
    bool live[RW];
    unsigned long long vs[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) live[j] = lane + WAVE * j < p.n_expert;
    slots_wait(p.slots + p.n_expert, live, vs, p.polls, p.n_expert - 1);
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        unsigned long long v = vs[j];
        if (live[j]) {
            if (v == SLOT_EMPTY) {
                lt = true;
                const float *w = p.rw + (size_t)i * p.k;
                float acc = -0.0f;
                for (int t = 0; t < p.k; ++t) {
                    const float prod = w[t] * p.x[t];
                    acc = acc + prod;
                }
                v = __float_as_uint(acc);
            }
        }
        l[j] = __uint_as_float((unsigned)v);
    }
    late = late || __any(lt);
}

// Slot order: the n_used routed experts sit in rsh.sorted[0..n_used) by
// ascending expert index, whichever way they were chosen. Every gate/up
// workgroup and the down launch then agree on which act row holds which
// expert even if one workgroup had to route exactly (a wait that gave up)
// while the others used the certified estimate: the two give the same set.
// By one whole wave; `id` holds the set on lanes < n_used.
__device__ void slots_by_index(int id, int n_used, int *sorted) {
    const int lane = threadIdx.x & 63;
    int rank = 0;
    for (int q = 0; q < n_used; ++q) {
        const int other = __shfl(id, q, WAVE);
        rank += (q != lane && other < id) ? 1 : 0;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane < n_used) sorted[rank] = id;
}

// The candidate set for the certification in select_experts: n_used rounds
// of a wave-wide max on a composite key, the order-preserving key of the
// estimate with its low 8 bits replaced by 255 - index. The keys are
// distinct, so the max names its expert directly (no ballot search for the
// lowest index holding it), which halves each round's dependent chain. Any
// choice among estimates that differ only in those low bits is as good as
// another: the certification accepts a set only if every member's interval
// lies above every other expert's, which the exact top-k set alone
// satisfies. Bit j of the result: expert lane + 64 j is chosen.
__device__ unsigned estimate_topk(const float T[RW], const bool live[RW], int n_used) {
    const int lane = threadIdx.x & 63;
    unsigned ck[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j)
        ck[j] = live[j] ? ((sort_key(T[j]) & ~0xFFu) | (255u - (unsigned)(lane + WAVE * j))) : 0u;
    unsigned taken = 0;
    for (int r = 0; r < n_used; ++r) {
        unsigned b = 0u;
#pragma unroll
        for (int j = 0; j < RW; ++j) b = max(b, ck[j]);
        const unsigned m = (unsigned)wave_reduce((int)b, 0, [](int x, int y) {
            return (int)max((unsigned)x, (unsigned)y);
        });
        if (m == 0u) break;
#pragma unroll
        for (int j = 0; j < RW; ++j)
            if (ck[j] == m) {
                taken |= 1u << j;
                ck[j] = 0u;
            }
    }
    return taken;
}

// The routed experts, by one whole wave, into rsh.sorted[0..n_used) (slot
// order above): from the estimates when they certify the exact top-k set,
// else by exact routing. Returns whether the estimate was used.
__device__ bool select_experts(const DecodeParams &p, RouteLds &rsh, bool &timed_out) {
    const int lane = threadIdx.x & 63;
    double T[RW], E[RW];
    float key[RW];
    bool live[RW], lt = false;
    unsigned long long vs[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) live[j] = lane + WAVE * j < p.n_expert;
    slots_wait(p.slots, live, vs, p.polls, p.n_expert - 1);
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const unsigned long long v = vs[j];
        lt = lt || (live[j] && v == SLOT_EMPTY);
        key[j] = __uint_as_float((unsigned)v);
        T[j] = key[j];
        E[j] = __uint_as_float((unsigned)(v >> 32));
    }
    const bool late = __any(lt);
    timed_out = timed_out || late;
    const unsigned taken = estimate_topk(key, live, p.n_used);
    // lo = min chosen (T - E), hi = max other (T + E), top = max (T + E):
    // each formed in double and rounded outward to float, so the 32-bit
    // reductions keep the test below conservative
    float lo = INFINITY, hi = -INFINITY, top = -INFINITY;
    bool fin = true;
    int n_taken = 0;
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        if (!live[j]) continue;
        fin = fin && isfinite(T[j]) && isfinite(E[j]);
        const float up = __double2float_ru(T[j] + E[j]);
        top = fmaxf(top, up);
        if (taken & (1u << j)) {
            lo = fminf(lo, __double2float_rd(T[j] - E[j]));
            ++n_taken;
        } else {
            hi = fmaxf(hi, up);
        }
    }
    lo = wave_reduce(lo, INFINITY, [](float a, float b) { return fminf(a, b); });
    hi = wave_reduce(hi, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    top = wave_reduce(top, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    fin = __all(fin) && wave_reduce(n_taken, 0, [](int a, int b) { return a + b; }) == p.n_used;
    // The chosen logits exceed the others by more than 2^-20 (1 + max |logit|):
    // after l - max, expf and the division by the total every chosen
    // probability stays strictly above every other one. And no chosen logit
    // lies 80 or more below the maximum, so none underflows to a tie at 0.
    const double dlo = lo, dhi = hi, dtop = top;
    const double mag = fmax(fabs(dtop), fabs(dlo));
    const bool certain = !late && fin && (dlo - dhi > 0x1p-20 * (1.0 + mag)) && (dlo > dtop - 80.0);
    if (certain) {
        // the chosen set (the lane's `taken` bits) in index order: column j
        // holds experts 64 j + lane
        int before = 0;
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            const unsigned long long m = __ballot((taken >> j) & 1u);
            if ((m >> lane) & 1ull) rsh.sorted[before + __popcll(m & ((1ull << lane) - 1ull))] = lane + WAVE * j;
            before += __popcll(m);
        }
    } else {
        float l[RW];
        wait_logits(p, l, timed_out);
        route_finish(l, p.n_expert, p.n_used, true, rsh, nullptr, nullptr, nullptr);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        slots_by_index(lane < p.n_used ? rsh.sorted[lane] : 0x7FFFFFFF, p.n_used, rsh.sorted);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    return certain;
}

typedef float f4v __attribute__((ext_vector_type(4)));

// The fused FFN norm (layer.rs:170-172 and CpuBackend::rms_norm / mul,
// llamd-cpu/src/lib.rs:55-75): v = a + b; x = (v * scale) * w with scale =
// 1 / sqrt(sum(v^2) / k + eps), the sum in the reference's order
// (exact_sum_nonneg). Every workgroup forms x itself, into xs (LDS); the
// first chain workgroup also writes v for launch 2's residual. Called by
// all threads of the workgroup.
// wrow (or null): a router row this wave stages into wdst (LDS) meanwhile.
__device__ void norm_prologue(const DecodeParams &p, float *xs, ExactSumLds &xl, bool write_sum,
                              const float *wrow, float4 *wdst) {
    const int m = xsum_run(p.k, 512), j0 = min((int)threadIdx.x * m, p.k - 1), lane = threadIdx.x & 63;
    float a[XSUM_M], b[XSUM_M], nw[XSUM_M], v[XSUM_M], sq[XSUM_M];
#pragma unroll
    for (int j = 0; j < XSUM_M; ++j) {
        const int i = min(j0 + j, p.k - 1);
        a[j] = p.norm_a[i];
        b[j] = p.norm_b[i];
        nw[j] = p.norm_w[i];  // needed after the sum: loaded with the row
    }
    f4v wr[KMAX / 256];
    if (wrow) {
#pragma unroll
        for (int j = 0; j < KMAX / 256; ++j)
            if (64 * j < p.k / 4) wr[j] = ((const f4v *)wrow)[64 * j + lane];
    }
#pragma unroll
    for (int j = 0; j < XSUM_M; ++j) {
        v[j] = a[j] + b[j];
        sq[j] = v[j] * v[j];
    }
    if (wrow) {
#pragma unroll
        for (int j = 0; j < KMAX / 256; ++j)
            if (64 * j < p.k / 4) *(f4v *)&wdst[64 * j + lane] = wr[j];
    }
    const float *na = p.norm_a, *nb = p.norm_b;
    const float sum = exact_sum_nonneg(sq, p.k, 512, xl, [na, nb](int i) {
        const float t = na[i] + nb[i];
        return t * t;
    });
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(sum, (float)p.k) + p.norm_eps));
#pragma unroll
    for (int j = 0; j < XSUM_M; ++j) {
        const int i = j0 + j;
        if (j < m && i < p.k) {
            xs[i] = (v[j] * scale) * nw[j];
            if (write_sum) p.norm_sum[i] = v[j];
        }
    }
    __syncthreads();
}

// w_in_lds: the norm prologue has already put each wave's router row in
// sm.prod (its loads ran under the norm); the products are then formed in
// place.
__device__ void chain_workgroup(const DecodeParams &p, DecodeLds &sm, int blk, int lane, int wave,
                                bool w_in_lds) {
    const int e = wave & 3;
    const int row = blk * CHAIN_EXPERTS + e;
    const int n4 = p.k / 4;
    if (wave < CHAIN_EXPERTS && row < p.n_expert) {
        const float4 *w4 = w_in_lds ? sm.prod[e] : (const float4 *)(p.rw + (size_t)row * p.k);
        const float4 *x4 = (const float4 *)p.x;  // LDS when the norm is fused
        float4 wr[KMAX / 256], xr[KMAX / 256];
#pragma unroll
        for (int j = 0; j < KMAX / 256; ++j)
            if (64 * j < n4) {
                wr[j] = w4[64 * j + lane];
                xr[j] = x4[64 * j + lane];
            }
#pragma unroll
        for (int j = 0; j < KMAX / 256; ++j)
            if (64 * j < n4)
                sm.prod[e][64 * j + lane] = make_float4(wr[j].x * xr[j].x, wr[j].y * xr[j].y,
                                                        wr[j].z * xr[j].z, wr[j].w * xr[j].w);
    }
    __syncthreads();
    if (row >= p.n_expert) return;
    if (wave >= CHAIN_EXPERTS) {
        // the estimate, while wave e runs the fold
        double T, E;
        fold_estimate((const float *)sm.prod[e], p.k, T, E);
        if (lane == 0) {
            p.est[row] = T;
            p.est[p.n_expert + row] = E;
            // as floats: T' = T rounded, E' >= E + |T - T'| rounded up
            const float tf = __double2float_rn(T);
            const float ef = __double2float_ru(E + 0x1p-24 * (1.0 + 0x1p-20) * fabs((double)tf));
            const bool fin = isfinite(tf) && isfinite(ef);
            slot_store(&p.slots[row], fin ? __float_as_uint(tf) : 0x7FC00000u,
                       fin ? __float_as_uint(ef) : 0x7FC00000u);
        }
    } else if (lane == 0) {
        // a latency-bound chain: first in line for issue on its SIMD
        __builtin_amdgcn_s_setprio(3);
        const float logit = seq_fold(sm.prod[e], n4);
        p.logits[row] = logit;
        slot_store(&p.slots[p.n_expert + row], __float_as_uint(logit), 0u);
    }
}

// Gate and up of one (slot, tile): waves 0-3 split the gate row's blocks four
// ways, waves 4-7 the up row's; the per-block terms meet in LDS and are folded
// in block order (the same bits as one wave walking the row).
__device__ void gateup_workgroup(const DecodeParams &p, DecodeLds &sm, int g, int lane, int wave) {
    const int slot = g / p.gu_tiles;
    const int t = g - slot * p.gu_tiles;
    const int half = wave >> 2, kc = wave & 3;
    const int n = lane & 15, s = lane >> 4;
    const int blocks = p.k / QK_K;
    const MaskSel msel = mask_selectors(n, (n >> 2) == s);
    for (int b = wave; b < blocks; b += 8) {
        const float4 xv = *(const float4 *)(p.x + (size_t)b * QK_K + 4 * lane);
        const float v[4] = {xv.x, xv.y, xv.z, xv.w};
        quantize_wave(v, lane, &sm.g.lq[b * QK_K], &sm.g.ld[b], nullptr);
    }
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);  // the selection gates every wave of the workgroup
        expf_ref_tab_fill(sm.g.tab);
        bool timed_out = false;
        const bool certain = select_experts(p, sm.g.rsh, timed_out);
        __builtin_amdgcn_s_setprio(0);
        if (g == 0 && lane < p.n_used) p.spec_ids[lane] = sm.g.rsh.sorted[lane];
        if (lane == 0 && p.stats) {
            if (g == 0 && certain) atomicAdd(&p.stats[2], 1);
            if (timed_out) p.stats[3] = 1;
        }
    }
    __syncthreads();
    const int expert = sm.g.rsh.sorted[slot];
    const uint8_t *seg0 = (half ? p.w_up : p.w_gate) + (size_t)expert * p.gu_stride +
                          (size_t)t * blocks * SEG_BYTES;
    const int bpc = (blocks + 3) / 4;
    const int b0 = kc * bpc;
    const int b1 = min(blocks, b0 + bpc);
    auto fetch = [&](BlockRegs &r, int b) {
        r.g = *(const uint4 *)(&sm.g.lq[b * QK_K + 16 * n]);
        r.ad = sm.g.ld[b];
    };
    float se = 0.0f, so = 0.0f;
    if (b0 < b1) {
        BlockRegs ra, rb;
        load_weights(ra, seg0 + (size_t)b0 * SEG_BYTES, lane, n);
        if (b0 + 1 < b1) load_weights(rb, seg0 + (size_t)(b0 + 1) * SEG_BYTES, lane, n);
        fetch(ra, b0);
        for (int b = b0; b < b1; b += 2) {
            if (b + 1 < b1) fetch(rb, b + 1);
            float te, to;
            block_terms(ra, msel, te, to);
            consume_terms<4>(b, te, to, se, so, sm.g.terms[half], n, s);
            if (b + 1 >= b1) break;
            if (b + 2 < b1) {
                load_weights(ra, seg0 + (size_t)(b + 2) * SEG_BYTES, lane, n);
                fetch(ra, b + 2);
            }
            block_terms(rb, msel, te, to);
            consume_terms<4>(b + 1, te, to, se, so, sm.g.terms[half], n, s);
            if (b + 3 < b1) load_weights(rb, seg0 + (size_t)(b + 3) * SEG_BYTES, lane, n);
        }
    }
    __syncthreads();
    if (kc == 0) {
        // fold in block order, classes 2s and 2s+1 on lane (n, s), then the
        // eight class sums in class order (dot.rs:195)
        se = 0.0f;
        so = 0.0f;
        for (int b = 0; b < blocks; ++b) {
            se = se + sm.g.terms[half][b][n][2 * s];
            so = so + sm.g.terms[half][b][n][2 * s + 1];
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
            sm.g.gu[half][n] = tot;
        }
    }
    __syncthreads();
    if (wave == 0 && lane < TILE_ROWS) {
        const int row = t * TILE_ROWS + lane;
        if (row < p.n_ff)
            p.act[(size_t)slot * p.n_ff + row] = silu_ref(sm.g.gu[0][lane], sm.g.tab) * sm.g.gu[1][lane];
    }
}

// The exact routing of one sequence (moe.rs:82-113) from the exact logits,
// by wave 0, into ids_out / w_out for launch 2's combine.
__device__ void router_workgroup(const DecodeParams &p, DecodeLds &sm, int lane, int wave) {
    if (wave != 0) return;
    __builtin_amdgcn_s_setprio(3);
    // the gate/up tiles' selection, made here the same way: when certified,
    // only the order of that set is left to the exact probabilities
    bool late = false;
    const bool certain = select_experts(p, sm.g.rsh, late);
    if (certain && lane < p.n_used) sm.g.given[lane] = sm.g.rsh.sorted[lane];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    expf_ref_tab_fill(sm.g.rsh.tab);
    float l[RW];
    wait_logits(p, l, late);
    route_finish(l, p.n_expert, p.n_used, true, sm.g.rsh, p.ids_out, p.w_out, nullptr,
                 certain ? sm.g.given : nullptr, true);
    if (lane == 0 && late && p.stats) p.stats[3] = 1;
}

// NORM: the fused FFN norm's buffers exist only in this instance (9 KB of
// LDS the other launches would otherwise carry).
template <bool NORM>
__global__ __launch_bounds__(512) void moe_router_gateup(DecodeParams p) {
    asm volatile("" ::"s"(p.w_gate), "s"(p.w_up), "s"(p.rw), "s"(p.x), "s"(p.slots),
                 "s"(p.gu_stride), "s"(p.k), "s"(p.n_expert), "s"(p.n_used), "s"(p.n_chain));
    __shared__ DecodeLds sm;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // all sequences' chain workgroups first (the gate/up ones wait on them),
    // then the gate/up tiles, then one router workgroup per sequence
    const int b = blockIdx.x, chains = p.n_chain * p.nseq, gus = p.n_gu * p.nseq;
    if constexpr (NORM) {
        __shared__ __align__(16) float xs[KMAX];  // the fused norm's output
        __shared__ ExactSumLds xl;
        // one sequence: every workgroup forms x itself (the router
        // workgroup for the fallback folds of wait_logits); chain waves 0-3
        // stage their router rows under it
        const int row = b * CHAIN_EXPERTS + (wave & 3);
        const bool stage = b < chains && wave < CHAIN_EXPERTS && row < p.n_expert;
        // the chain workgroups' norm leads to the router folds, the longest
        // chain of the launch: their waves go first in issue on shared SIMDs
        if (b < chains) __builtin_amdgcn_s_setprio(2);
        norm_prologue(p, xs, xl, b == 0, stage ? p.rw + (size_t)row * p.k : nullptr,
                      sm.prod[wave & 3]);
        if (b < chains) __builtin_amdgcn_s_setprio(0);
        p.x = xs;
    }
    if (b < chains) {
        chain_workgroup(for_seq(p, b / p.n_chain), sm, b % p.n_chain, lane, wave, p.norm_w != nullptr);
    } else if (b < chains + gus) {
        const int g = b - chains;
        gateup_workgroup(for_seq(p, g / p.n_gu), sm, g % p.n_gu, lane, wave);
    } else {
        router_workgroup(for_seq(p, b - chains - gus), sm, lane, wave);
    }
}

// Launch 2: wave e < n_used computes the tile for expert spec_ids[e] on act
// row e (Q8_K of act in LDS, quantize_q8_k bits), and the tile's rows are
// combined in the exact routing's order (ids_out / w_out, from launch 1):
// out = res + (((0 + w0*y[ids0]) + w1*y[ids1]) + ...). Workgroup 0 counts
// the call and empties the hand-off words.
__global__ __launch_bounds__(1024) void moe_down_route(DecodeParams pb) {
    const DecodeParams p = for_seq(pb, blockIdx.y);
    asm volatile("" ::"s"(p.w_down), "s"(p.down_stride), "s"(p.spec_ids), "s"(p.act), "s"(p.n_ff),
                 "s"(p.bf), "s"(p.n_used));
    __shared__ float ys[MAX_USED][TILE_ROWS];
    __shared__ __align__(16) int8_t lq[MAX_USED][DOWN_ACT_BLOCKS * QK_K];
    __shared__ float ld[MAX_USED][DOWN_ACT_BLOCKS];
    __shared__ int rids[MAX_USED], sid[MAX_USED];
    __shared__ float rwt[MAX_USED];
    const int lane = threadIdx.x & 63;
    const int e = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = blockIdx.x;
    const int n = lane & 15, s = lane >> 4;
    if (e == 0 && lane < p.n_used) {
        // launch 1's routing and the act rows' experts; used after the matvec
        rids[lane] = p.ids_out[lane];
        rwt[lane] = p.w_out[lane];
        sid[lane] = p.spec_ids[lane];
    }
    // the residual row, loaded now so its latency hides behind the matvec
    const int orow = t * TILE_ROWS + lane;
    const float resv = e == 0 && lane < TILE_ROWS && p.res && orow < p.k ? p.res[orow] : 0.0f;
    if (e < p.n_used) {
        const MaskSel msel = mask_selectors(n, (n >> 2) == s);
        // the activations do not depend on the expert id: their loads go first
        const float *a = p.act + (size_t)e * p.n_ff;
        float4 av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j < p.bf) av[j] = *(const float4 *)(a + (size_t)j * QK_K + 4 * lane);
        const uint8_t *seg0 = p.w_down + (size_t)p.spec_ids[e] * p.down_stride +
                              (size_t)t * p.bf * SEG_BYTES;
        BlockRegs ra, rb;
        load_weights(ra, seg0, lane, n);
        if (p.bf > 1) load_weights(rb, seg0 + SEG_BYTES, lane, n);
        for (int c0 = 0; c0 < p.bf; c0 += 4) {
            if (c0 > 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (c0 + j < p.bf) av[j] = *(const float4 *)(a + (size_t)(c0 + j) * QK_K + 4 * lane);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (c0 + j < p.bf) {
                    const float v[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
                    quantize_wave(v, lane, &lq[e][(c0 + j) * QK_K], &ld[e][c0 + j], nullptr);
                }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        auto fetch = [&](BlockRegs &r, int b) {
            r.g = *(const uint4 *)(&lq[e][b * QK_K + 16 * n]);
            r.ad = ld[e][b];
        };
        float se = 0.0f, so = 0.0f;
        fetch(ra, 0);
        for (int b = 0; b < p.bf; b += 2) {
            if (b + 1 < p.bf) fetch(rb, b + 1);
            float te, to;
            block_terms(ra, msel, te, to);
            se = se + te;
            so = so + to;
            if (b + 1 >= p.bf) break;
            if (b + 2 < p.bf) {
                load_weights(ra, seg0 + (size_t)(b + 2) * SEG_BYTES, lane, n);
                fetch(ra, b + 2);
            }
            block_terms(rb, msel, te, to);
            se = se + te;
            so = so + to;
            if (b + 3 < p.bf) load_weights(rb, seg0 + (size_t)(b + 3) * SEG_BYTES, lane, n);
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
    }
    __syncthreads();
    if (e == 0) {
        // act row of each routed expert (the routing's order -> spec order)
        int pj = 0;
        if (lane < p.n_used) {
            const int id = rids[lane];
#pragma unroll
            for (int j = MAX_USED - 1; j >= 0; --j)
                if (j < p.n_used && sid[j] == id) pj = j;
        }
        float yv[MAX_USED], wv[MAX_USED];
#pragma unroll
        for (int q = 0; q < MAX_USED; ++q) {
            const int jq = __shfl(pj, q, WAVE);
            yv[q] = q < p.n_used && lane < TILE_ROWS ? ys[jq][lane] : 0.0f;
            wv[q] = q < p.n_used ? rwt[q] : 0.0f;
        }
        const int row = t * TILE_ROWS + lane;
        if (lane < TILE_ROWS && row < p.k) {
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < MAX_USED; ++q)
                if (q < p.n_used) {
                    const float prod = wv[q] * yv[q];
                    acc = acc + prod;
                }
            p.out[row] = p.res ? resv + acc : acc;
        }
    }
    if (t == 0 && e == 0) {
        if (lane == 0 && p.stats) {
            atomicAdd(&p.stats[0], 1);
            atomicAdd(&p.stats[1], 1);
        }
        for (int i = lane; i < 2 * p.n_expert; i += WAVE) p.slots[i] = SLOT_EMPTY;
    }
}

}  // namespace

int launch_moe_decode(const MoeDecodeLaunch &l, hipStream_t st) {
    if (l.k <= 0 || l.k % QK_K || l.k > KMAX || l.k / QK_K > GU_MAX_BLOCKS) return -1;
    if (l.n_ff <= 0 || l.n_ff % QK_K || l.n_ff / QK_K > DOWN_ACT_BLOCKS) return -1;
    if (l.n_expert <= 0 || l.n_expert > ROUTE_MAX_EXPERTS || l.n_used <= 0 ||
        l.n_used > MAX_USED || l.n_used > l.n_expert || l.nseq <= 0)
        return -1;
    DecodeParams p;
    p.w_gate = (const uint8_t *)l.w_gate;
    p.w_up = (const uint8_t *)l.w_up;
    p.w_down = (const uint8_t *)l.w_down;
    p.rw = l.router;
    p.x = l.x;
    p.res = l.res;
    p.out = l.out;
    p.logits = l.logits;
    p.est = l.est;
    p.slots = l.slots;
    p.act = l.act;
    p.spec_ids = l.spec_ids;
    p.ids_out = l.ids_out;
    p.w_out = l.w_out;
    p.stats = l.stats;
    p.gu_stride = l.gu_stride;
    p.down_stride = l.down_stride;
    p.k = l.k;
    p.n_expert = l.n_expert;
    p.n_used = l.n_used;
    p.n_ff = l.n_ff;
    p.gu_tiles = (l.n_ff + TILE_ROWS - 1) / TILE_ROWS;
    p.bf = l.n_ff / QK_K;
    p.down_tiles = (l.k + TILE_ROWS - 1) / TILE_ROWS;
    p.n_chain = (l.n_expert + CHAIN_EXPERTS - 1) / CHAIN_EXPERTS;
    p.n_gu = l.n_used * p.gu_tiles;
    p.nseq = l.nseq;
    p.norm_a = l.norm_a;
    p.norm_b = l.norm_b;
    p.norm_w = l.norm_w;
    p.norm_eps = l.norm_eps;
    p.norm_sum = l.norm_sum;
    p.polls = l.polls;
    if (p.polls < 0) return -1;
    if (p.norm_w && (l.nseq != 1 || !l.norm_a || !l.norm_b || !l.norm_sum || l.res != l.norm_sum ||
                     l.k > KMAX || l.k > XSUM_M * 512))
        return -1;
    if (p.norm_w)
        hipLaunchKernelGGL(moe_router_gateup<true>, dim3((p.n_chain + p.n_gu + 1) * l.nseq), dim3(512),
                           0, st, p);
    else
        hipLaunchKernelGGL(moe_router_gateup<false>, dim3((p.n_chain + p.n_gu + 1) * l.nseq), dim3(512),
                           0, st, p);
    hipLaunchKernelGGL(moe_down_route, dim3(p.down_tiles, l.nseq), dim3(64 * l.n_used), 0, st, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
