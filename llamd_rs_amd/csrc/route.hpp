// route.hpp -- one-wave top-k routing core (moe.rs:73-113), shared by the
// router kernels and the expert matvec's routing prologue.
//
// n_expert <= 256 experts, lane l owning experts l, l+64, l+128, l+192.
// Top-k is n_sel rounds of a wave-wide (key desc, index asc) arg-max on one
// 64-bit key: exactly the first n_sel entries of Rust's stable sort_by in
// moe.rs:93-100 (a total order once ties go to the lower index).
#pragma once

#include "common.hpp"
#include "expf_ref.h"

namespace llamd {

constexpr int ROUTE_MAX_EXPERTS = 256;
constexpr int ROUTE_MAX_USED = 64;

constexpr int RW = ROUTE_MAX_EXPERTS / WAVE;  // experts per lane

struct RouteLds {
    uint64_t tab[32];  // expf_ref's table
    float p[ROUTE_MAX_EXPERTS];
    int sorted[ROUTE_MAX_USED + 1];
    int member[ROUTE_MAX_EXPERTS];      // route_finish with a given set: 1 for its experts
    unsigned ckey[ROUTE_MAX_USED];      // the given set's probability keys
    int cid[ROUTE_MAX_USED];            // and ids
};

// Order-preserving 32-bit key of a float (larger float, larger key); 0 is
// kept for "not a candidate".
__device__ __forceinline__ unsigned sort_key(float v) {
    const unsigned u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Select the n_sel best of val[] (desc, ties to the lower index); experts
// with live[j] false never win. Marks the chosen in `taken`. A NaN value
// ranks above +inf (the reference's comparator leaves NaN unordered). Each
// round: a 32-bit wave max of the keys, then a ballot per register column
// finds the lowest index holding that key (index lane + 64 j rises with j).
__device__ void wave_select(const float val[RW], const bool live[RW], int n_sel, unsigned &taken,
                            int *sorted) {
    const int lane = threadIdx.x & 63;
    unsigned key[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) key[j] = live[j] ? sort_key(val[j]) : 0u;
    for (int r = 0; r < n_sel; ++r) {
        unsigned b = 0u;
#pragma unroll
        for (int j = 0; j < RW; ++j) b = max(b, key[j]);
        const unsigned m = (unsigned)wave_reduce((int)b, 0, [](int x, int y) {
            return (int)max((unsigned)x, (unsigned)y);
        });
        int bi = 0x7FFFFFFF;
        if (m != 0u) {
#pragma unroll
            for (int j = RW - 1; j >= 0; --j) {
                const unsigned long long mask = __ballot(key[j] == m);
                if (mask) bi = 64 * j + __ffsll((long long)mask) - 1;
            }
            if ((bi & 63) == lane) {
                taken |= 1u << (bi >> 6);
#pragma unroll
                for (int j = 0; j < RW; ++j)
                    if (j == (bi >> 6)) key[j] = 0u;
            }
        }
        if (lane == 0) sorted[r] = bi;
    }
}

// softmax of this lane's logits l[] exactly as moe.rs:82-87 (max fold, exp,
// sequential total from -0.0, divide); if `resort`, select by probability;
// then gather, clamp and renormalise (moe.rs:103-105).
__device__ void route_finish(const float l[RW], int n_expert, int n_used, bool resort,
                             RouteLds &sh, int32_t *ids, float *weights, float *logits_used,
                             const int *given = nullptr, bool tab_ready = false,
                             float *probs_out = nullptr) {
    const int lane = threadIdx.x & 63;
    if (!tab_ready) expf_ref_tab_fill(sh.tab);
    float m = -INFINITY;  // f32::max fold: NaN-ignoring, order-free
#pragma unroll
    for (int j = 0; j < RW; ++j)
        if (lane + WAVE * j < n_expert) m = fmaxf(m, l[j]);
    const float mx = wave_reduce(m, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    float p[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        p[j] = 0.0f;
        if (i < n_expert) {
            p[j] = expf_ref_tab(l[j] - mx, sh.tab);
            sh.p[i] = p[j];
            if (logits_used) logits_used[i] = l[j];
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float total = 0.0f;
    if (lane == 0) {
        // 64 values per step: the LDS reads are issued together and retire
        // in order, so the dependent adds start on the first
        float acc = -0.0f;
        int i = 0;
        for (; i + 64 <= n_expert; i += 64) {
            float4 u[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) u[j] = *(const float4 *)(sh.p + i + 4 * j);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                acc = acc + u[j].x; acc = acc + u[j].y; acc = acc + u[j].z; acc = acc + u[j].w;
            }
        }
        for (; i < n_expert; ++i) acc = acc + sh.p[i];
        total = acc;
    }
    total = __shfl(total, 0, WAVE);
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        if (i < n_expert) {
            p[j] = p[j] / total;
            sh.p[i] = p[j];
            if (probs_out) probs_out[i] = p[j];
        }
    }
    bool ranked = false;
    if (resort && given) {
        // The set is known (certified from the estimates): order its n_used
        // experts by (probability desc, index asc) -- after checking that
        // every member's probability key lies strictly above every other
        // expert's, so the set is the top n_used by probability; else the
        // full selection below runs.
        const int id = lane < n_used ? given[lane] : 0;
        // membership flags in LDS (one wave: a wave barrier orders them)
#pragma unroll
        for (int j = 0; j < RW; ++j)
            if (lane + WAVE * j < n_expert) sh.member[lane + WAVE * j] = 0;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (lane < n_used) sh.member[id] = 1;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        unsigned lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            const int i = lane + WAVE * j;
            if (i < n_expert) {
                const unsigned k = sort_key(p[j]);
                if (sh.member[i]) lo = min(lo, k);
                else hi = max(hi, k);
            }
        }
        lo = (unsigned)wave_reduce((int)lo, -1, [](int a, int b) { return (int)min((unsigned)a, (unsigned)b); });
        hi = (unsigned)wave_reduce((int)hi, 0, [](int a, int b) { return (int)max((unsigned)a, (unsigned)b); });
        if (lo > hi) {
            // each member's place: how many members beat it (the n_used
            // (key, id) pairs read back from LDS together)
            const unsigned key = lane < n_used ? sort_key(sh.p[id]) : 0u;
            if (lane < n_used) {
                sh.ckey[lane] = key;
                sh.cid[lane] = id;
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            int rank = 0;
            for (int r = 0; r < n_used; r += 8) {
                unsigned kr[8];
                int ir[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    kr[u] = sh.ckey[min(r + u, n_used - 1)];
                    ir[u] = sh.cid[min(r + u, n_used - 1)];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    rank += (r + u < n_used && (kr[u] > key || (kr[u] == key && ir[u] < id))) ? 1 : 0;
            }
            if (lane < n_used) sh.sorted[rank] = id;
            ranked = true;
        }
    }
    if (resort && !ranked) {
        bool live[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) live[j] = lane + WAVE * j < n_expert;
        unsigned taken = 0;
        wave_select(p, live, n_used, taken, sh.sorted);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (ids) {
        // raw = p[chosen]; sum from -0.0 in routing order, clamped; w = raw /
        // sum (moe.rs:103-105). Lane q gathers raw q; lane 0 adds them in order.
        const int id = lane < n_used ? sh.sorted[lane] : 0;
        const float raw = lane < n_used ? sh.p[id] : 0.0f;
        // the first 8 by readlane with immediate lane numbers (no LDS round
        // trip), any beyond one at a time; -0.0 past n_used changes nothing
        float wsum = -0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(raw), u));
            wsum = wsum + (u < n_used ? r : -0.0f);
        }
        for (int q = 8; q < n_used; ++q)
            wsum = wsum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(raw), q));
        wsum = fmaxf(wsum, WEIGHT_SUM_FLOOR);
        if (lane < n_used) {
            ids[lane] = id;
            weights[lane] = raw / wsum;
        }
    }
}

// ---- the router fold and its certified estimate ------------------------------
//
// The reference's logit is a sequential f32 fold of the row's products from
// -0.0 (moe.rs:73-80 via the f32 matvec). seq_fold is that fold, run by one
// lane over products parked in LDS (n4 float4s, a multiple of 32).
__device__ __forceinline__ float seq_fold(const float4 *prod, int n4) {
    // 128 products per step: the 16-byte LDS reads are issued together and
    // retire in order, so the adds start on the first while the rest arrive
    float acc = -0.0f;
    for (int i = 0; i < n4; i += 32) {
        float4 v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = prod[i + j];
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            acc = acc + v[j].x;
            acc = acc + v[j].y;
            acc = acc + v[j].z;
            acc = acc + v[j].w;
        }
    }
    return acc;
}

// The exact sum T of the same products (in double) and a bound E with
// |seq_fold - T| <= E, from the whole wave in ~1 us instead of the fold's ~7.
//
// Recursive summation S_k = fl(S_{k-1} + p_k) commits an error of at most
// u |S_{k-1} + p_k| per step (u = 2^-24, round to nearest; additions whose
// result is subnormal are exact). With D_k = |S_k - T_k| (T_k the exact
// prefix sums) this gives D_k <= (1 + u) D_{k-1} + u |T_k|, hence
// D_n <= u (1 + u)^n sum_k |T_k| (Higham, Accuracy and Stability of Numerical
// Algorithms, 2nd ed., section 4.2). The prefix sums are formed in double
// (each lane a contiguous run of n/64 products, then a wave scan); the slack
// factor 1 + 2^-10 covers (1 + u)^2048 and the double roundings, and
// 2^-40 sum |p| covers the error of T itself. Non-finite products make T or
// E non-finite, which callers treat as "no estimate".
__device__ __forceinline__ void fold_estimate(const float *prod, int n, double &T, double &E) {
    const int lane = threadIdx.x & 63;
    const int len = n / WAVE;  // n is a multiple of 256: len is a multiple of 4
    const float4 *seg = (const float4 *)(prod + lane * len);
    double s = 0.0, a = 0.0;
    for (int j = 0; j < len / 4; ++j) {
        const float4 v = seg[j];
        s += (double)v.x; s += (double)v.y; s += (double)v.z; s += (double)v.w;
        a += fabs((double)v.x) + fabs((double)v.y) + fabs((double)v.z) + fabs((double)v.w);
    }
    const double incl = wave_inclusive_sum(s);
    double run = incl - s;  // exclusive prefix: the sum of the products before this run
    double pabs = 0.0;
    for (int j = 0; j < len / 4; ++j) {
        const float4 v = seg[j];
        run += (double)v.x; pabs += fabs(run);
        run += (double)v.y; pabs += fabs(run);
        run += (double)v.z; pabs += fabs(run);
        run += (double)v.w; pabs += fabs(run);
    }
    T = readlane63(incl);
    const double sum_prefix = wave_sum_d(pabs), sum_abs = wave_sum_d(a);
    E = 0x1p-24 * (1.0 + 0x1p-10) * sum_prefix + 0x1p-40 * sum_abs;
}

// Publication of one value per expert between workgroups of one launch, with
// no cache-wide fences: the value and its "ready" mark travel in ONE 64-bit
// word written with a relaxed agent-scope atomic store and polled with
// relaxed agent-scope atomic loads (coherent across the XCDs' L2s; an
// agent-scope release or acquire would write back or invalidate a whole L2
// per use). A slot holds SLOT_EMPTY until its word is stored; the consumer of
// the last call resets the slots to SLOT_EMPTY for the next.
constexpr unsigned long long SLOT_EMPTY = ~0ull;

__device__ __forceinline__ void slot_store(unsigned long long *slot, unsigned lo, unsigned hi) {
    __hip_atomic_store(slot, ((unsigned long long)hi << 32) | lo, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait for the lane's RW slots (base + lane + 64 j, j < RW, those
// with live[j]) to be filled: at most `polls` passes (about a quarter of a
// second at the default 2^18). Every pass loads all slots still empty
// together, so one round trip to memory serves all of them. A producer
// normally has a lower workgroup index and is already placed, but HIP does
// not promise dispatch order, so every caller must survive a slot left
// SLOT_EMPTY: the MoE decode kernel then computes the value it waited for
// itself (wait_logits), the same bits.
//
// While the producers are still at work, one lane watches one slot (the
// last one, `watch`, normally among the last filled) and the others wait:
// hundreds of waiting workgroups polling every slot would put tens of
// thousands of uncached loads per microsecond on the few lines that hold the
// slots. The passes spent watching count against `polls`.
__device__ __forceinline__ void slots_wait(const unsigned long long *base, const bool live[RW],
                                           unsigned long long v[RW], int polls, int watch = -1) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < RW; ++j) v[j] = live[j] ? SLOT_EMPTY : 0ull;
    if (watch >= 0) {
        int used = 0;
        if (lane == 0) {
            while (used < polls &&
                   __hip_atomic_load(base + watch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == SLOT_EMPTY) {
                ++used;
                __builtin_amdgcn_s_sleep(2);
            }
        }
        polls -= __shfl(used, 0, WAVE);
    }
    for (int it = 0; it < polls; ++it) {
#pragma unroll
        for (int j = 0; j < RW; ++j)
            if (v[j] == SLOT_EMPTY)
                v[j] = __hip_atomic_load(base + lane + WAVE * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool pending = false;
#pragma unroll
        for (int j = 0; j < RW; ++j) pending = pending || v[j] == SLOT_EMPTY;
        if (!pending) break;
        __builtin_amdgcn_s_sleep(2);
    }
}

}  // namespace llamd
