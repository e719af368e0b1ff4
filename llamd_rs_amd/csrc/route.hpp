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
                             RouteLds &sh, int32_t *ids, float *weights, float *logits_used) {
    const int lane = threadIdx.x & 63;
    expf_ref_tab_fill(sh.tab);
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
        float acc = -0.0f;
        int i = 0;
        for (; i + 8 <= n_expert; i += 8) {
            const float4 u = *(const float4 *)(sh.p + i);
            const float4 v = *(const float4 *)(sh.p + i + 4);
            acc = acc + u.x; acc = acc + u.y; acc = acc + u.z; acc = acc + u.w;
            acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
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
        }
    }
    if (resort) {
        bool live[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) live[j] = lane + WAVE * j < n_expert;
        unsigned taken = 0;
        wave_select(p, live, n_used, taken, sh.sorted);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane == 0 && ids) {
        // raw = p[chosen]; sum from -0.0, clamped; w = raw / sum (moe.rs:103-105)
        float wsum = -0.0f;
        for (int q = 0; q < n_used; ++q) wsum = wsum + sh.p[sh.sorted[q]];
        wsum = fmaxf(wsum, WEIGHT_SUM_FLOOR);
        for (int q = 0; q < n_used; ++q) {
            ids[q] = sh.sorted[q];
            weights[q] = sh.p[sh.sorted[q]] / wsum;
        }
    }
}


}  // namespace llamd
