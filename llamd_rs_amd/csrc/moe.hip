// moe.hip -- router, top-k routing, expert combine, argmax, and the f32 /
// Q8_0 matvecs of the reference's fallback path (model.rs:253-262).
//
// EXPERT SELECTION IS BIT-EXACT. The reference routes on logits from a
// SEQUENTIAL f32 sum (the F32 router goes through matvec_quant's fallback,
// crates/llamd-models/src/model.rs:253-262) followed by softmax, a stable sort
// with ties to the lower index, and renormalisation (moe.rs:73-113). A
// sequential sum of 2048 terms is a 2048-step dependency chain; doing it on
// every token would cost microseconds on a path that otherwise takes one.
// Instead:
//   1. router_bound: one wave per expert computes the logit in double (the
//      "centre", within ~1e-12 relative of the exact sum of the rounded
//      products) and a rigorous radius R such that the reference's f32 fold
//      is within R of the centre. R uses the running-error bound for
//      recursive summation: |fold - exact| <= u/(1-u) * sum_{k>=2} |S^_k| and
//      |S^_k| <= |S_k| + gamma_{k-1} A_k (S_k exact prefix sums, A_k prefix
//      sums of |products|), with the S_k from a double-precision scan.
//   2. moe_route: ranks experts by centre. If every decision that fixes the
//      chosen ids and their order is separated by more than the two radii
//      (and no chosen probability can underflow), the reference's ids are
//      provably these. Otherwise -- or when exact mode is requested -- the
//      workgroup recomputes every logit as the reference's exact sequential
//      fold and routes on those bits, with glibc-identical expf.
// Probabilities and weights are then computed with the reference's formulas
// and order of operations. The ids are therefore always identical to the CPU
// path; the weights are identical in exact mode and within a few ulp
// otherwise (REDUCTION).
#include <float.h>

#include "common.hpp"
#include "expf_ref.h"
#include "launch.hpp"
#include "q8k_wave.hpp"

namespace llamd {
namespace {

// Phase timestamps for measurement builds; compiled out otherwise.
#ifndef LLAMD_PROBE
#define LLAMD_PROBE(slot) ((void)0)
#endif
#ifndef LLAMD_DEBUG_DECIDE
#define LLAMD_DEBUG_DECIDE(i, v) ((void)0)
#endif

constexpr int ROUTE_MAX_EXPERTS = 256;
constexpr int ROUTE_MAX_USED = 64;

// ---- routing core (one wave), shared by the kernels below -----------------
// n_expert <= 256 experts, lane l owning experts l, l+64, l+128, l+192. Top-k
// is n_sel rounds of a wave-wide (key desc, index asc) arg-max: exactly the
// first n_sel entries of Rust's stable sort_by in moe.rs:93-100 (a total
// order once ties go to the lower index).
constexpr int RW = ROUTE_MAX_EXPERTS / WAVE;  // experts per lane

struct RouteLds {
    float p[ROUTE_MAX_EXPERTS];
    int sorted[ROUTE_MAX_USED + 1];
};

__device__ __forceinline__ bool beats(double av, int ai, double bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ void wave_best(double &v, int &i) { wave_argmax(v, i, (double)-INFINITY); }

__device__ __forceinline__ double wave_max_d(double v) {
    return wave_reduce(v, (double)-INFINITY, [](double a, double b) { return fmax(a, b); });
}

// Select the n_sel best of key[] (per-lane registers, invalid = -inf with
// index INT_MAX); marks the chosen in `taken`, writes their indices to sorted.
__device__ void wave_select(const double key[RW], int n_sel, unsigned &taken, int *sorted) {
    const int lane = threadIdx.x & 63;
    for (int r = 0; r < n_sel; ++r) {
        double bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            const bool live = !(taken & (1u << j)) && key[j] != -INFINITY;
            argmax_step(bv, bi, live ? key[j] : (double)-INFINITY, live ? lane + WAVE * j : 0x7FFFFFFF);
        }
        wave_best(bv, bi);
        taken |= (bi != 0x7FFFFFFF && (bi & 63) == lane) ? 1u << (bi >> 6) : 0u;
        if (lane == 0) sorted[r] = bi;
    }
}

// Is the order of the n_used best centres (and the set) provably the
// reference's? c/r: this lane's centres and radii. Returns the verdict on
// every lane and leaves the selection in sh.sorted.
__device__ bool route_decide(const double c[RW], const double r[RW], int n_expert, int n_used,
                             int force_exact, RouteLds &sh) {
    const int lane = threadIdx.x & 63;
    double key[RW];
    double bad = 0.0;
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const bool live = lane + WAVE * j < n_expert;
        if (live && (isnan(c[j]) || isinf(c[j]))) bad = 1.0;
        key[j] = live && !isnan(c[j]) ? c[j] : -INFINITY;
    }
    bad = wave_max_d(bad);
    LLAMD_PROBE(6);
    unsigned taken = 0;
    wave_select(key, n_used, taken, sh.sorted);
    LLAMD_PROBE(7);
    // the largest c + r among experts not chosen
    double mrest = -DBL_MAX;
#pragma unroll
    for (int j = 0; j < RW; ++j)
        if (lane + WAVE * j < n_expert && !(taken & (1u << j))) mrest = fmax(mrest, c[j] + r[j]);
    mrest = wave_max_d(mrest);
    __builtin_amdgcn_wave_barrier();
    // centre and radius of the chosen, in order, gathered by lane 0 via LDS
    __shared__ double cr[2][ROUTE_MAX_USED];
    for (int q = 0; q < n_used; ++q) {
        const int i = sh.sorted[q];
        if ((i & 63) == lane) {
#pragma unroll
            for (int j = 0; j < RW; ++j)
                if ((i >> 6) == j) { cr[0][q] = c[j]; cr[1][q] = r[j]; }
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    int ok = 0;
    if (lane == 0) {
        bool good = !force_exact && bad == 0.0 && sh.sorted[0] != 0x7FFFFFFF;
        const double cmax = cr[0][0];
        // Separation required on top of the two radii so the reference's
        // probabilities exp(l - max) / total cannot collapse to equal floats
        // (where its tie rule, index order, would decide): 1e-6 relative
        // keeps well clear of f32 rounding.
        const double rel = 1e-6 * (1.0 + fabs(cmax));
        for (int q = 0; good && q + 1 < n_used; ++q)
            good = (cr[0][q] - cr[1][q]) - (cr[0][q + 1] + cr[1][q + 1]) > rel * (1.0 + fabs(cr[0][q]));
        if (good && n_used < n_expert)
            good = (cr[0][n_used - 1] - cr[1][n_used - 1]) - mrest > rel * (1.0 + fabs(cr[0][n_used - 1]));
        // chosen probabilities must stay far from exp() underflow, where
        // zero-probability ties would fall back to index order
        if (good) good = cr[0][n_used - 1] - cmax > -80.0;
        ok = good ? 1 : 0;
        LLAMD_DEBUG_DECIDE(0, bad);
        LLAMD_DEBUG_DECIDE(1, mrest);
        LLAMD_DEBUG_DECIDE(2, (double)sh.sorted[0]);
        for (int q = 0; q < n_used && q < 8; ++q) {
            LLAMD_DEBUG_DECIDE(3 + 2 * q, cr[0][q]);
            LLAMD_DEBUG_DECIDE(4 + 2 * q, cr[1][q]);
        }
    }
    return __shfl(ok, 0, WAVE) != 0;
}

// softmax of this lane's logits l[] exactly as moe.rs:82-87 (max fold, exp,
// sequential total from -0.0, divide); if `resort`, select by probability;
// then gather, clamp and renormalise (moe.rs:103-105).
__device__ void route_finish(const float l[RW], int n_expert, int n_used, bool resort,
                             RouteLds &sh, int32_t *ids, float *weights, float *logits_used) {
    const int lane = threadIdx.x & 63;
    double m = -INFINITY;  // f32::max fold: NaN-ignoring, order-free
#pragma unroll
    for (int j = 0; j < RW; ++j)
        if (lane + WAVE * j < n_expert && !isnan(l[j])) m = fmax(m, (double)l[j]);
    const float mx = (float)wave_max_d(m);
    float p[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        p[j] = 0.0f;
        if (i < n_expert) {
            p[j] = expf_ref(l[j] - mx);
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
        double key[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) key[j] = lane + WAVE * j < n_expert ? (double)p[j] : -INFINITY;
        // probabilities are >= 0, so -inf only marks absent experts
        unsigned taken = 0;
        wave_select(key, n_used, taken, sh.sorted);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane == 0) {
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

// Loads that must see other workgroups' stores from the same kernel: bypass
// the per-CU vector cache.
__device__ __forceinline__ double load_dev(const double *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true in exactly one workgroup: the last of `n` to arrive. The
// counter returns to zero for the next launch.
__device__ bool last_arrival(int *counter, int n) {
    __shared__ int is_last;
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        const int prev = atomicAdd(counter, 1);
        is_last = prev == n - 1;
        if (is_last) {
            __threadfence();
            atomicExch(counter, 0);
        }
    }
    __syncthreads();
    return is_last != 0;
}

struct RouterArgs {
    const float *w;          // f32 router [n_expert][k]
    const float *x;          // [k]
    int n_expert, k, n_used, force_exact;
    float *logit_f;          // [n_expert] float(centre)
    double *centre, *radius; // [n_expert]
    float *exact_l;          // [n_expert] reference fold (exact pass)
    int32_t *ids;            // [n_used]
    float *weights;          // [n_used]
    float *logits_used;      // [n_expert] the logits the routing used
    int *flag;               // 1: the exact pass must run
    int *counters;           // [2] arrival counters (zero between launches)
    int *stats;              // [2] calls, calls that needed the exact pass
    // fused Q8_K quantisation of x for the expert matvecs
    int8_t *xq;
    float *xd;
    int xblocks;
};

// The reference's fold s = -0.0; s += w[t] * x[t] (model.rs:253-262) for every
// row, by one 256-thread workgroup: 32-column tiles of all rows are staged in
// LDS (four tiles in flight) and thread r adds row r's products in order.
// Results land in sh.p (as scratch) indexed by row.
__device__ void exact_fold_wg(const RouterArgs &a, RouteLds &sh, float *lds, int lds_floats) {
    const int tid = threadIdx.x;
    // columns per tile: two tiles of n_expert x (tc + 1) floats must fit
    int tc = 32;
    while (tc > 4 && 2 * a.n_expert * (tc + 1) > lds_floats) tc /= 2;
    const int ld = tc + 1;
    const int ntile = a.k / tc;
    auto stage = [&](int t) {
        float *dst = lds + (t & 1) * a.n_expert * ld;
        for (int idx = tid; idx < a.n_expert * (tc / 4); idx += blockDim.x) {
            const int r = idx / (tc / 4), c4 = idx % (tc / 4);
            const float4 v = *(const float4 *)(a.w + (size_t)r * a.k + (size_t)t * tc + 4 * c4);
            float *d = dst + r * ld + 4 * c4;
            d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
        }
    };
    stage(0);
    float acc = -0.0f;
    for (int t = 0; t < ntile; ++t) {
        __syncthreads();
        if (t + 1 < ntile) stage(t + 1);
        if (tid < a.n_expert) {
            const float *row = lds + (t & 1) * a.n_expert * ld + tid * ld;
            const float *xs = a.x + (size_t)t * tc;
            for (int c = 0; c < tc; ++c) {
                const float p = row[c] * xs[c];
                acc = acc + p;
            }
        }
    }
    __syncthreads();
    if (tid < a.n_expert) sh.p[tid] = acc;
    __syncthreads();
}

// ---- 1. router logits with a rigorous error radius, then the fast route ----
// Workgroups [0, nr): one wave per expert row; lane l owns elements
// [l*k/64, (l+1)*k/64). Workgroups [nr, nr + nq): Q8_K of x, a wave per block.
// The last router workgroup to finish ranks the centres and routes when the
// order is proven; otherwise it raises `flag` for router_exact.
__global__ __launch_bounds__(256) void router_fast(RouterArgs a) {
    const int nr = (a.n_expert + 3) / 4;
    const int lane = threadIdx.x & 63;
    if ((int)blockIdx.x >= nr) {
        const int blk = ((int)blockIdx.x - nr) * 4 + (threadIdx.x >> 6);
        if (blk < a.xblocks) {
            const float4 xv = *(const float4 *)(a.x + (size_t)blk * QK_K + 4 * lane);
            const float v[4] = {xv.x, xv.y, xv.z, xv.w};
            quantize_block_wave(v, lane, a.xq + (size_t)blk * QK_K, a.xd + blk);
        }
        return;
    }
    LLAMD_PROBE(0);
    // Coalesced loads staged through LDS so that each lane then owns 32
    // CONTIGUOUS elements (the prefix-sum bound needs index order). Rows are
    // padded by 4 floats every 32 so the per-lane 16-byte reads of a 16-lane
    // group hit disjoint banks.
    constexpr int PAD = 36;  // floats per 32-element lane chunk
    __shared__ float stage_flat[5 * 64 * PAD];  // x, then one row per wave
    float (*stage)[64 * PAD] = (float (*)[64 * PAD])stage_flat;
    const int wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    const int per = a.k / 64;  // elements per lane (32 at k = 2048)
    for (int v = wv; v < 5; v += 4) {
        const float *src = v == 0 ? a.x : a.w + (size_t)(blockIdx.x * 4 + v - 1) * a.k;
        if (v == 0 || blockIdx.x * 4 + v - 1 < a.n_expert)
            for (int e4 = lane; e4 < a.k / 4; e4 += 64) {
                const float4 q = *(const float4 *)(src + 4 * e4);
                const int e = 4 * e4;
                *(float4 *)(&stage[v][(e / per) * PAD + e % per]) = q;
            }
    }
    __syncthreads();
    if (row < a.n_expert && per <= 32) {
        const float *xs = &stage[0][lane * PAD];
        const float *ws = &stage[1 + wv][lane * PAD];
        float pr[32];
        double tot = 0.0, absum = 0.0;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            if (i < per) {
                const float4 w4 = *(const float4 *)(ws + i);
                const float4 x4 = *(const float4 *)(xs + i);
                // the reference's rounded products
                pr[i] = w4.x * x4.x; pr[i + 1] = w4.y * x4.y;
                pr[i + 2] = w4.z * x4.z; pr[i + 3] = w4.w * x4.w;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    tot += (double)pr[i + j];
                    absum += fabs((double)pr[i + j]);
                }
            }
        }
        // exclusive prefix of the lane totals, then |S_k| over this lane's k
        const double pre = wave_inclusive_sum(tot) - tot;
        double sabs = 0.0, run = pre;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            if (i < per) {
                run += (double)pr[i];
                if (lane * per + i >= 1) sabs += fabs(run);
            }
        }
        const double S = wave_sum_d(tot);
        const double A = wave_sum_d(absum);
        const double SA = wave_sum_d(sabs);
        if (lane == 0) {
            const double u = 0x1p-24;
            const double n = (double)a.k;
            const double gam = n * u / (1.0 - n * u);
            // |fold - S| <= u/(1-u) sum|S^_k|, |S^_k| <= |S_k| + gamma A; the
            // double-precision scan and sums add far less than 1e-9 A
            const double r = u / (1.0 - u) * (SA + n * gam * A) * (1.0 + 1e-6) + 1e-9 * A + 1e-30;
            a.centre[row] = S;
            a.radius[row] = r;
            a.logit_f[row] = (float)S;
        }
    }
    LLAMD_PROBE(1);
    if (!last_arrival(&a.counters[0], nr)) return;
    LLAMD_PROBE(2);
    __shared__ RouteLds sh;
    __shared__ int verdict;
    if (threadIdx.x < WAVE) {
        double c[RW], r[RW];
        float l[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            const int i = lane + WAVE * j;
            c[j] = i < a.n_expert ? load_dev(&a.centre[i]) : 0.0;
            r[j] = i < a.n_expert ? load_dev(&a.radius[i]) : 0.0;
            l[j] = i < a.n_expert ? load_dev(&a.logit_f[i]) : 0.0f;
        }
        LLAMD_PROBE(3);
        const bool ok = route_decide(c, r, a.n_expert, a.n_used, a.force_exact, sh);
        LLAMD_PROBE(4);
        if (lane == 0) {
            verdict = ok ? 0 : 1;
            *a.flag = a.force_exact ? 1 : 0;  // exact mode: router_exact runs next
            if (a.stats) a.stats[0] += 1;
        }
        if (ok) route_finish(l, a.n_expert, a.n_used, false, sh, a.ids, a.weights, a.logits_used);
        LLAMD_PROBE(5);
    }
    __syncthreads();
    if (verdict == 0 || a.force_exact) return;
    // The order was not provable (rare): this workgroup computes the
    // reference's exact sequential fold for every row and routes on it.
    exact_fold_wg(a, sh, stage_flat, 5 * 64 * PAD);
    if (threadIdx.x < WAVE) {
        float l[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            const int i = lane + WAVE * j;
            l[j] = i < a.n_expert ? sh.p[i] : 0.0f;
        }
        route_finish(l, a.n_expert, a.n_used, true, sh, a.ids, a.weights, a.logits_used);
        if (lane == 0 && a.stats) a.stats[1] += 1;
    }
}

// ---- 2. the reference's exact fold, only when router_fast could not prove --
// One workgroup (one wave) per expert row: products of 64 columns at a time
// are staged in LDS and lane 0 adds them in order, s = -0.0; s += w[t]*x[t]
// (model.rs:253-262), while the next 64 columns load. The last row to finish
// routes on the exact logits with the reference's own sort.
__global__ __launch_bounds__(64) void router_exact(RouterArgs a) {
    if (__hip_atomic_load(a.flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) return;
    const int row = blockIdx.x;
    const int lane = threadIdx.x;
    __shared__ float prod[2][64];
    const float *wr = a.w + (size_t)row * a.k;
    float wv = lane < a.k ? wr[lane] : 0.0f;
    float xv = lane < a.k ? a.x[lane] : 0.0f;
    float acc = -0.0f;
    int buf = 0;
    for (int t0 = 0; t0 < a.k; t0 += 64) {
        prod[buf][lane] = wv * xv;
        if (t0 + 64 + lane < a.k) {
            wv = wr[t0 + 64 + lane];
            xv = a.x[t0 + 64 + lane];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (lane == 0) {
            const int cols = min(64, a.k - t0);
            for (int c = 0; c < cols; ++c) acc = acc + prod[buf][c];
        }
        buf ^= 1;
    }
    if (lane == 0) a.exact_l[row] = acc;
    if (!last_arrival(&a.counters[1], a.n_expert)) return;
    __shared__ RouteLds sh;
    float l[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        l[j] = i < a.n_expert ? load_dev(&a.exact_l[i]) : 0.0f;
    }
    route_finish(l, a.n_expert, a.n_used, true, sh, a.ids, a.weights, a.logits_used);
    if (lane == 0 && a.stats) a.stats[1] += 1;
}

// Routing from given logits (llamd_hip_route / llamd_fwd_router): exact
// inputs, radius 0; ties or near-collapses go through the reference's sort.
__global__ __launch_bounds__(64) void route_logits(const float *logits, int n_expert, int n_used,
                                                   int32_t *ids, float *weights) {
    __shared__ RouteLds sh;
    const int lane = threadIdx.x;
    double c[RW], r[RW];
    float l[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        l[j] = i < n_expert ? logits[i] : 0.0f;
        c[j] = (double)l[j];
        r[j] = 0.0;
    }
    const bool ok = route_decide(c, r, n_expert, n_used, 0, sh);
    route_finish(l, n_expert, n_used, !ok, sh, ids, weights, nullptr);
}

// ---- 3. weighted combine + residual (layer.rs:245-258, 281-287) -------------
// out[i] = res[i] + (((0 + w0*d0[i]) + w1*d1[i]) + ...), experts in routing order.
// blockIdx.y = token (prefill); down is [n_tok][n_used][n_embd].
__global__ void moe_combine(const float *down, const float *weights, const float *res, float *out,
                            int n_used, int n_embd) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_embd) return;
    const size_t tok = blockIdx.y;
    down += tok * n_used * n_embd;
    weights += tok * n_used;
    if (res) res += tok * n_embd;
    out += tok * n_embd;
    float acc = 0.0f;
    for (int e = 0; e < n_used; ++e) {
        const float p = weights[e] * down[(size_t)e * n_embd + i];
        acc = acc + p;
    }
    out[i] = res ? res[i] + acc : acc;
}

// ---- 4. argmax: strict '>', lowest index wins (device_forward.rs:23-37) -----
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(256) void argmax_partial(const float *x, int n, int ld, float *pv,
                                                      int *pi) {
    const int seq = blockIdx.y;
    const float *xs = x + (size_t)seq * ld;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float v = xs[i];
        if (!isnan(v)) better(bv, bi, v, i);
    }
    wave_argmax(bv, bi, -INFINITY);
    __shared__ float sv[4];
    __shared__ int si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) better(bv, bi, sv[w], si[w]);
        pv[(size_t)seq * gridDim.x + blockIdx.x] = bv;
        pi[(size_t)seq * gridDim.x + blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(64) void argmax_final(const float *x, int ld, const float *pv,
                                                   const int *pi, int nparts, int32_t *out) {
    const int seq = blockIdx.x;
    const int lane = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = lane; i < nparts; i += 64)
        better(bv, bi, pv[(size_t)seq * nparts + i], pi[(size_t)seq * nparts + i]);
    wave_argmax(bv, bi, -INFINITY);
    if (lane == 0) {
        // the reference's incumbent is index 0: a NaN there is never beaten,
        // and when nothing beats -inf the answer stays 0
        const float v0 = x[(size_t)seq * ld];
        out[seq] = (isnan(v0) || bi == 0x7FFFFFFF) ? 0 : bi;
    }
}

// ---- 5. Q8_0 matvec (R8: dequantize then f32 dot) ----------------------------
// Planar layout: qs [rows][k] int8, then d [rows][k/32] f16. One wave handles
// ROWS_PER_WAVE rows; lane l owns Q8_0 blocks l, l+64, ... and loads each
// block's 32 activations once for all its rows. Products are d*q rounded
// (the dequantized weight, exact) times x, accumulated with FMA; within
// REDUCTION of the reference's sequential sum.
constexpr int Q80_ROWS_PER_WAVE = 4;

__global__ __launch_bounds__(256) void q8_0_mv(const int8_t *qs, const uint16_t *dp, const float *x,
                                               float *y, int rows, int k) {
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * Q80_ROWS_PER_WAVE;
    if (r0 >= rows) return;
    const int nb = k / 32;
    float acc[Q80_ROWS_PER_WAVE];
#pragma unroll
    for (int r = 0; r < Q80_ROWS_PER_WAVE; ++r) acc[r] = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        float xv[32];
        const float4 *xp = (const float4 *)(x + (size_t)b * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = xp[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < Q80_ROWS_PER_WAVE; ++r) {
            const int row = r0 + r;
            if (row >= rows) break;
            const uint4 *qp = (const uint4 *)(qs + (size_t)row * k + (size_t)b * 32);
            const uint4 qa = qp[0], qb = qp[1];
            const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            const float d = f16_bits_to_f32(dp[(size_t)row * nb + b]);
            float s = acc[r];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int q = (int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 0xFF);
                const float wv = d * (float)q;
                s = fmaf(wv, xv[i], s);
            }
            acc[r] = s;
        }
    }
#pragma unroll
    for (int r = 0; r < Q80_ROWS_PER_WAVE; ++r) {
        const float t = wave_sum_f(acc[r]);
        if (lane == 0 && r0 + r < rows) y[r0 + r] = t;
    }
}

__global__ __launch_bounds__(256) void q8_0_dequant(const int8_t *qs, const uint16_t *dp, float *out,
                                                    size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = f16_bits_to_f32(dp[i / 32]) * (float)qs[i];
}

// Plain f32 matvec (one wave per row, FMA accumulation): Backend-style helper.
__global__ __launch_bounds__(256) void f32_mv(const float *w, const float *x, float *y, int rows,
                                              int k) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *wr = w + (size_t)row * k;
    float s = 0.0f;
    for (int i = lane; i < k; i += 64) s = fmaf(wr[i], x[i], s);
    s = wave_sum_f(s);
    if (lane == 0) y[row] = s;
}

}  // namespace

int launch_router(const RouterLaunch &l, hipStream_t st) {
    RouterArgs a;
    a.w = l.w; a.x = l.x; a.n_expert = l.n_expert; a.k = l.k; a.n_used = l.n_used;
    a.force_exact = l.force_exact; a.logit_f = l.logit_f; a.centre = l.centre;
    a.radius = l.radius; a.exact_l = l.exact_l; a.ids = l.ids; a.weights = l.weights;
    a.logits_used = l.logits_used; a.flag = l.flag; a.counters = l.counters; a.stats = l.stats;
    a.xq = l.xq; a.xd = l.xd; a.xblocks = l.xblocks;
    const int nr = (l.n_expert + 3) / 4, nq = (l.xblocks + 3) / 4;
    hipLaunchKernelGGL(router_fast, dim3(nr + nq), dim3(256), 0, st, a);
    // exact mode: the reference's fold on every row, one workgroup per row
    if (l.force_exact) hipLaunchKernelGGL(router_exact, dim3(l.n_expert), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_route_logits(const float *logits, int n_expert, int n_used, int32_t *ids,
                        float *weights, hipStream_t st) {
    hipLaunchKernelGGL(route_logits, dim3(1), dim3(64), 0, st, logits, n_expert, n_used, ids,
                       weights);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_moe_combine(const float *down, const float *weights, const float *res, float *out,
                       int n_used, int n_embd, int n_tok, hipStream_t st) {
    hipLaunchKernelGGL(moe_combine, dim3((n_embd + 255) / 256, n_tok), dim3(256), 0, st, down,
                       weights, res, out, n_used, n_embd);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int argmax_parts(int n) {
    int parts = (n + 4095) / 4096;
    if (parts < 1) parts = 1;
    if (parts > 1024) parts = 1024;
    return parts;
}

int launch_argmax(const float *x, int n, int ld, int nseq, float *pv, int *pi, int32_t *out,
                  hipStream_t st) {
    const int parts = argmax_parts(n);
    hipLaunchKernelGGL(argmax_partial, dim3(parts, nseq), dim3(256), 0, st, x, n, ld, pv, pi);
    hipLaunchKernelGGL(argmax_final, dim3(nseq), dim3(64), 0, st, x, ld, pv, pi, parts, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q8_0_mv(const void *planar, const float *x, float *y, int rows, int k, hipStream_t st) {
    const int8_t *qs = (const int8_t *)planar;
    const uint16_t *dp = (const uint16_t *)((const uint8_t *)planar + (size_t)rows * k);
    const int waves = (rows + Q80_ROWS_PER_WAVE - 1) / Q80_ROWS_PER_WAVE;
    hipLaunchKernelGGL(q8_0_mv, dim3((waves + 3) / 4), dim3(256), 0, st, qs, dp, x, y, rows, k);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_q8_0_dequant(const void *planar, int rows, int k, float *out, hipStream_t st) {
    const int8_t *qs = (const int8_t *)planar;
    const uint16_t *dp = (const uint16_t *)((const uint8_t *)planar + (size_t)rows * k);
    const size_t n = (size_t)rows * k;
    hipLaunchKernelGGL(q8_0_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, qs, dp,
                       out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_f32_mv(const float *w, const float *x, float *y, int rows, int k, hipStream_t st) {
    hipLaunchKernelGGL(f32_mv, dim3((rows + 3) / 4), dim3(256), 0, st, w, x, y, rows, k);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
