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

constexpr int ROUTE_MAX_EXPERTS = 256;
constexpr int ROUTE_MAX_USED = 64;

// ---- routing core, shared by the kernels below ---------------------------
// One workgroup (any multiple of 64 threads) routes n_expert <= 256 experts
// held in LDS. `c`/`r` are the centre and radius of every logit; `l` the
// float logits the probabilities are computed from.
struct RouteLds {
    double c[ROUTE_MAX_EXPERTS];
    double r[ROUTE_MAX_EXPERTS];
    float l[ROUTE_MAX_EXPERTS];
    float p[ROUTE_MAX_EXPERTS];
    int sorted[ROUTE_MAX_EXPERTS];
    float mx, total;
    int flag;
};

// Rank experts by key (descending), ties to the lower index: the order of
// Rust's stable sort_by in moe.rs:93-100 for a total order.
template <class T>
__device__ void rank_desc(const T *key, int n, int *sorted) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const T ki = key[i];
        int rank = 0;
        for (int j = 0; j < n; ++j) {
            const T kj = key[j];
            rank += (kj > ki || (kj == ki && j < i)) ? 1 : 0;
        }
        sorted[rank] = i;
    }
    __syncthreads();
}

// Workgroup-wide max of a double (order-free), result on every thread.
__device__ double block_max_d(double v, double *red) {
    for (int m = 32; m >= 1; m >>= 1) v = fmax(v, shfl_xor_d(v, m));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    double r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmax(r, red[i]);
    __syncthreads();
    return r;
}

// Sequential f32 sum v[0] + v[1] + ... from -0.0 (Rust's .sum()), on one
// thread, with the loads batched ahead of the dependent adds.
__device__ float seq_sum(const float *v, int n) {
    float acc = -0.0f;
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        const float4 a = *(const float4 *)(v + i);
        const float4 b = *(const float4 *)(v + i + 4);
        acc = acc + a.x; acc = acc + a.y; acc = acc + a.z; acc = acc + a.w;
        acc = acc + b.x; acc = acc + b.y; acc = acc + b.z; acc = acc + b.w;
    }
    for (; i < n; ++i) acc = acc + v[i];
    return acc;
}

// Is the order of the n_used best logits (and the set) provably the
// reference's? Result in sh.flag (0 = proven, 1 = not), on every thread.
__device__ void decide(RouteLds &sh, int n_expert, int n_used, int force_exact, double *red) {
    // every centre finite; the largest (c + r) outside the chosen set
    double bad = 0.0, mrest = -DBL_MAX;
    for (int q = threadIdx.x; q < n_expert; q += blockDim.x) {
        const int j = sh.sorted[q];
        if (isnan(sh.c[j]) || isinf(sh.c[j])) bad = 1.0;
        if (q >= n_used) mrest = fmax(mrest, sh.c[j] + sh.r[j]);
    }
    bad = block_max_d(bad, red);
    mrest = block_max_d(mrest, red);
    if (threadIdx.x == 0) {
        bool ok = !force_exact && bad == 0.0;
        const double cmax = sh.c[sh.sorted[0]];
        // Separation required on top of the two radii so the reference's
        // probabilities exp(l - max) / total cannot collapse to equal floats
        // (where its tie rule, index order, would decide): 1e-6 relative
        // keeps well clear of f32 rounding.
        const double rel = 1e-6 * (1.0 + fabs(cmax));
        for (int q = 0; ok && q + 1 < n_used; ++q) {
            const int a = sh.sorted[q], b = sh.sorted[q + 1];
            ok = (sh.c[a] - sh.r[a]) - (sh.c[b] + sh.r[b]) > rel * (1.0 + fabs(sh.c[a]));
        }
        if (ok && n_used < n_expert) {
            const int last = sh.sorted[n_used - 1];
            ok = (sh.c[last] - sh.r[last]) - mrest > rel * (1.0 + fabs(sh.c[last]));
        }
        // chosen probabilities must stay far from exp() underflow, where
        // zero-probability ties would fall back to index order
        if (ok) ok = (sh.c[sh.sorted[n_used - 1]] - cmax) > -80.0;
        sh.flag = ok ? 0 : 1;
    }
    __syncthreads();
}

// softmax over sh.l exactly as moe.rs:82-87 (max fold, exp, sequential
// total from -0.0, divide), then, if `resort`, rank by probability; then
// gather, clamp and renormalise (moe.rs:103-105) into ids/weights.
__device__ void finish_route(RouteLds &sh, int n_expert, int n_used, bool resort, int32_t *ids,
                             float *weights, float *logits_used, double *red) {
    const int tid = threadIdx.x;
    // f32::max fold: NaN-ignoring and order-free
    double m = -INFINITY;
    for (int i = tid; i < n_expert; i += blockDim.x)
        if (!isnan(sh.l[i])) m = fmax(m, (double)sh.l[i]);
    const float mx = (float)block_max_d(m, red);
    for (int i = tid; i < n_expert; i += blockDim.x) sh.p[i] = expf_ref(sh.l[i] - mx);
    __syncthreads();
    if (tid == 0) sh.total = seq_sum(sh.p, n_expert);
    __syncthreads();
    for (int i = tid; i < n_expert; i += blockDim.x) sh.p[i] = sh.p[i] / sh.total;
    __syncthreads();
    if (resort) rank_desc(sh.p, n_expert, sh.sorted);
    if (tid == 0) {
        float raw[ROUTE_MAX_USED];
        float wsum = -0.0f;
        for (int q = 0; q < n_used; ++q) {
            raw[q] = sh.p[sh.sorted[q]];
            wsum = wsum + raw[q];
        }
        wsum = fmaxf(wsum, WEIGHT_SUM_FLOOR);
        for (int q = 0; q < n_used; ++q) {
            ids[q] = sh.sorted[q];
            weights[q] = raw[q] / wsum;
        }
    }
    if (logits_used)
        for (int i = tid; i < n_expert; i += blockDim.x) logits_used[i] = sh.l[i];
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
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row < a.n_expert) {
        const int per = a.k / 64;
        const float *wr = a.w + (size_t)row * a.k + (size_t)lane * per;
        const float *xr = a.x + (size_t)lane * per;
        double tot = 0.0, absum = 0.0;
        for (int i = 0; i < per; i += 4) {
            const float4 w4 = *(const float4 *)(wr + i);
            const float4 x4 = *(const float4 *)(xr + i);
            // the reference's rounded products
            const float p0 = w4.x * x4.x, p1 = w4.y * x4.y, p2 = w4.z * x4.z, p3 = w4.w * x4.w;
            tot += (double)p0; tot += (double)p1; tot += (double)p2; tot += (double)p3;
            absum += fabs((double)p0) + fabs((double)p1) + fabs((double)p2) + fabs((double)p3);
        }
        double incl = tot;
        for (int o = 1; o < 64; o <<= 1) {
            const double v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        double pre = __shfl_up(incl, 1, 64);
        if (lane == 0) pre = 0.0;
        double sabs = 0.0, run = pre;
        for (int i = 0; i < per; i += 4) {
            const float4 w4 = *(const float4 *)(wr + i);
            const float4 x4 = *(const float4 *)(xr + i);
            const float pr[4] = {w4.x * x4.x, w4.y * x4.y, w4.z * x4.z, w4.w * x4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                run += (double)pr[j];
                if (lane * per + i + j >= 1) sabs += fabs(run);
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
    if (!last_arrival(&a.counters[0], nr)) return;
    __shared__ RouteLds sh;
    __shared__ double red[4];
    for (int i = threadIdx.x; i < a.n_expert; i += blockDim.x) {
        sh.c[i] = load_dev(&a.centre[i]);
        sh.r[i] = load_dev(&a.radius[i]);
        sh.l[i] = load_dev(&a.logit_f[i]);
    }
    __syncthreads();
    rank_desc(sh.c, a.n_expert, sh.sorted);
    decide(sh, a.n_expert, a.n_used, a.force_exact, red);
    if (threadIdx.x == 0) {
        *a.flag = sh.flag;
        if (a.stats) a.stats[0] += 1;
    }
    if (sh.flag == 0)
        finish_route(sh, a.n_expert, a.n_used, false, a.ids, a.weights, a.logits_used, red);
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
    __shared__ double red[4];
    for (int i = threadIdx.x; i < a.n_expert; i += blockDim.x) sh.l[i] = load_dev(&a.exact_l[i]);
    __syncthreads();
    finish_route(sh, a.n_expert, a.n_used, true, a.ids, a.weights, a.logits_used, red);
    if (threadIdx.x == 0 && a.stats) a.stats[1] += 1;
}

// Routing from given logits (llamd_hip_route / llamd_fwd_router): exact
// inputs, radius 0; ties or near-collapses go through the reference's sort.
__global__ __launch_bounds__(256) void route_logits(const float *logits, int n_expert, int n_used,
                                                    int32_t *ids, float *weights) {
    __shared__ RouteLds sh;
    __shared__ double red[4];
    for (int i = threadIdx.x; i < n_expert; i += blockDim.x) {
        sh.l[i] = logits[i];
        sh.c[i] = (double)logits[i];
        sh.r[i] = 0.0;
    }
    __syncthreads();
    rank_desc(sh.c, n_expert, sh.sorted);
    decide(sh, n_expert, n_used, 0, red);
    finish_route(sh, n_expert, n_used, sh.flag != 0, ids, weights, nullptr, red);
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
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = shfl_xor_f(bv, m);
        const int oi = shfl_xor_i(bi, m);
        better(bv, bi, ov, oi);
    }
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
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = shfl_xor_f(bv, m);
        const int oi = shfl_xor_i(bi, m);
        better(bv, bi, ov, oi);
    }
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
    hipLaunchKernelGGL(router_exact, dim3(l.n_expert), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_route_logits(const float *logits, int n_expert, int n_used, int32_t *ids,
                        float *weights, hipStream_t st) {
    hipLaunchKernelGGL(route_logits, dim3(1), dim3(256), 0, st, logits, n_expert, n_used, ids,
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
