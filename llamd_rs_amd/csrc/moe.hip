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

namespace llamd {
namespace {

constexpr int ROUTE_MAX_EXPERTS = 256;
constexpr int ROUTE_MAX_USED = 64;

// ---- 1. router logits with a rigorous error radius -------------------------
// One wave per expert row. Lane l owns elements [l*per, (l+1)*per).
__global__ __launch_bounds__(256) void router_bound(const float *w, const float *x, int n_expert,
                                                    int k, float *logit_f, double *centre,
                                                    double *radius) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_expert) return;
    const int per = k / 64;
    const float *wr = w + (size_t)row * k + (size_t)lane * per;
    const float *xr = x + (size_t)lane * per;

    double tot = 0.0, absum = 0.0;
    for (int i = 0; i < per; ++i) {
        const float p = wr[i] * xr[i];  // the reference's rounded product
        tot += (double)p;
        absum += fabs((double)p);
    }
    // exclusive scan of lane totals
    double incl = tot;
    for (int o = 1; o < 64; o <<= 1) {
        const double v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    double pre = __shfl_up(incl, 1, 64);
    if (lane == 0) pre = 0.0;
    // sum of |prefix sums| over global indices 1..k-1 (the fold's k >= 2)
    double sabs = 0.0;
    double run = pre;
    for (int i = 0; i < per; ++i) {
        const float p = wr[i] * xr[i];
        run += (double)p;
        if (lane * per + i >= 1) sabs += fabs(run);
    }
    const double S = wave_sum_d(tot);
    const double A = wave_sum_d(absum);
    const double SA = wave_sum_d(sabs);
    if (lane == 0) {
        const double u = 0x1p-24;
        const double n = (double)k;
        const double gam = n * u / (1.0 - n * u);
        // double rounding in the scan and the sums: far below 1e-9 * A
        const double r = u / (1.0 - u) * (SA + n * gam * A) * (1.0 + 1e-6) + 1e-9 * A + 1e-30;
        centre[row] = S;
        radius[row] = r;
        logit_f[row] = (float)S;
    }
}

// ---- 2. routing -------------------------------------------------------------
struct RouteShared {
    double c[ROUTE_MAX_EXPERTS];
    double r[ROUTE_MAX_EXPERTS];
    float l[ROUTE_MAX_EXPERTS];
    float p[ROUTE_MAX_EXPERTS];
    int sorted[ROUTE_MAX_EXPERTS];
    float tile[ROUTE_MAX_EXPERTS][33];
    int flag;
};

// Exact reference fold for every row: s = -0.0; s += w[t] * x[t] in order.
__device__ void exact_logits(const float *w, const float *x, int n_expert, int k, RouteShared &sh) {
    const int tid = threadIdx.x;
    float acc = -0.0f;
    for (int t0 = 0; t0 < k; t0 += 32) {
        const int cols = (k - t0) < 32 ? (k - t0) : 32;
        for (int idx = tid; idx < n_expert * 32; idx += blockDim.x) {
            const int r = idx >> 5, c = idx & 31;
            sh.tile[r][c] = c < cols ? w[(size_t)r * k + t0 + c] : 0.0f;
        }
        __syncthreads();
        if (tid < n_expert) {
            for (int c = 0; c < cols; ++c) {
                const float p = sh.tile[tid][c] * x[t0 + c];
                acc = acc + p;
            }
        }
        __syncthreads();
    }
    if (tid < n_expert) sh.l[tid] = acc;
    __syncthreads();
}

// Single workgroup of 256 threads; n_expert <= 256.
__global__ __launch_bounds__(256) void moe_route(const float *logit_f, const double *centre,
                                                 const double *radius, const float *w,
                                                 const float *x, int n_expert, int k, int n_used,
                                                 int force_exact, int32_t *ids, float *weights,
                                                 float *logits_used, int *stats) {
    __shared__ RouteShared sh;
    const int tid = threadIdx.x;
    if (tid < n_expert) {
        // without a centre the given logits are exact (radius 0)
        sh.c[tid] = centre ? centre[tid] : (double)logit_f[tid];
        sh.r[tid] = centre ? radius[tid] : 0.0;
        sh.l[tid] = logit_f[tid];
    }
    __syncthreads();
    // rank by centre, ties to the lower index
    if (tid < n_expert) {
        const double ci = sh.c[tid];
        int rank = 0;
        for (int j = 0; j < n_expert; ++j) {
            const double cj = sh.c[j];
            rank += (cj > ci || (cj == ci && j < tid)) ? 1 : 0;
        }
        sh.sorted[rank] = tid;
    }
    __syncthreads();
    if (tid == 0) {
        bool ok = !force_exact;
        double cmax = sh.c[sh.sorted[0]];
        for (int q = 0; q < n_expert && ok; ++q) ok = !isnan(sh.c[q]) && !isinf(sh.c[q]);
        // Separation needed on top of the two radii so that the reference's
        // probabilities cannot collapse to equal floats (then its tie rule,
        // index order, would decide): exp(l - max) / total keeps a relative
        // gap of 1e-6 well clear of f32 rounding.
        const double rel = 1e-6 * (1.0 + fabs(cmax));
        for (int q = 0; ok && q + 1 < n_used; ++q) {
            const int a = sh.sorted[q], b = sh.sorted[q + 1];
            ok = (sh.c[a] - sh.r[a]) - (sh.c[b] + sh.r[b]) > rel * (1.0 + fabs(sh.c[a]));
        }
        if (ok && n_used < n_expert) {
            double mrest = -DBL_MAX;
            for (int q = n_used; q < n_expert; ++q) {
                const int j = sh.sorted[q];
                mrest = fmax(mrest, sh.c[j] + sh.r[j]);
            }
            const int last = sh.sorted[n_used - 1];
            ok = (sh.c[last] - sh.r[last]) - mrest > rel * (1.0 + fabs(sh.c[last]));
        }
        // every chosen probability must stay far from underflow, where
        // exp() == 0 ties would fall back to index order
        if (ok) ok = (sh.c[sh.sorted[n_used - 1]] - cmax) > -80.0;
        sh.flag = ok ? 0 : 1;
    }
    __syncthreads();
    const bool exact = sh.flag != 0;
    // with no weights the given logits are already the reference's bits
    if (exact && w) exact_logits(w, x, n_expert, k, sh);

    // softmax exactly as moe.rs:82-87
    if (tid == 0) {
        float mx = -INFINITY;
        for (int i = 0; i < n_expert; ++i) mx = fmaxf(mx, sh.l[i]);
        sh.tile[0][0] = mx;
    }
    __syncthreads();
    const float mx = sh.tile[0][0];
    if (tid < n_expert) sh.p[tid] = expf_ref(sh.l[tid] - mx);
    __syncthreads();
    if (tid == 0) {
        float total = -0.0f;
        for (int i = 0; i < n_expert; ++i) total = total + sh.p[i];
        sh.tile[0][1] = total;
    }
    __syncthreads();
    if (tid < n_expert) sh.p[tid] = sh.p[tid] / sh.tile[0][1];
    __syncthreads();
    if (exact) {
        // stable sort by probability desc, ties to the lower index (moe.rs:93-100)
        if (tid < n_expert) {
            const float pi = sh.p[tid];
            int rank = 0;
            for (int j = 0; j < n_expert; ++j) {
                const float pj = sh.p[j];
                rank += (pj > pi || (pj == pi && j < tid)) ? 1 : 0;
            }
            sh.sorted[rank] = tid;
        }
        __syncthreads();
    }
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
        if (stats) {
            stats[0] += 1;
            stats[1] += exact ? 1 : 0;
        }
    }
    if (logits_used && tid < n_expert) logits_used[tid] = sh.l[tid];
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

int launch_router_bound(const float *w, const float *x, int n_expert, int k, float *logit_f,
                        double *centre, double *radius, hipStream_t st) {
    hipLaunchKernelGGL(router_bound, dim3((n_expert + 3) / 4), dim3(256), 0, st, w, x, n_expert, k,
                       logit_f, centre, radius);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_moe_route(const float *logit_f, const double *centre, const double *radius,
                     const float *w, const float *x, int n_expert, int k, int n_used,
                     int force_exact, int32_t *ids, float *weights, float *logits_used,
                     int *stats, hipStream_t st) {
    hipLaunchKernelGGL(moe_route, dim3(1), dim3(256), 0, st, logit_f, centre, radius, w, x,
                       n_expert, k, n_used, force_exact, ids, weights, logits_used, stats);
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
