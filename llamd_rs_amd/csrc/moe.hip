// moe.hip -- router logits, top-k routing, expert combine, argmax, and the
// f32 / Q8_0 matvecs of the reference's fallback path (model.rs:253-262).
//
// EXPERT SELECTION AND ROUTING WEIGHTS ARE BIT-EXACT. The reference routes on
// logits from a SEQUENTIAL f32 sum (the F32 router goes through
// matvec_quant's fallback, crates/llamd-models/src/model.rs:253-262)
// followed by softmax, a stable sort with ties to the lower index, and
// renormalisation (moe.rs:73-113). router_logits reproduces the fold bit for
// bit: one wave per expert forms the rounded products in parallel and one
// lane adds them in order. The softmax / top-k / renormalisation (route.hpp,
// glibc-identical expf) runs in the prologue of the gate/up kernel, so the
// routed expert ids and weights are the CPU path's on every call.
#include <float.h>

#include "common.hpp"
#include "expf_ref.h"
#include "launch.hpp"
#include "q8k_wave.hpp"
#include "route.hpp"

namespace llamd {
namespace {

struct RouterArgs {
    const float *w;          // f32 router [n_expert][k]
    const float *x;          // [nseq][k] (blockIdx.y = sequence)
    int n_expert, k;
    float *logits;           // [nseq][n_expert] the reference's logits, bit for bit
    // fused Q8_K quantisation of x for the expert matvecs
    int8_t *xq;
    float *xd;
    int xblocks;
};

// The reference's router logits, bit for bit, on every call: wave w of
// workgroup b owns row b*RPW + w. All 64 lanes form the rounded products
// w[t]*x[t] (coalesced 16-byte loads, the whole row in flight at once) into
// LDS; lane 0 then runs the sequential fold s = -0.0; s += p[t]
// (model.rs:253-262) from 16-byte LDS reads. Workgroups past the rows
// quantize x to Q8_K for the expert matvecs. The routing itself happens in
// the gate/up kernel's prologue.
template <int RPW>
__global__ __launch_bounds__(64 * RPW) void router_logits(RouterArgs a) {
    // all kernarg fields in one batch before the first global load
    asm volatile("" ::"s"(a.w), "s"(a.x), "s"(a.n_expert), "s"(a.k), "s"(a.logits), "s"(a.xq),
                 "s"(a.xd), "s"(a.xblocks));
    constexpr int KMAX = 2048;
    __shared__ float4 prod[RPW][KMAX / 4];
    const int nr = (a.n_expert + RPW - 1) / RPW;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    if ((int)blockIdx.x >= nr) {
        // (xblocks > 0 only with one sequence)
        const int blk = ((int)blockIdx.x - nr) * RPW + wv;
        if (blk < a.xblocks) {
            const float4 xv = *(const float4 *)(a.x + (size_t)blk * QK_K + 4 * lane);
            const float v[4] = {xv.x, xv.y, xv.z, xv.w};
            quantize_block_wave(v, lane, a.xq + (size_t)blk * QK_K, a.xd + blk);
        }
        return;
    }
    const int row = blockIdx.x * RPW + wv;
    if (row >= a.n_expert) return;
    const float4 *w4 = (const float4 *)(a.w + (size_t)row * a.k);
    const float4 *x4 = (const float4 *)(a.x + (size_t)blockIdx.y * a.k);
    const int n4 = a.k / 4;  // a multiple of 64 (k is a multiple of 256)
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
            prod[wv][64 * j + lane] = make_float4(wr[j].x * xr[j].x, wr[j].y * xr[j].y,
                                                  wr[j].z * xr[j].z, wr[j].w * xr[j].w);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane == 0) a.logits[(size_t)blockIdx.y * a.n_expert + row] = seq_fold(prod[wv], n4);
}
// Routing from given logits (llamd_hip_route / llamd_fwd_router).
// One workgroup per sequence (blockIdx.x): logits [nseq][n_expert] -> ids,
// weights [nseq][n_used], and (probs not null) the softmax [nseq][n_expert].
__global__ __launch_bounds__(64) void route_logits(const float *logits, int n_expert, int n_used,
                                                   int32_t *ids, float *weights, float *probs) {
    __shared__ RouteLds sh;
    const int lane = threadIdx.x;
    logits += (size_t)blockIdx.x * n_expert;
    ids += (size_t)blockIdx.x * n_used;
    weights += (size_t)blockIdx.x * n_used;
    if (probs) probs += (size_t)blockIdx.x * n_expert;
    float l[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int i = lane + WAVE * j;
        l[j] = i < n_expert ? logits[i] : 0.0f;
    }
    route_finish(l, n_expert, n_used, true, sh, ids, weights, nullptr, nullptr, false, probs);
}

// ---- 3. weighted combine + residual (layer.rs:245-258, 281-287) -------------
// out[i] = res[i] + (((0 + w0*d0[i]) + w1*d1[i]) + ...), experts in routing order.
// blockIdx.y = token (prefill); down is [n_tok][n_used][n_embd].
// skip (optional): pair slots of the grouped prefill; a pair with slot < 0
// had an out-of-range expert id and adds no term.
// (256 threads per workgroup: a constant, so no implicit kernel arguments)
template <int V>
__global__ __launch_bounds__(256) void moe_combine(const float *down, const float *weights, const float *res, float *out,
                            int n_used, int n_embd, const int32_t *skip) {
    typedef float fv __attribute__((ext_vector_type(V)));
    const int i = V * (blockIdx.x * 256 + threadIdx.x);  // this thread's first element
    if (i >= n_embd) return;
    const size_t tok = blockIdx.y;
    down += tok * n_used * n_embd;
    weights += tok * n_used;
    if (skip) skip += tok * n_used;
    if (res) res += tok * n_embd;
    out += tok * n_embd;
    // every operand is loaded before the first add (a pair with no expert
    // still has a row in `down`, unused), so the loads are one round trip
    // instead of one per expert; the adds keep the routing order. V = 4:
    // four consecutive elements per thread, 16-byte loads.
    constexpr int E = 16;  // n_used <= 16
    float wv[E];
    fv dv[E];
    bool live[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        live[e] = e < n_used && !(skip && skip[e] < 0);
        wv[e] = e < n_used ? weights[e] : 0.0f;
        dv[e] = e < n_used ? *(const fv *)(down + (size_t)e * n_embd + i) : fv{};
    }
    const fv r = res ? *(const fv *)(res + i) : fv{};
    fv acc = fv{};
#pragma unroll
    for (int e = 0; e < E; ++e) {
#pragma unroll
        for (int c = 0; c < V; ++c) {
            const float p = wv[e] * dv[e][c];
            acc[c] = live[e] ? acc[c] + p : acc[c];
        }
    }
    if (res) {
#pragma unroll
        for (int c = 0; c < V; ++c) acc[c] = r[c] + acc[c];
    }
    *(fv *)(out + i) = acc;
}

// ---- 4. argmax: strict '>', lowest index wins (device_forward.rs:23-37) -----
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// (nparts = the grid's width, passed so the kernel needs no implicit arguments)
__global__ __launch_bounds__(256) void argmax_partial(const float *x, int n, int ld, float *pv,
                                                      int *pi, int nparts) {
    const int seq = blockIdx.y;
    const float *xs = x + (size_t)seq * ld;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += nparts * 256) {
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
        pv[(size_t)seq * nparts + blockIdx.x] = bv;
        pi[(size_t)seq * nparts + blockIdx.x] = bi;
    }
}

template <int NT>
__global__ __launch_bounds__(NT) void argmax_final(const float *x, int ld, const float *pv,
                                                   const int *pi, int nparts, int32_t *out) {
    asm volatile("" ::"s"(x), "s"(ld), "s"(pv), "s"(pi), "s"(nparts), "s"(out));
    const int seq = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    // eight independent candidate loads in flight per thread before reducing
    constexpr int U = 8;
    const float *sv_in = pv + (size_t)seq * nparts;
    const int *si_in = pi + (size_t)seq * nparts;
    // the reference's incumbent (index 0), loaded before the reduction so its
    // round trip overlaps the candidates'
    const float v0 = threadIdx.x == 0 ? x[(size_t)seq * ld] : 0.0f;
    for (int base = threadIdx.x; base < nparts; base += U * NT) {
        float v[U];
        int id[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * NT;
            v[u] = i < nparts ? sv_in[i] : -INFINITY;
            id[u] = i < nparts ? si_in[i] : 0x7FFFFFFF;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) argmax_step(bv, bi, v[u], id[u]);
    }
    wave_argmax(bv, bi, -INFINITY);
    __shared__ float sv[16];
    __shared__ int si[16];
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < NT / 64; ++w) better(bv, bi, sv[w], si[w]);
        // the reference's incumbent is index 0: a NaN there is never beaten,
        // and when nothing beats -inf the answer stays 0
        out[seq] = (isnan(v0) || bi == 0x7FFFFFFF) ? 0 : bi;
    }
}

// ---- 5. Q8_0 matvec (R8: dequantize then f32 dot) ----------------------------
// Planar layout: qs [rows][k] int8, then d [rows][k/32] f16. One wave handles
// ROWS_PER_WAVE rows; lane l owns Q8_0 blocks l, l+64, ... and loads each
// block's 32 activations once for all its rows. Products are d*q rounded
// (the dequantized weight, exact) times x, accumulated with FMA; within
// REDUCTION of the reference's sequential sum. Two rows per wave measured
// best at 4096 x 2048 on MI355X (per launch, graph replay: 1 row 6.3 us,
// 2 rows 4.7, 4 rows 4.8, 8 rows 6.4; loading all rows' words before the
// arithmetic was slower, 5.3).
constexpr int Q80_ROWS_PER_WAVE = 2;

__global__ __launch_bounds__(256) void q8_0_mv(const int8_t *qs, const uint16_t *dp, const float *x,
                                               float *y, int rows, int k) {
    asm volatile("" ::"s"(qs), "s"(dp), "s"(x), "s"(y), "s"(rows), "s"(k));
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
    a.w = l.w; a.x = l.x; a.n_expert = l.n_expert; a.k = l.k; a.logits = l.logits;
    a.xq = l.xq; a.xd = l.xd; a.xblocks = l.xblocks;
    if (l.k % QK_K || l.k > 2048 || l.nseq <= 0 || (l.nseq > 1 && l.xblocks)) return -1;
    // one row per workgroup spreads the sequential folds over the most CUs
    hipLaunchKernelGGL(router_logits<1>, dim3(l.n_expert + l.xblocks, l.nseq), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_route_logits(const float *logits, int n_expert, int n_used, int32_t *ids,
                        float *weights, hipStream_t st, int nseq, float *probs) {
    if (nseq <= 0) return -1;
    hipLaunchKernelGGL(route_logits, dim3(nseq), dim3(64), 0, st, logits, n_expert, n_used, ids,
                       weights, probs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_moe_combine(const float *down, const float *weights, const float *res, float *out,
                       int n_used, int n_embd, int n_tok, hipStream_t st, const int32_t *skip) {
    if (n_used < 1 || n_used > 16) return -1;
    // 16-byte vectors when every row starts 16-byte aligned
    const bool vec = n_embd % 4 == 0 && ((uintptr_t)down | (uintptr_t)out | (uintptr_t)res) % 16 == 0;
    if (vec)
        hipLaunchKernelGGL(moe_combine<4>, dim3((n_embd / 4 + 255) / 256, n_tok), dim3(256), 0, st,
                           down, weights, res, out, n_used, n_embd, skip);
    else
        hipLaunchKernelGGL(moe_combine<1>, dim3((n_embd + 255) / 256, n_tok), dim3(256), 0, st, down,
                           weights, res, out, n_used, n_embd, skip);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int argmax_parts(int n) {
    int parts = (n + 4095) / 4096;
    if (parts < 1) parts = 1;
    if (parts > 1024) parts = 1024;
    return parts;
}

int launch_argmax(const float *x, int n, int ld, int nseq, float *pv, int *pi, int32_t *out,
                  hipStream_t st, int max_parts) {
    int parts = argmax_parts(n);
    if (max_parts > 0 && parts > max_parts) parts = max_parts;
    hipLaunchKernelGGL(argmax_partial, dim3(parts, nseq), dim3(256), 0, st, x, n, ld, pv, pi, parts);
    hipLaunchKernelGGL(argmax_final<64>, dim3(nseq), dim3(64), 0, st, x, ld, pv, pi, parts, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_argmax_final(const float *x, int ld, int nseq, const float *pv, const int *pi,
                        int nparts, int32_t *out, hipStream_t st) {
    hipLaunchKernelGGL(argmax_final<1024>, dim3(nseq), dim3(1024), 0, st, x, ld, pv, pi, nparts, out);
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

int launch_matvec_f32_exact(const float *w, const float *x, float *y, int rows, int k, int nseq,
                            hipStream_t st) {
    if (rows <= 0 || k <= 0 || nseq <= 0) return -1;
    if (k % QK_K == 0 && k <= 2048) {
        RouterLaunch l;
        l.w = w;
        l.x = x;
        l.n_expert = rows;
        l.k = k;
        l.logits = y;
        l.xq = nullptr;
        l.xd = nullptr;
        l.xblocks = 0;
        l.nseq = nseq;
        return launch_router(l, st);
    }
    for (int s = 0; s < nseq; ++s)
        if (launch_f32_mv(w, x + (size_t)s * k, y + (size_t)s * rows, rows, k, st)) return -1;
    return 0;
}

int launch_f32_mv(const float *w, const float *x, float *y, int rows, int k, hipStream_t st) {
    hipLaunchKernelGGL(f32_mv, dim3((rows + 3) / 4), dim3(256), 0, st, w, x, y, rows, k);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
