// norm.hip -- RMSNorm (+ weight, + Q8_K) in front of the attention
// projections, bit-identical to the reference CPU path.
//
// CpuBackend::rms_norm (crates/llamd-cpu/src/lib.rs:55-75) sums the squares
// of a row in f32, IN ORDER, from 0.0, then scale = 1 / sqrt(sum / n + eps)
// and out = x * scale; the layer then multiplies by the norm weight as a
// separate tensor op (be.mul, layer.rs:101-104 and per_head_rms_norm,
// layer.rs:62-79). The in-order sum is a dependency chain. For whole rows the
// workgroup reproduces it with exact_sum_nonneg (exact_sum.hpp: every step
// whose rounding a bound certifies is applied as a known increment, one lane
// replays the rest); for the 128-wide per-head norm, all lanes form the
// rounded squares into LDS and one lane adds them in order. sqrt and the
// divide are correctly rounded (sqrt_rn, __fdiv_rn), as Rust's f32 sqrt and
// `/` are.
//
// The fused variant then forms (x * scale) * w for each 256-element block and
// quantizes it to Q8_K with one wave per block, writing the reference's
// BlockQ8K arrays for the Q / K / V matvecs.
#include "common.hpp"
#include "exact_sum.hpp"
#include "row_scale.hpp"
#include "launch.hpp"
#include "q8k_wave.hpp"
#include "q6k_tile.hpp"

namespace llamd {
namespace {

constexpr int NORM_MAX = 8192;  // longest row (the exact sum's bound holds to 8192 terms)

// This thread's run of a row (xsum_run(n) contiguous elements starting at
// threadIdx.x * run) into registers; lanes past the row's end read its last
// element (unconditional loads) and are ignored by the callers.
__device__ __forceinline__ void load_run(const float *src, int n, int nt, float (&v)[XSUM_M]) {
    const int m = xsum_run(n, nt), j0 = min((int)threadIdx.x * m, n - 1);
    if ((m & 3) == 0 && m <= XSUM_M && j0 + m <= n && ((uintptr_t)(src + j0) & 15) == 0) {
#pragma unroll
        for (int k = 0; k < XSUM_M; k += 4) {
            const float4 q = k < m ? *(const float4 *)(src + j0 + k) : make_float4(0, 0, 0, 0);
            v[k] = q.x;
            v[k + 1] = q.y;
            v[k + 2] = q.z;
            v[k + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < XSUM_M; ++k) v[k] = src[min(j0 + k, n - 1)];
    }
}

// 1 / sqrt(sum of v^2 / n + eps) for a row whose runs the threads hold in
// vals (load_run), the sum in the reference's order, by the whole workgroup
// (every thread calls it; every thread gets the scale). src is the row in
// global memory, read only by the serial fallback.
__device__ float row_scale_block(const float *src, const float (&vals)[XSUM_M], int n, int nt,
                                 float eps, ExactSumLds &L) {
    float sq[XSUM_M];
#pragma unroll
    for (int k = 0; k < XSUM_M; ++k) sq[k] = vals[k] * vals[k];
    const float sum = exact_sum_nonneg(sq, n, nt, L, [src](int i) {
        const float v = src[i];
        return v * v;
    });
    const float mean = __fdiv_rn(sum, (float)n);
    return __fdiv_rn(1.0f, sqrt_rn(mean + eps));
}

// Threads for a one-row workgroup: enough that each run fits in registers.
inline int row_threads(int n) {
    const int need = ((n + XSUM_M - 1) / XSUM_M + WAVE - 1) / WAVE * WAVE;
    return need < 512 ? 512 : (need > 1024 ? 1024 : need);
}

// out[r][i] = (x[r][i] * scale_r) * w[i % w_len], one workgroup per row
// (rows = heads for the per-head QK norm). w may be null (no multiply).
// NT: the thread count when the launch fixes it (no implicit kernel
// arguments then), 0 for any other (blockDim).
template <int NT>
__global__ __launch_bounds__(NT ? NT : 1024) void rms_norm_mul(const float *x, const float *w, float *out,
                                                     int n, int w_len, float eps) {
    const int nt = NT ? NT : (int)blockDim.x;
    __shared__ ExactSumLds xs;
    const int r = blockIdx.x;
    const float *src = x + (size_t)r * n;
    float v[XSUM_M];
    load_run(src, n, nt, v);
    const int m = xsum_run(n, nt), j0 = (int)threadIdx.x * m;
    // the weights of this thread's run, loaded with the row (not after the sum)
    float wv[XSUM_M];
#pragma unroll
    for (int k = 0; k < XSUM_M; ++k) {
        const int i = min(j0 + k, n - 1);
        wv[k] = w && m <= XSUM_M ? w[w_len == n ? i : i % w_len] : 1.0f;
    }
    const float scale = row_scale_block(src, v, n, nt, eps, xs);
    float *dst = out + (size_t)r * n;
    if (m <= XSUM_M) {
#pragma unroll
        for (int k = 0; k < XSUM_M; ++k) {
            const int i = j0 + k;
            if (k < m && i < n) {
                const float y = v[k] * scale;
                dst[i] = w ? y * wv[k] : y;
            }
        }
    } else {
        for (int i = threadIdx.x; i < n; i += nt) {
            const float y = src[i] * scale;
            dst[i] = w ? y * w[w_len == n ? i : i % w_len] : y;
        }
    }
}

// One row of n = 256 * blocks per workgroup (row blockIdx.x of x, out, qs,
// d, inv_out): the workgroup finds the scale, then wave k forms block k (and
// k + waves, ...) of (x * scale) * w and quantizes it.
template <int NT>
__global__ __launch_bounds__(NT ? NT : 1024) void rms_norm_quant(const float *x, const float *w, float *out,
                                                       int8_t *qs, float *d, float *inv_out,
                                                       int n, float eps) {
    const int nt = NT ? NT : (int)blockDim.x;
    __shared__ ExactSumLds xs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t r = blockIdx.x;
    x += r * n;
    if (out) out += r * n;
    qs += r * n;
    d += r * (n / QK_K);
    if (inv_out) inv_out += r;
    float v0[XSUM_M];
    load_run(x, n, nt, v0);
    const int blocks = n / QK_K, waves = nt >> 6;
    // runs of 4: thread t holds x[4t .. 4t+3], so wave b holds block b and
    // quantizes it from registers; its weights are loaded with the row
    const bool run4 = xsum_run(n, nt) == 4;
    float4 w4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (run4 && wave < blocks) w4 = *(const float4 *)(w + wave * QK_K + 4 * lane);
    const float scale = row_scale_block(x, v0, n, nt, eps, xs);
    if (inv_out && threadIdx.x == 0) *inv_out = scale;
    if (run4) {
        if (wave < blocks) {
            const size_t o = (size_t)wave * QK_K + 4 * lane;
            const float v[4] = {(v0[0] * scale) * w4.x, (v0[1] * scale) * w4.y, (v0[2] * scale) * w4.z,
                                (v0[3] * scale) * w4.w};
            if (out) *(float4 *)(out + o) = make_float4(v[0], v[1], v[2], v[3]);
            quantize_wave(v, lane, qs + o - 4 * lane, d + wave, nullptr);
        }
        return;
    }
    for (int b = wave; b < blocks; b += waves) {
        const size_t o = (size_t)b * QK_K + 4 * lane;
        const float4 xv = *(const float4 *)(x + o);
        const float4 wv = *(const float4 *)(w + o);
        const float v[4] = {(xv.x * scale) * wv.x, (xv.y * scale) * wv.y, (xv.z * scale) * wv.z,
                            (xv.w * scale) * wv.w};
        if (out) *(float4 *)(out + o) = make_float4(v[0], v[1], v[2], v[3]);
        quantize_wave(v, lane, qs + (size_t)b * QK_K, d + b, nullptr);
    }
}

// Per-head QK-norm, RoPE and the KV-cache store of one decode step, one
// workgroup (one wave) per head: Q heads [0, n_head) in place, K heads after
// them into the cache row of this position, with V copied beside them.
//   norm: out = (x * scale) * w            (layer.rs:62-79; skipped if w is null)
//   RoPE: x[i] = a*cos - b*sin, x[i + hd/2] = a*sin + b*cos   (lib.rs:196-205)
// cs[pos][i] = (cos, sin), computed on the host with the reference's libm calls.
__global__ __launch_bounds__(64) void qk_norm_rope_store(float *q, const float *k, const float *v,
                                                         const float *qw, const float *kw,
                                                         const float2 *cs, const int32_t *pos_p,
                                                         int n_head, int n_head_kv, int hd,
                                                         float eps, float *kc, float *vc) {
    __shared__ __align__(16) float sq[256];
    __shared__ float buf[256];
    const int lane = threadIdx.x, h = blockIdx.x, half = hd / 2, pos = pos_p[0];
    const bool isq = h < n_head;
    const int hh = isq ? h : h - n_head;
    const float *src = isq ? q + (size_t)hh * hd : k + (size_t)hh * hd;
    const float *w = isq ? qw : kw;
    const int kv_dim = n_head_kv * hd;
    if (w) {
        const float scale = row_scale_wave(src, hd, eps, sq);
        for (int d = lane; d < hd; d += WAVE) buf[d] = (src[d] * scale) * w[d];
    } else {
        for (int d = lane; d < hd; d += WAVE) buf[d] = src[d];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const float2 *row = cs + (size_t)pos * half;
    float *dst = isq ? q + (size_t)hh * hd : kc + (size_t)pos * kv_dim + (size_t)hh * hd;
    for (int i = lane; i < half; i += WAVE) {
        const float a = buf[i], b = buf[i + half];
        const float2 c = row[i];
        dst[i] = a * c.x - b * c.y;
        dst[i + half] = a * c.y + b * c.x;
    }
    if (!isq)
        for (int d = lane; d < hd; d += WAVE)
            vc[(size_t)pos * kv_dim + (size_t)hh * hd + d] = v[(size_t)hh * hd + d];
}

// ffn_inp = x + o (the attention residual, layer.rs:170), then
// out = rms_norm(ffn_inp) * w: one row, one workgroup.
template <int NT>
__global__ __launch_bounds__(NT ? NT : 1024) void add_rms_norm_mul(const float *x, const float *o,
                                                         const float *w, float *sum_out,
                                                         float *out, int n, float eps) {
    const int nt = NT ? NT : (int)blockDim.x;
    __shared__ ExactSumLds xs;
    const int m = xsum_run(n, nt), j0 = (int)threadIdx.x * m;
    float v[XSUM_M], ov[XSUM_M], wv[XSUM_M];
    load_run(x, n, nt, v);
    load_run(o, n, nt, ov);
    // the weights of this thread's run, loaded with the rows (not after the sum)
#pragma unroll
    for (int k = 0; k < XSUM_M; ++k) wv[k] = m <= XSUM_M ? w[min(j0 + k, n - 1)] : 0.0f;
#pragma unroll
    for (int k = 0; k < XSUM_M; ++k) {
        v[k] = v[k] + ov[k];
        if (k < m && j0 + k < n) sum_out[j0 + k] = v[k];
    }
    if (m > XSUM_M)
        for (int i = threadIdx.x; i < n; i += nt) sum_out[i] = x[i] + o[i];
    // the serial fallback reads sum_out back; exact_sum_nonneg's barriers
    // order these stores before it
    const float scale = row_scale_block(sum_out, v, n, nt, eps, xs);
    if (m <= XSUM_M) {
#pragma unroll
        for (int k = 0; k < XSUM_M; ++k)
            if (k < m && j0 + k < n) out[j0 + k] = (v[k] * scale) * wv[k];
    } else {
        for (int i = threadIdx.x; i < n; i += nt) out[i] = (sum_out[i] * scale) * w[i];
    }
}


// The attention front end of a decode step in one launch: RMSNorm -> Q8_K
// (rms_norm_quant's bits) -> the Q, K and V matvecs (q6k_mv_b1's bits, the
// reference's dot_q6k_q8k per row: per-block class terms added in block
// order, then the eight class sums in order). The 16-row tiles of Q, K and V
// are numbered one after another; a workgroup takes two consecutive tiles
// (the norm is formed once per two tiles, and a decode step's 320 tiles fit
// 160 CUs, one workgroup each).
// Every workgroup forms the norm and the Q8_K itself, into LDS; its tiles'
// weights are requested right after the row, so they stream in under the
// in-order sum.
constexpr int NQ_MAX_BLOCKS = 8;  // n <= 2048: one activation block per wave
constexpr int NQ_TPW = 2;         // tiles per workgroup
constexpr int NQ_UNITS = NQ_TPW * NQ_MAX_BLOCKS;  // (tile, block) units, two per wave

struct NormQkvArgs {
    const float *x, *w;
    const uint8_t *wq, *wk, *wv;  // tiled Q6_K
    float *yq, *yk, *yv;
    int tq, tk, tv;               // 16-row tiles per matrix
    int rq, rk, rv;               // rows per matrix
    int n;
    float eps;
};

// Tile T of the Q | K | V numbering: its matrix's weights, output, rows and
// its index inside that matrix.
struct NqTile {
    const uint8_t *w;
    float *y;
    int rows, t;
};
__device__ __forceinline__ NqTile nq_tile(const NormQkvArgs &a, int T) {
    if (T < a.tq) return {a.wq, a.yq, a.rq, T};
    T -= a.tq;
    if (T < a.tk) return {a.wk, a.yk, a.rk, T};
    return {a.wv, a.yv, a.rv, T - a.tk};
}

__global__ __launch_bounds__(512) void norm_qkv(NormQkvArgs a) {
    constexpr int TPW = NQ_TPW;
    __shared__ ExactSumLds xl;
    __shared__ __align__(16) float xs[NQ_MAX_BLOCKS * QK_K];
    __shared__ __align__(16) int8_t lq[NQ_MAX_BLOCKS * QK_K];
    __shared__ float ld[NQ_MAX_BLOCKS];
    __shared__ float terms[NQ_UNITS][TILE_ROWS][8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, s = lane >> 4;
    const int blocks = a.n / QK_K, total = a.tq + a.tk + a.tv, T0 = blockIdx.x * TPW;
    // the row first: its loads return before the weights queued behind them
    // (every load below is unconditional, at a clamped address when its unit
    // is unused, so the first use of the row waits for the row alone)
    const int m = xsum_run(a.n, 512), j0 = (int)threadIdx.x * m;
    const bool run4 = m == 4;  // thread t holds x[4t .. 4t+3]: wave w holds block w
    float v[XSUM_M];
    if (run4) {
        const float4 q = *(const float4 *)(a.x + j0);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
#pragma unroll
        for (int k = 4; k < XSUM_M; ++k) v[k] = 0.0f;
    } else {
        load_run(a.x, a.n, 512, v);
    }
    // unit u = j * blocks + b: block b of the workgroup's tile j; wave w
    // takes units w and w + 8
    const int u0 = wave, u1 = wave + 8, units = TPW * blocks;
    const bool live0 = u0 < units && T0 + u0 / blocks < total;
    const bool live1 = u1 < units && T0 + u1 / blocks < total;
    BlockRegs r0, r1;
    {
        const NqTile t0 = nq_tile(a, live0 ? T0 + u0 / blocks : 0);
        const NqTile t1 = nq_tile(a, live1 ? T0 + u1 / blocks : 0);
        load_weights(r0, t0.w + ((size_t)t0.t * blocks + (live0 ? u0 % blocks : 0)) * SEG_BYTES, lane, n);
        load_weights(r1, t1.w + ((size_t)t1.t * blocks + (live1 ? u1 % blocks : 0)) * SEG_BYTES, lane, n);
    }
    // the norm weight of this wave's activation block
    const float4 nw0 = *(const float4 *)(a.w + min(wave, blocks - 1) * QK_K + 4 * lane);
    if (!run4) {
        // the row into LDS for the blocks' quantization below
#pragma unroll
        for (int k = 0; k < XSUM_M; ++k)
            if (k < m && j0 + k < a.n) xs[j0 + k] = v[k];
    }
    const float scale = row_scale_block(a.x, v, a.n, 512, a.eps, xl);  // synchronises the workgroup
    // (x * scale) * w, quantized: wave b quantizes block b
    const auto quant = [&](const float4 &xv, int b, const float4 &wv) {
        const float q[4] = {(xv.x * scale) * wv.x, (xv.y * scale) * wv.y, (xv.z * scale) * wv.z,
                            (xv.w * scale) * wv.w};
        quantize_wave(q, lane, lq + b * QK_K, ld + b, nullptr);
    };
    if (run4)
        quant(make_float4(v[0], v[1], v[2], v[3]), wave, nw0);
    else if (wave < blocks)
        quant(*(const float4 *)(xs + wave * QK_K + 4 * lane), wave, nw0);
    __syncthreads();
    // the per-block class terms of this wave's units
    const MaskSel msel = mask_selectors(n, (n >> 2) == s);
    const auto terms_of = [&](BlockRegs &r, int u) {
        const int b = u % blocks;
        r.g = *(const uint4 *)(lq + b * QK_K + 16 * n);
        r.ad = ld[b];
        float te, to;
        block_terms(r, msel, te, to);
        terms[u][n][2 * s] = te;
        terms[u][n][2 * s + 1] = to;
    };
    if (live0) terms_of(r0, u0);
    if (live1) terms_of(r1, u1);
    __syncthreads();
    // wave j folds tile j: block order, then the class sums in order
    if (wave < TPW && T0 + wave < total) {
        float se = 0.0f, so = 0.0f;
        for (int b = 0; b < blocks; ++b) {
            se = se + terms[wave * blocks + b][n][2 * s];
            so = so + terms[wave * blocks + b][n][2 * s + 1];
        }
        float cls[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cls[2 * q] = __shfl(se, n + 16 * q, WAVE);
            cls[2 * q + 1] = __shfl(so, n + 16 * q, WAVE);
        }
        const NqTile tl = nq_tile(a, T0 + wave);
        const int row = tl.t * TILE_ROWS + n;
        if (s == 0 && row < tl.rows) {
            float tot = -0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) tot = tot + cls[c];
            tl.y[row] = tot;
        }
    }
}

}  // namespace

int launch_qk_norm_rope_store(float *q, const float *k, const float *v, const float *qw,
                              const float *kw, const float2 *cs, const int32_t *pos, int n_head,
                              int n_head_kv, int hd, float eps, float *kc, float *vc,
                              hipStream_t st) {
    if (hd <= 0 || hd % 2 || hd > 256 || n_head <= 0 || n_head_kv <= 0) return -1;
    hipLaunchKernelGGL(qk_norm_rope_store, dim3(n_head + n_head_kv), dim3(64), 0, st, q, k, v, qw,
                       kw, cs, pos, n_head, n_head_kv, hd, eps, kc, vc);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_add_rms_norm_mul(const float *x, const float *o, const float *w, float *sum_out,
                            float *out, int n, float eps, hipStream_t st) {
    if (n <= 0 || n > NORM_MAX || !w) return -1;
    const int nt = row_threads(n);
    if (nt == 512)
        hipLaunchKernelGGL(add_rms_norm_mul<512>, dim3(1), dim3(nt), 0, st, x, o, w, sum_out, out, n, eps);
    else
        hipLaunchKernelGGL(add_rms_norm_mul<0>, dim3(1), dim3(nt), 0, st, x, o, w, sum_out, out, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_rms_norm_mul(const float *x, const float *w, float *out, int rows, int n, int w_len,
                        float eps, hipStream_t st) {
    if (rows <= 0 || n <= 0 || n > NORM_MAX || (w && w_len <= 0)) return -1;
    const int nt = row_threads(n);
    if (nt == 512)
        hipLaunchKernelGGL(rms_norm_mul<512>, dim3(rows), dim3(nt), 0, st, x, w, out, n, w_len, eps);
    else
        hipLaunchKernelGGL(rms_norm_mul<0>, dim3(rows), dim3(nt), 0, st, x, w, out, n, w_len, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

bool norm_qkv_fits(int n, const int rows[3]) {
    return n > 0 && n % QK_K == 0 && n / QK_K <= NQ_MAX_BLOCKS && rows[0] > 0 &&
           rows[1] > 0 && rows[2] > 0;
}

int launch_norm_qkv(const float *x, const float *w, float eps, const void *const wt[3],
                    float *const y[3], const int rows[3], int n, hipStream_t st) {
    if (!x || !w || !norm_qkv_fits(n, rows)) return -1;
    NormQkvArgs a;
    a.x = x;
    a.w = w;
    a.wq = (const uint8_t *)wt[0];
    a.wk = (const uint8_t *)wt[1];
    a.wv = (const uint8_t *)wt[2];
    a.yq = y[0];
    a.yk = y[1];
    a.yv = y[2];
    a.rq = rows[0];
    a.rk = rows[1];
    a.rv = rows[2];
    a.tq = (rows[0] + TILE_ROWS - 1) / TILE_ROWS;
    a.tk = (rows[1] + TILE_ROWS - 1) / TILE_ROWS;
    a.tv = (rows[2] + TILE_ROWS - 1) / TILE_ROWS;
    a.n = n;
    a.eps = eps;
    const int total = a.tq + a.tk + a.tv;
    hipLaunchKernelGGL(norm_qkv, dim3((total + NQ_TPW - 1) / NQ_TPW), dim3(512), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_rms_norm_quant(const float *x, const float *w, float *out, int8_t *qs, float *d,
                          float *inv_out, int n, float eps, hipStream_t st, int rows) {
    if (n <= 0 || n % QK_K || n > NORM_MAX || !w || rows <= 0) return -1;
    const int waves = n / QK_K < 16 ? n / QK_K : 16;
    if (waves == 8)
        hipLaunchKernelGGL(rms_norm_quant<512>, dim3(rows), dim3(512), 0, st, x, w, out, qs, d, inv_out,
                           n, eps);
    else
        hipLaunchKernelGGL(rms_norm_quant<0>, dim3(rows), dim3(64 * waves), 0, st, x, w, out, qs, d,
                           inv_out, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
