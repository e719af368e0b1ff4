// compat.hip -- device kernels behind the entry points that make this library
// a link-compatible replacement for crates/llamd-rocm: weights in the
// reference's own device layouts (ggml 210-byte blocks, the planar repack),
// the unsigned-activation ("udot") operand form, and the f32 pieces of the
// decode step that take a position or a per-sequence meta row.
//
// Weights. The reference uploads Q6_K either verbatim (DevBuf::from_bytes,
// crates/llamd-runtime/src/device.rs:231-233) or as four planes
// (repack_q6k_planar, crates/llamd-quant/src/dot.rs:400-423: ql, qh, sc, d,
// block-major). Both are permutations of the same bytes. q6k_retile gathers
// either form into this library's tiled segments (host/layout.cpp defines
// them: tile_segment is the host statement of the same permutation), so every
// Q6_K entry point runs the MFMA kernels of q6k_mv.hip on it.
//
// Activations. The udot entry points (crates/llamd-rocm/kernels/
// llamd_udot.hip:55-75) carry Q8_K quants biased to unsigned, b = q ^ 0x80,
// and per-16 sums of b. The signed quants are recovered exactly by the same
// XOR, so the matvecs here are the bit-exact signed kernels, not the
// reference's reassociated udot identity.
//
// f32 pieces. RoPE reads cos / sin from a table the host fills with the
// reference CPU path's own libm calls (theta = pos / powf(base, 2i/hd),
// crates/llamd-cpu/src/lib.rs:183-205); norms and attention are the bit-exact
// kernels of norm.hip and decode.hip with a sequence stride added.
#include <algorithm>

#include "common.hpp"
#include "expf_ref.h"
#include "launch.hpp"
#include "q8k_wave.hpp"
#include "row_scale.hpp"

namespace llamd {
namespace {

// ---- Q6_K: ggml / planar bytes -> tiled segments -----------------------------
// Byte (field f, j) of block i sits at base + off[f] + i * stride[f] + j for
// the fields ql (128 B), qh (64 B), sc (16 B), d (2 B).
__device__ __forceinline__ int code6_at(const Q6kSource &s, size_t i, int e) {
    const int h = e >> 7, ii = e & 127, q4 = ii >> 5, l = ii & 31;
    const uint8_t lo = s.base[s.off[0] + i * s.stride[0] + h * 64 + l + (q4 & 1) * 32];
    const uint8_t hi = s.base[s.off[1] + i * s.stride[1] + h * 32 + l];
    return ((lo >> (4 * (q4 >> 1))) & 0xF) | (((hi >> (2 * q4)) & 3) << 4);
}

// One thread per output dword of the tiled layout (840 per 3360-byte segment).
__global__ __launch_bounds__(256) void q6k_retile(Q6kSource s, int rows, int blocks, uint32_t *out,
                                                  long n_dw) {
    for (long g = (long)blockIdx.x * 256 + threadIdx.x; g < n_dw; g += (long)gridDim.x * 256) {
        const long seg = g / 840;
        const int o = (int)(g - seg * 840) * 4;
        const int t = (int)(seg / blocks), b = (int)(seg - (long)t * blocks);
        uint32_t val = 0;
        if (o < SEG_SC) {
            const int part = o >> 10, L = (o & 1023) >> 4, q = (o & 15) >> 2;
            const int n = L & 15, sq = L >> 4, r = 16 * t + n;
            if (r < rows) {
                const size_t i = (size_t)r * blocks + b;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int m0 = 8 * sq + j, m1 = m0 + 4;
                    uint32_t byte;
                    if (part < 2) {
                        const int c = 4 * part + q;
                        byte = (code6_at(s, i, 8 * m0 + c) & 0xF) |
                               ((code6_at(s, i, 8 * m1 + c) & 0xF) << 4);
                    } else {
                        const int c0 = 2 * q, c1 = 2 * q + 1;
                        byte = (code6_at(s, i, 8 * m0 + c0) >> 4) |
                               ((code6_at(s, i, 8 * m1 + c0) >> 4) << 2) |
                               ((code6_at(s, i, 8 * m0 + c1) >> 4) << 4) |
                               ((code6_at(s, i, 8 * m1 + c1) >> 4) << 6);
                    }
                    val |= byte << (8 * j);
                }
            }
        } else if (o < SEG_D) {
            const int L = (o - SEG_SC) >> 2, n = L & 15, sq = L >> 4, r = 16 * t + n;
            if (r < rows) {
                const uint8_t *sc = s.base + s.off[2] + ((size_t)r * blocks + b) * s.stride[2] + 4 * sq;
                val = (uint32_t)sc[0] | ((uint32_t)sc[1] << 8) | ((uint32_t)sc[2] << 16) |
                      ((uint32_t)sc[3] << 24);
            }
        } else {
            const int n0 = (o - SEG_D) >> 1;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int r = 16 * t + n0 + k;
                if (r < rows) {
                    const uint8_t *dp = s.base + s.off[3] + ((size_t)r * blocks + b) * s.stride[3];
                    val |= ((uint32_t)dp[0] | ((uint32_t)dp[1] << 8)) << (16 * k);
                }
            }
        }
        out[g] = val;
    }
}

// ---- memset without a memset node (graph-capture safe) -----------------------
// (the grid-stride kernels below take their grid width as an argument: no
// implicit kernel arguments, a smaller kernarg segment per launch)
__global__ __launch_bounds__(256) void fill_bytes(uint8_t *p, uint8_t v, size_t head, size_t n16,
                                                  size_t tail, unsigned nblk) {
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, step = (size_t)nblk * 256;
    const uint32_t w = 0x01010101u * v;
    const uint4 q = make_uint4(w, w, w, w);
    for (size_t i = tid; i < head; i += step) p[i] = v;
    uint4 *mid = (uint4 *)(p + head);
    for (size_t i = tid; i < n16; i += step) mid[i] = q;
    uint8_t *end = p + head + n16 * 16;
    for (size_t i = tid; i < tail; i += step) end[i] = v;
}

// ---- activations -------------------------------------------------------------
// Natural-layout Q8_K quants (signed, or biased with `flip` = 0x80808080)
// [n_act][blocks * 256] -> signed natural copy.
__global__ __launch_bounds__(256) void act_unbias(const uint32_t *q, uint32_t flip, uint32_t *out,
                                                  size_t n_dw, unsigned nblk) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n_dw; i += (size_t)nblk * 256)
        out[i] = q[i] ^ flip;
}

// Natural-layout quants and scales of n_act tokens -> the token-chunked
// operand layout of q6k_mv_batched (q8k_wave.hpp): block b of chunk k is 4 KiB
// at (k * blocks + b) * 4096, class plane c = e % 8 at c * 512, token n of the
// chunk at n * 32, byte e / 8. Token slots past n_act are zero.
__global__ __launch_bounds__(256) void act_to_chunks(const uint8_t *q, const float *d, uint8_t flip,
                                                     int n_act, int blocks, uint8_t *cq, float *cd,
                                                     size_t n_bytes, unsigned nblk) {
    for (size_t D = (size_t)blockIdx.x * 256 + threadIdx.x; D < n_bytes;
         D += (size_t)nblk * 256) {
        const size_t kb = D >> 12;  // chunk * blocks + block
        const int w = (int)(D & 4095);
        const int k = (int)(kb / blocks), b = (int)(kb - (size_t)k * blocks);
        const int c = w >> 9, tn = (w & 511) >> 5, m = w & 31;
        const int t = 16 * k + tn, e = 8 * m + c;
        cq[D] = t < n_act ? (uint8_t)(q[((size_t)t * blocks + b) * QK_K + e] ^ flip) : (uint8_t)0;
        if (w < 16) {
            const int tt = 16 * k + w;
            cd[kb * 16 + w] = tt < n_act ? d[(size_t)tt * blocks + b] : 0.0f;
        }
    }
}

// In place: signed Q8_K quants -> b = q ^ 0x80, and the per-16 sums of b
// (llamd_udot.hip:55-75 and 148-159). One wave per 256-value block, four
// values per lane, four lanes per group.
__global__ __launch_bounds__(256) void bias_sums(const int8_t *qs, uint8_t *qb, int32_t *sb,
                                                 int nblocks) {
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    const uint32_t v = ((const uint32_t *)(qs + (size_t)b * QK_K))[lane] ^ 0x80808080u;
    ((uint32_t *)(qb + (size_t)b * QK_K))[lane] = v;
    int s = (int)(v & 0xFF) + (int)((v >> 8) & 0xFF) + (int)((v >> 16) & 0xFF) + (int)(v >> 24);
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    if ((lane & 3) == 0) sb[(size_t)b * 16 + (lane >> 2)] = s;
}

// ---- RoPE / QK-norm / cache store with a position per sequence ---------------
// One wave per head g of n_seq * n_heads: pos = pos_p[s * pos_stride] (or
// pos_fixed, or s itself when pos_fixed < 0 and there is no pos_p). With w:
// x = (x * scale) * w first (per_head_rms_norm, crates/llamd-runtime/src/
// layer.rs:62-79). Then NeoX rotation with the table row of pos
// (a*cos - b*sin, a*sin + b*cos), in place; with kc, the rotated head and the
// matching v head are also stored at row pos of the sequence's cache slice.
// The table (host libm: cosf / sinf of pos / powf(base, 2i/hd), the CPU
// path's own calls) covers positions below cs_rows; a position past it is
// rotated with theta = pos / den[i] (the table's denominators, so theta is
// the CPU's bit for bit) and the device's sincosf, within a few ulp of the
// CPU's cos / sin (no table, so any position a cache holds works). A
// negative position (device meta) writes NaN and stores nothing; a position
// at or past cache_rows is rotated but not stored.
__global__ __launch_bounds__(64) void head_norm_rope(HeadRopeArgs a) {
    __shared__ __align__(16) float sq[256];
    __shared__ float buf[256];
    const int lane = threadIdx.x, g = blockIdx.x, s = g / a.n_heads, hh = g - s * a.n_heads;
    const int hd = a.hd, half = hd / 2;
    int pos = a.pos_fixed;
    if (a.pos_p) pos = a.pos_p[(size_t)s * a.pos_stride];
    else if (pos < 0) pos = s;
    float *x = a.x + ((size_t)s * a.n_heads + hh) * hd;
    if (a.w) {
        const float scale = row_scale_wave(x, hd, a.eps, sq);
        for (int d = lane; d < hd; d += WAVE) buf[d] = (x[d] * scale) * a.w[d];
    } else {
        for (int d = lane; d < hd; d += WAVE) buf[d] = x[d];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const bool ok = pos >= 0;
    const bool in_table = ok && pos < a.cs_rows;
    const float2 *row = a.cs + (size_t)(in_table ? pos : 0) * half;
    float *kc = nullptr, *vc = nullptr;
    if (a.kc && ok && pos < a.cache_rows) {
        const size_t o = (size_t)s * a.cache_seq_stride + (size_t)pos * a.kv_dim + (size_t)hh * hd;
        kc = a.kc + o;
        vc = a.vc + o;
    }
    for (int i = lane; i < half; i += WAVE) {
        const float p = buf[i], q = buf[i + half];
        float2 c;
        if (in_table) {
            c = row[i];
        } else {
            const float theta = (float)pos / a.den[i];
            sincosf(theta, &c.y, &c.x);
        }
        float lo = p * c.x - q * c.y;
        float hi = p * c.y + q * c.x;
        if (!ok) lo = hi = __builtin_nanf("");
        x[i] = lo;
        x[i + half] = hi;
        if (kc) {
            kc[i] = lo;
            kc[i + half] = hi;
        }
    }
    if (vc) {
        const float *v = a.v + (size_t)s * a.n_heads * hd + (size_t)hh * hd;
        for (int d = lane; d < hd; d += WAVE) vc[d] = v[d];
    }
}

// kc[pos * kv_dim + i] = k[i], likewise v (llamd_forward.hip fk_kv_store).
__global__ __launch_bounds__(256) void kv_store(float *kc, float *vc, const float *k, const float *v,
                                                int pos, int kv_dim) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= kv_dim) return;
    kc[(size_t)pos * kv_dim + i] = k[i];
    vc[(size_t)pos * kv_dim + i] = v[i];
}

// ---- elementwise (CpuBackend::add / mul / scale / silu, lib.rs:103-118) -----
__global__ __launch_bounds__(256) void ew_binary(const float *a, const float *b, float *o, size_t n,
                                                 int op, unsigned nblk) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)nblk * 256)
        o[i] = op == 0 ? a[i] + b[i] : a[i] * b[i];
}

__global__ __launch_bounds__(256) void ew_scale(const float *x, float by, float *o, size_t n,
                                                unsigned nblk) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)nblk * 256)
        o[i] = x[i] * by;
}

__global__ __launch_bounds__(256) void ew_silu(const float *x, float *o, size_t n, unsigned nblk) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 64) expf_ref_tab_fill(tab);
    __syncthreads();
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)nblk * 256)
        o[i] = silu_ref(x[i], tab);
}

// CpuBackend::softmax per row (lib.rs:81-101): max fold, e = exp(s - max),
// the sum of e in order from 0.0, inv = 1 / sum, e * inv. One wave per row;
// lane 0 adds the row in order.
__global__ __launch_bounds__(64) void softmax_rows(const float *x, float *o, int n) {
    __shared__ uint64_t tab[32];
    __shared__ float red;
    const int lane = threadIdx.x;
    const float *src = x + (size_t)blockIdx.x * n;
    float *dst = o + (size_t)blockIdx.x * n;
    expf_ref_tab_fill(tab);
    float m = -INFINITY;
    for (int i = lane; i < n; i += WAVE) m = fmaxf(m, src[i]);
    m = wave_reduce(m, -INFINITY, [](float p, float q) { return fmaxf(p, q); });
    m = __shfl(m, 63, WAVE);
    for (int i = lane; i < n; i += WAVE) dst[i] = expf_ref_tab(src[i] - m, tab);
    __threadfence();  // the other lanes' e values reach memory before lane 0 reads them
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) sum = sum + dst[i];
        red = __fdiv_rn(1.0f, sum);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const float inv = red;
    for (int i = lane; i < n; i += WAVE) dst[i] = dst[i] * inv;
}

// CpuBackend::matmul (lib.rs:126-149): out[j * m + i] = sum over t in order
// of w[i][t] * x[j][t], from 0.0, unfused. One thread per output element;
// the 64 rows of a wave read their w rows through LDS in 64-wide k strips.
__global__ __launch_bounds__(64) void matmul_f32_seq(const float *w, const float *x, float *out,
                                                     int m, int n, int k) {
    __shared__ float ws[64][65];
    const int lane = threadIdx.x;
    const int i0 = blockIdx.x * 64, j = blockIdx.y;
    const float *xr = x + (size_t)j * k;
    float acc = 0.0f;
    for (int t0 = 0; t0 < k; t0 += 64) {
        const int kt = min(64, k - t0);
        for (int r = 0; r < 64; ++r) {
            const int i = i0 + r;
            ws[r][lane] = (i < m && lane < kt) ? w[(size_t)i * k + t0 + lane] : 0.0f;
        }
        __syncthreads();
        for (int t = 0; t < kt; ++t) acc = acc + ws[lane][t] * xr[t0 + t];
        __syncthreads();
    }
    if (i0 + lane < m) out[(size_t)j * m + i0 + lane] = acc;
}

}  // namespace

int launch_q6k_retile(const Q6kSource &s, int rows, int blocks, void *tiled, hipStream_t st) {
    if (rows <= 0 || blocks <= 0) return -1;
    const long n_dw = (long)((rows + 15) / 16) * blocks * 840;
    const long grid = std::min<long>((n_dw + 255) / 256, 65536);
    hipLaunchKernelGGL(q6k_retile, dim3((unsigned)grid), dim3(256), 0, st, s, rows, blocks,
                       (uint32_t *)tiled, n_dw);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fill(void *p, int value, size_t bytes, hipStream_t st) {
    if (!bytes) return 0;
    const size_t mis = (16 - ((uintptr_t)p & 15)) & 15;
    const size_t head = std::min(mis, bytes);
    const size_t n16 = (bytes - head) / 16, tail = bytes - head - n16 * 16;
    const size_t work = std::max(std::max(head, tail), n16);
    const size_t grid = std::min<size_t>((work + 255) / 256, 8192);
    const unsigned nblk = (unsigned)std::max<size_t>(grid, 1);
    hipLaunchKernelGGL(fill_bytes, dim3(nblk), dim3(256), 0, st, (uint8_t *)p, (uint8_t)value, head,
                       n16, tail, nblk);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_act_unbias(const void *q, bool biased, int n_act, int blocks, int8_t *out,
                      hipStream_t st) {
    const size_t n_dw = (size_t)n_act * blocks * QK_K / 4;
    const size_t grid = std::min<size_t>((n_dw + 255) / 256, 4096);
    const unsigned nblk = (unsigned)std::max<size_t>(grid, 1);
    hipLaunchKernelGGL(act_unbias, dim3(nblk), dim3(256), 0, st, (const uint32_t *)q,
                       biased ? 0x80808080u : 0u, (uint32_t *)out, n_dw, nblk);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_act_to_chunks(const void *q, const float *d, bool biased, int n_act, int blocks,
                         int8_t *cq, float *cd, hipStream_t st) {
    const size_t chunks = (size_t)(n_act + 15) / 16;
    const size_t n_bytes = chunks * blocks * 4096;
    const size_t grid = std::min<size_t>((n_bytes + 255) / 256, 8192);
    hipLaunchKernelGGL(act_to_chunks, dim3((unsigned)grid), dim3(256), 0, st, (const uint8_t *)q, d,
                       (uint8_t)(biased ? 0x80 : 0), n_act, blocks, (uint8_t *)cq, cd, n_bytes,
                       (unsigned)grid);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_bias_sums(const int8_t *qs, uint8_t *qb, int32_t *sb, int nblocks, hipStream_t st) {
    if (nblocks <= 0) return -1;
    hipLaunchKernelGGL(bias_sums, dim3((nblocks + 3) / 4), dim3(256), 0, st, qs, qb, sb, nblocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_head_norm_rope(const HeadRopeArgs &a, int nseq, hipStream_t st) {
    if (a.hd <= 0 || a.hd % 2 || a.hd > 256 || a.n_heads <= 0 || nseq <= 0 || !a.cs) return -1;
    hipLaunchKernelGGL(head_norm_rope, dim3(nseq * a.n_heads), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_kv_store(float *kc, float *vc, const float *k, const float *v, int pos, int kv_dim,
                    hipStream_t st) {
    if (kv_dim <= 0 || pos < 0) return -1;
    hipLaunchKernelGGL(kv_store, dim3((kv_dim + 255) / 256), dim3(256), 0, st, kc, vc, k, v, pos,
                       kv_dim);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

static unsigned ew_grid(size_t n) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>((n + 255) / 256, 16384));
}

int launch_ew(int op, const float *a, const float *b, float by, float *o, size_t n,
              hipStream_t st) {
    if (!n) return 0;
    if (op == EW_ADD || op == EW_MUL)
        hipLaunchKernelGGL(ew_binary, dim3(ew_grid(n)), dim3(256), 0, st, a, b, o, n,
                           op == EW_ADD ? 0 : 1, ew_grid(n));
    else if (op == EW_SCALE)
        hipLaunchKernelGGL(ew_scale, dim3(ew_grid(n)), dim3(256), 0, st, a, by, o, n, ew_grid(n));
    else if (op == EW_SILU)
        hipLaunchKernelGGL(ew_silu, dim3(ew_grid(n)), dim3(256), 0, st, a, o, n, ew_grid(n));
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_softmax_rows(const float *x, float *o, int rows, int n, hipStream_t st) {
    if (rows <= 0 || n <= 0) return -1;
    hipLaunchKernelGGL(softmax_rows, dim3(rows), dim3(64), 0, st, x, o, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_matmul_f32_seq(const float *w, const float *x, float *out, int m, int n, int k,
                          hipStream_t st) {
    if (m <= 0 || n <= 0 || k <= 0 || n > 65535) return -1;
    hipLaunchKernelGGL(matmul_f32_seq, dim3((m + 63) / 64, n), dim3(64), 0, st, w, x, out, m, n, k);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
