// exact_sum.hpp -- the in-order f32 sum of non-negative terms,
//     float sum = 0.0f; for (j = 0; j < n; ++j) sum += t[j];
// reproduced bit for bit by a whole workgroup in a few passes instead of n
// dependent additions by one lane. Used for the sum of squares of RMSNorm
// (crates/llamd-cpu/src/lib.rs:55-66: `sum += v * v` from 0.0 in order).
//
// Why it is exact. Let S_j be the reference's running sum after terms
// 0..j and T_j the exact one. For non-negative terms, recursive summation
// gives |S_j - T_j| <= E_j = u (1 + u)^n (j + 1) T_j with u = 2^-24
// (each step errs by at most u |S_{j-1} + t_j|; Higham, Accuracy and
// Stability of Numerical Algorithms, 2nd ed., section 4.2). Prefix sums T_j
// are formed in double by a scan; their own error is far below 2^-40 T_{n-1},
// which the bound adds as slack.
// Step j is *certain* when the bound places both S_{j-1} and the exact
// S_{j-1} + t_j inside one binade [2^e, 2^(e+1)) -- below the point
// 2^(e+1) - 2^(e-24) from which round-to-nearest would carry into the next
// binade -- and t_j / 2^(e-23) is not an exact tie (x.5). Then S_{j-1} is an
// integer multiple of the grid q = 2^(e-23), and
//     S_j = fl(S_{j-1} + t_j) = S_{j-1} + q * rint(t_j / q)
// whatever the exact value of S_{j-1}: the step adds a known increment. A
// term t_j == 0 is certain with increment 0. Every other step is *uncertain*
// and is replayed as a real f32 addition.
// Consecutive certain steps lie in one binade (S_j is in both of their
// certified intervals), so every partial sum of their increments is a
// multiple of q below 2^(e+1): exactly representable in f32, under any
// association. One lane then walks only the uncertain steps:
//     S = S + (increments since the last uncertain step)   -- exact
//     S = S + t_u                                          -- the real step
// and finally adds the increments after the last one. Every certain step is
// thereby applied with its exact effect and every uncertain one is the
// reference's own addition, so the result is the reference's, bit for bit.
// Rows with non-finite terms, more than XSUM_LIST_MAX uncertain steps, or
// more than 8192 terms (the bound's (1 + u)^n slack) fold serially instead.
//
// A row of normally distributed values has ~15-20 uncertain steps at
// n = 2048 (a binade crossing or two per power of two the sum passes, and
// the first term).
#pragma once
#include "common.hpp"

namespace llamd {

constexpr int XSUM_LIST_MAX = 256;
constexpr int XSUM_MAX_WAVES = 16;
constexpr int XSUM_MAX_N = 8192;

struct ExactSumLds {
    double wtot[XSUM_MAX_WAVES];  // per-wave sum of the terms (double)
    float wseg[XSUM_MAX_WAVES];   // per-wave segmented increment sum
    int wflag[XSUM_MAX_WAVES];    // per-wave: has an uncertain step
    int wcnt[XSUM_MAX_WAVES];     // per-wave count of uncertain steps
    float2 list[XSUM_LIST_MAX];   // (increments before, term) per uncertain step
    float result;
};

// Inclusive segmented scan over the wave: (v, f) with f = "an uncertain step
// lies in or before this thread's run, after the scan's start", combined as
// (f_b ? v_b : v_a + v_b). Lanes outside a DPP source get (0, 0).
__device__ __forceinline__ void seg_step(float &v, int &f, float ov, int of) {
    v = f ? v : ov + v;
    f |= of;
}
__device__ __forceinline__ void wave_seg_scan(float &v, int &f) {
    seg_step(v, f, dpp<DPP_ROW_SHR1, 0xF, true>(0.0f, v), dpp<DPP_ROW_SHR1, 0xF, true>(0, f));
    seg_step(v, f, dpp<DPP_ROW_SHR2, 0xF, true>(0.0f, v), dpp<DPP_ROW_SHR2, 0xF, true>(0, f));
    seg_step(v, f, dpp<DPP_ROW_SHR4, 0xF, true>(0.0f, v), dpp<DPP_ROW_SHR4, 0xF, true>(0, f));
    seg_step(v, f, dpp<DPP_ROW_SHR8, 0xF, true>(0.0f, v), dpp<DPP_ROW_SHR8, 0xF, true>(0, f));
    seg_step(v, f, dpp<DPP_BCAST15, 0xA>(0.0f, v), dpp<DPP_BCAST15, 0xA>(0, f));
    seg_step(v, f, dpp<DPP_BCAST31, 0xC>(0.0f, v), dpp<DPP_BCAST31, 0xC>(0, f));
}

__device__ __forceinline__ int read_lane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float read_lane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double read_lane(double v, int l) {
    const long long x = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)x, l), hi = __builtin_amdgcn_readlane((int)(x >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// The run of terms a thread holds: thread t of the workgroup owns terms
// [t m, t m + m) of the row, m = ceil(n / threads) <= XSUM_M, in registers.
constexpr int XSUM_M = 8;

// (nt: the workgroup's thread count, a constant where the caller knows it, so
// that the kernel needs no implicit kernel arguments)
__device__ __forceinline__ int xsum_run(int n, int nt) { return (n + nt - 1) / nt; }

// All threads of the workgroup call this (it synchronises the workgroup);
// nt (the thread count) is a multiple of 64, at most 64 * XSUM_MAX_WAVES, and
// at least n / XSUM_M. v[0..cnt) are this thread's terms j0 .. j0 + cnt - 1 (j0 =
// threadIdx.x * xsum_run(n, nt); cnt = what remains of the row, at most the run),
// non-negative or NaN. term(j) recomputes term j for the serial fallback.
// Returns the reference's sum on every thread.
template <class Term>
__device__ float exact_sum_nonneg(const float (&vin)[XSUM_M], int n, int nt, ExactSumLds &L, Term term) {
    constexpr int M = XSUM_M;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int m = xsum_run(n, nt);
    const int j0 = min(tid * m, n), cnt_here = min(m, n - j0);
    float v[M];
#pragma unroll
    for (int k = 0; k < M; ++k) v[k] = k < cnt_here ? vin[k] : 0.0f;

    // pass 1: prefix sums of the terms in double
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < M; ++k)
        if (k < m) s += (double)v[k];  // m is uniform: runs shorter than M skip the rest
    const double incl = wave_inclusive_sum(s);
    if (lane == WAVE - 1) L.wtot[wave] = incl;
    __syncthreads();
    // the waves' totals, combined by the lanes of every wave at once (the
    // same DPP scan in every wave, so ttot is identical across the workgroup)
    const double wsc = wave_inclusive_sum(lane < nw ? L.wtot[lane] : 0.0);
    const double ttot = read_lane(wsc, nw - 1);
    const double woff = wave ? read_lane(wsc, wave - 1) : 0.0;
    bool serial = !(ttot < INFINITY) || n > XSUM_MAX_N || m > M;  // NaN, inf, too long
    int total = 0;
    float tail = 0.0f;
    if (!serial) {
        // pass 2: classify each step (branch-free); certain -> its increment,
        // uncertain -> minus its term (> 0 there: the sign marks it).
        // The bound is taken once per run: with ep = the largest bound on
        // |S - T| within the run, every step's interval lies inside
        // [T_start - ep, T_end + ep]. If that holds one binade e (below its
        // carry point), every step of the run is in range with grid 2^(e-23);
        // if it spans e and e + 1, a step is in range below the boundary
        // B = 2^(e+1) when T_j < B (1 - 2^-25) - ep and above it when
        // T_{j-1} >= B + ep; a run spanning more (the first terms of a row)
        // leaves its non-zero steps uncertain.
        const double c = 0x1p-24 * (1.0 + 0x1p-10), slack = 0x1p-40 * ttot;
        const double tstart = woff + (incl - s), tend = tstart + s;
        const double ep = c * (double)(j0 + M) * tend + slack;
        const double lo = tstart - ep, hi = tend + ep;
        const unsigned long long lob = (unsigned long long)__double_as_longlong(lo);
        const unsigned long long hib = (unsigned long long)__double_as_longlong(hi);
        const int e_run = (int)(lob >> 52) - 1023;  // meaningful when lo is normal
        // the carry point of binade e, 2^e (2 - 2^-24), as a double bit pattern:
        // positive doubles order as their bit patterns
        const auto carry_bits = [](int e) {
            return ((unsigned long long)(e + 1023) << 52) | 0x000FFFFFF0000000ull;
        };
        double thr_a = -INFINITY, thr_b = INFINITY;  // no step in range
        if (lo >= 0x1p-126 && lo < 0x1p126) {
            if (hib < carry_bits(e_run)) {
                thr_a = INFINITY;  // one binade: every step
            } else if (hib < carry_bits(e_run + 1)) {
                const double bnd = ldexp(1.0, e_run + 1);
                thr_a = (bnd - ldexp(bnd, -25)) - ep;
                thr_b = bnd + ep;
            }
        }
        double tprev = tstart;
        float seg = 0.0f;
        int flag = 0, cnt = 0;
#pragma unroll
        for (int k = 0; k < M; ++k) {
            if (k >= m) break;  // uniform; the skipped terms are zeros (certain, no increment)
            const float p = v[k];
            const double tj = tprev + (double)p;
            const bool above = tprev >= thr_b;
            const bool range = (tj < thr_a) | above;
            const int e = above ? e_run + 1 : e_run;
            const float r = ldexpf(p, 23 - e);  // exact in range: p < 2^e
            const float inc = ldexpf(rintf(r), e - 23);
            const bool zero = p == 0.0f;
            const bool certain = zero | (range & (r - floorf(r) != 0.5f));
            v[k] = zero ? 0.0f : (certain ? inc : -p);
            seg = certain ? seg + v[k] : 0.0f;
            flag |= certain ? 0 : 1;
            cnt += certain ? 0 : 1;
            tprev = tj;
        }
        // segmented scan of the increments and a scan of the counts
        float sv = seg;
        int sf = flag;
        wave_seg_scan(sv, sf);
        const int ci = wave_incl_sum_i(cnt);
        if (lane == WAVE - 1) {
            L.wseg[wave] = sv;
            L.wflag[wave] = sf;
            L.wcnt[wave] = ci;
        }
        // this thread's exclusive carry within the wave
        const float ev = dpp<DPP_WAVE_SHR1, 0xF, true>(0.0f, sv);
        const int ef = dpp<DPP_WAVE_SHR1, 0xF, true>(0, sf);
        __syncthreads();
        float gv = lane < nw ? L.wseg[lane] : 0.0f;
        int gf = lane < nw ? L.wflag[lane] : 0;
        wave_seg_scan(gv, gf);
        const int gc = wave_incl_sum_i(lane < nw ? L.wcnt[lane] : 0);
        tail = read_lane(gv, nw - 1);
        total = read_lane(gc, nw - 1);
        const float wc = wave ? read_lane(gv, wave - 1) : 0.0f;
        int off = (wave ? read_lane(gc, wave - 1) : 0) + ci - cnt;
        serial = total > XSUM_LIST_MAX;
        if (!serial && cnt) {
            float carry = ef ? ev : wc + ev;
#pragma unroll
            for (int k = 0; k < M; ++k) {
                if (k >= m) break;
                if (v[k] < 0.0f) {
                    L.list[off++] = make_float2(carry, -v[k]);
                    carry = 0.0f;
                } else {
                    carry = carry + v[k];
                }
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        if (serial) {
            for (int j = 0; j < n; ++j) sum = sum + term(j);
        } else {
            int i = 0;
            for (; i + 16 <= total; i += 16) {
                float2 e[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) e[k] = L.list[i + k];
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    sum = sum + e[k].x;
                    sum = sum + e[k].y;
                }
            }
            for (; i < total; ++i) {
                const float2 e = L.list[i];
                sum = sum + e.x;
                sum = sum + e.y;
            }
            sum = sum + tail;
        }
        L.result = sum;
    }
    __syncthreads();
    return L.result;
}

}  // namespace llamd
