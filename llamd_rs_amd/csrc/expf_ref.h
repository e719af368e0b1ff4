// expf_ref.h -- single-precision exp, bit-identical to glibc's expf.
//
// WHY. The reference computes softmax probabilities (crates/llamd-models/src/
// moe.rs:83) and SiLU (crates/llamd-cpu/src/lib.rs:104) with Rust's f32::exp,
// which on linux-gnu is glibc's expf. Expert selection admits no tolerance, and
// a near-tied routing decision is decided by the last bit of those
// probabilities, so the device must produce the same bits -- "correctly
// rounded" is not enough: glibc's expf is not correctly rounded everywhere.
//
// METHOD. The published algorithm glibc has used since 2.28 (contributed from
// Arm's optimized-routines, sysdeps/ieee754/flt-32/e_expf.c): with N = 32,
//     z  = x * N/ln2          (double)
//     k  = round-to-nearest(z) via the 1.5*2^52 shift, r = z - k
//     s  = 2^(k/N) = T[k mod N] with k/N added into the exponent field
//     y  = s * (C0 r^3 + C1 r^2 + C2 r + 1), evaluated as
//          (C0 r + C1) r^2 + (C2 r + 1)
//     return (float) y
// The table is 2^(i/32) for i = 0..31, correctly rounded to double; the
// three polynomial coefficients are those of glibc's exp2f_data. x86-64 glibc
// dispatches expf to a build compiled with FMA on CPUs that have it; there
// every multiply whose only uses are additions is fused into them (x*N/ln2 +
// shift, x*N/ln2 - k, and the three polynomial steps). EXPF_REF_FMA=1 (the
// default) is that variant. tests/test_expf.py pins this header against the
// host's libm expf (all 2^32 inputs in the full run, a dense sample in the
// quick run) and regenerates the table from 2^(i/32) with Python's decimal
// module.
//
// Used by both the host (tests) and the device (router, SwiGLU). Plain IEEE
// double arithmetic only, so every compiler/target evaluates it identically.
#ifndef LLAMD_EXPF_REF_H
#define LLAMD_EXPF_REF_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define EXPF_REF_FN __host__ __device__ static inline
#else
#define EXPF_REF_FN static inline
#endif

#ifndef EXPF_REF_FMA
#define EXPF_REF_FMA 1
#endif

// 2^(i/32), i = 0..31, as IEEE double bit patterns with (i << 47) subtracted so
// that adding k << 47 for the full k rebuilds 2^(k/32)'s exponent.
// Generated from 2^(i/32) rounded to nearest double; pinned by
// tests/test_expf.py (regenerates it with Python's decimal module).
#define EXPF_REF_TAB                                                            \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,       \
     0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,       \
     0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,       \
     0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,       \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,       \
     0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,       \
     0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,       \
     0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,       \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,       \
     0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,       \
     0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

EXPF_REF_FN double expf_ref_asdouble(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
EXPF_REF_FN uint64_t expf_ref_asuint64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
EXPF_REF_FN uint32_t expf_ref_asuint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
EXPF_REF_FN float expf_ref_asfloat(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

#if defined(__HIP_DEVICE_COMPILE__)
#define EXPF_REF_FMA_OP(a, b, c) __fma_rn((a), (b), (c))
#define EXPF_REF_MUL(a, b) __dmul_rn((a), (b))
#define EXPF_REF_ADD(a, b) __dadd_rn((a), (b))
#define EXPF_REF_SUB(a, b) __dsub_rn((a), (b))
#else
#define EXPF_REF_FMA_OP(a, b, c) __builtin_fma((a), (b), (c))
#define EXPF_REF_MUL(a, b) ((a) * (b))
#define EXPF_REF_ADD(a, b) ((a) + (b))
#define EXPF_REF_SUB(a, b) ((a) - (b))
#endif

#if EXPF_REF_FMA
#define EXPF_REF_MADD(a, b, c) EXPF_REF_FMA_OP(a, b, c)
#else
#define EXPF_REF_MADD(a, b, c) EXPF_REF_ADD(EXPF_REF_MUL(a, b), (c))
#endif

// The core with the table passed in: device code keeps a copy in LDS so the
// lookup is not a dependent global-memory load.
EXPF_REF_FN float expf_ref_tab(float x, const uint64_t *tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;

    const uint32_t ux = expf_ref_asuint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // top12(88.0f): |x| >= 88, or inf/nan
        if (ux == 0xff800000u) return 0.0f;               // -inf
        if (abstop >= 0x7f8) return x + x;                 // nan or +inf
        if (x > 0x1.62e42ep6f) return expf_ref_asfloat(0x7f800000u);  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;               // underflow
    }
    const double xd = (double)x;
    // z = x*N/ln2 feeds both the rounding shift and r = z - k; the FMA build
    // fuses the multiply into each of them.
    double kd = EXPF_REF_MADD(inv_ln2_n, xd, shift);
    const uint64_t ki = expf_ref_asuint64(kd);
    kd = EXPF_REF_SUB(kd, shift);
    const double r = EXPF_REF_MADD(inv_ln2_n, xd, -kd);
    double z;
    uint64_t t = tab[ki % 32];
    t += ki << (52 - 5);
    const double s = expf_ref_asdouble(t);
    z = EXPF_REF_MADD(c0, r, c1);
    const double r2 = EXPF_REF_MUL(r, r);
    double y = EXPF_REF_MADD(c2, r, 1.0);
    y = EXPF_REF_MADD(z, r2, y);
    y = EXPF_REF_MUL(y, s);
    return (float)y;
}

EXPF_REF_FN float expf_ref(float x) {
    const uint64_t tab[32] = EXPF_REF_TAB;
    return expf_ref_tab(x, tab);
}

#if defined(__HIPCC__)
static __constant__ uint64_t k_expf_ref_tab[32] = EXPF_REF_TAB;

// Copy the table into LDS (32 x 8 B) with this wave; every wave that reads it
// calls this first (the writes of several waves carry identical values).
__device__ static inline void expf_ref_tab_fill(uint64_t *lds_tab) {
    const int lane = threadIdx.x & 63;
    if (lane < 32) lds_tab[lane] = k_expf_ref_tab[lane];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}
#endif

#endif
