/*
 * expf with the exact results of glibc 2.35 on x86-64, for device code.
 *
 * glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, the optimized-routines
 * algorithm) writes x*N/ln2 = k + r with N = 32, takes 2^(k/N) from a
 * 32-entry table and 2^(r/N) from a cubic, all in double, and rounds once
 * to float. On x86-64 with FMA the library runs a build of that C file
 * compiled with FMA contraction, so kd, r and the cubic are fused. The
 * table holds the bits of 2^(i/32) rounded to nearest, minus i << 47; the
 * cubic's coefficients are the published ones of that algorithm.
 *
 * This header compiles for the GPU (hipcc) and for the host (a C compiler
 * with -ffp-contract=off); the host build exists so the restatement can be
 * compared with the host's expf on every float (tests/test_expf_restatement.py).
 */
#ifndef MIA_EXPF_GLIBC_H
#define MIA_EXPF_GLIBC_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define MIA_EXPF_FN static __device__ __forceinline__
#define MIA_EXPF_TABLE static __constant__ const
#else
#define MIA_EXPF_FN static inline
#define MIA_EXPF_TABLE static const
#endif

MIA_EXPF_TABLE uint64_t mia_expf_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL,
    0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL,
    0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL,
    0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL,
    0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL,
    0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL,
    0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL,
    0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL,
    0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

/* The algorithm with the table passed in (device code may keep a copy in
 * LDS, where a lookup costs far less than a global-memory load). */
MIA_EXPF_FN float mia_expf_glibc_tab(float x, const uint64_t *tab) {
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                   /* |x| >= 88 or nan */
        if (ux == 0xff800000u) return 0.0f;  /* -inf */
        if (abstop >= 0x7f8) return x + x;   /* inf, nan */
        if (x > 0x1.62e42ep6f) {             /* overflow */
            const uint32_t inf = 0x7f800000u;
            float r;
            memcpy(&r, &inf, 4);
            return r;
        }
        if (x < -0x1.9fe368p6f) return 0.0f; /* underflow */
    }
    const double n = 32.0;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * n;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / n / n / n;
    const double c1 = 0x1.ebfce50fac4f3p-3 / n / n;
    const double c2 = 0x1.62e42ff0c52d6p-1 / n;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd = kd - shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    double s;
    memcpy(&s, &t, 8);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

MIA_EXPF_FN float mia_expf_glibc(float x) { return mia_expf_glibc_tab(x, mia_expf_tab); }

#endif
