#ifndef MIA_SYNTH_H
#define MIA_SYNTH_H
/*
 * Seeded synthetic tensors for the Qwen3-30B-A3B MoE FFN workloads.
 *
 * There is no checkpoint to load offline, so every weight and input is drawn
 * from a counter-based generator keyed by (seed, stream, index). The same
 * header is compiled by the host C compiler and by hipcc for device code, and
 * the arithmetic is restricted to integer ops and IEEE-754 double +, -, *, /
 * and sqrt (all correctly rounded on both sides, evaluated in a fixed order
 * with contraction disabled), so a tensor generated in HBM is bit-identical
 * to the same tensor generated on the CPU.
 *
 * Normal deviates use the Box-Muller transform; ln() and cos() are evaluated
 * with fixed polynomials written out below rather than libm, whose last bits
 * differ between glibc and the device math library.
 *
 * Stream ids (which tensor a value belongs to):
 *   x input             MIA_STREAM_X                      index t*dim + i
 *   router of layer l   MIA_STREAM_ROUTER + l             index e*dim + i
 *   expert matrix       MIA_STREAM_EXPERT + (l*E + e)*3 + m  (m: 0 gate, 1 up, 2 down)
 *                                                        index row*cols + col
 * Gate/up are [expert_hidden x dim], down is [dim x expert_hidden], row-major,
 * the shapes of the expert blob in the .mia format.
 */
#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define MIA_SYNTH_FN static inline __host__ __device__
#else
#define MIA_SYNTH_FN static inline
#endif

#define MIA_STREAM_X ((uint64_t)1 << 40)
#define MIA_STREAM_ROUTER ((uint64_t)2 << 40)
#define MIA_STREAM_EXPERT ((uint64_t)3 << 40)

MIA_SYNTH_FN uint64_t mia_synth_mix(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ULL;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return z;
}

/* Key of one tensor: hoisted out of per-element loops. */
MIA_SYNTH_FN uint64_t mia_synth_key(uint64_t seed, uint64_t stream) {
    return mia_synth_mix(mia_synth_mix(seed ^ 0x6A09E667F3BCC909ULL) + stream);
}

MIA_SYNTH_FN uint64_t mia_synth_bits(uint64_t key, uint64_t i) {
    return mia_synth_mix(key + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

/* ln(u) for u in (0, 1]: u = m * 2^k with m in [sqrt(1/2), sqrt(2)),
 * ln m = 2 atanh(s), s = (m-1)/(m+1), |s| < 0.1716; odd series to s^23. */
MIA_SYNTH_FN double mia_synth_ln(double u) {
    union {
        double d;
        uint64_t b;
    } v;
    v.d = u;
    int k = (int)((v.b >> 52) & 0x7FF) - 1023;
    v.b = (v.b & 0x000FFFFFFFFFFFFFULL) | 0x3FF0000000000000ULL; /* m in [1,2) */
    double m = v.d;
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        k = k + 1;
    }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double p = 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    double lnm = 2.0 * s * p;
    return (double)k * 0.6931471805599453 + lnm;
}

/* cos(2*pi*f) with f = w / 2^32, using the exact quadrant split of w. */
MIA_SYNTH_FN double mia_synth_cos2pi(uint32_t w) {
    uint32_t q = w >> 30;
    double phi = (double)(w & 0x3FFFFFFFu) * (1.0 / 1073741824.0) *
                 1.5707963267948966; /* [0, pi/2) */
    double p2 = phi * phi;
    /* Taylor series of cos and sin to degree 22/23. */
    double c = -1.0 / 1124000727777607680000.0;          /* -1/22! */
    c = c * p2 + 1.0 / 2432902008176640000.0;            /* 1/20! */
    c = c * p2 - 1.0 / 6402373705728000.0;               /* 1/18! */
    c = c * p2 + 1.0 / 20922789888000.0;                 /* 1/16! */
    c = c * p2 - 1.0 / 87178291200.0;                    /* 1/14! */
    c = c * p2 + 1.0 / 479001600.0;                      /* 1/12! */
    c = c * p2 - 1.0 / 3628800.0;                        /* 1/10! */
    c = c * p2 + 1.0 / 40320.0;                          /* 1/8!  */
    c = c * p2 - 1.0 / 720.0;                            /* 1/6!  */
    c = c * p2 + 1.0 / 24.0;                             /* 1/4!  */
    c = c * p2 - 0.5;                                    /* 1/2!  */
    c = c * p2 + 1.0;
    double s = -1.0 / 25852016738884976640000.0;         /* -1/23! */
    s = s * p2 + 1.0 / 51090942171709440000.0;           /* 1/21! */
    s = s * p2 - 1.0 / 121645100408832000.0;             /* 1/19! */
    s = s * p2 + 1.0 / 355687428096000.0;                /* 1/17! */
    s = s * p2 - 1.0 / 1307674368000.0;                  /* 1/15! */
    s = s * p2 + 1.0 / 6227020800.0;                     /* 1/13! */
    s = s * p2 - 1.0 / 39916800.0;                       /* 1/11! */
    s = s * p2 + 1.0 / 362880.0;                         /* 1/9!  */
    s = s * p2 - 1.0 / 5040.0;                           /* 1/7!  */
    s = s * p2 + 1.0 / 120.0;                            /* 1/5!  */
    s = s * p2 - 1.0 / 6.0;                              /* 1/3!  */
    s = s * p2 + 1.0;
    s = s * phi;
    if (q == 0) return c;
    if (q == 1) return -s;
    if (q == 2) return -c;
    return s;
}

/* Standard normal deviate number i of the tensor with key `key`. */
MIA_SYNTH_FN double mia_synth_normal(uint64_t key, uint64_t i) {
    uint64_t b = mia_synth_bits(key, i);
    double u1 = ((double)(uint32_t)(b >> 32) + 0.5) * (1.0 / 4294967296.0);
    double r = sqrt(-2.0 * mia_synth_ln(u1));
    return r * mia_synth_cos2pi((uint32_t)b);
}

/* fp32 value sigma * N(0,1), rounded once from double. */
MIA_SYNTH_FN float mia_synth_f32(uint64_t key, uint64_t i, double sigma) {
    return (float)(mia_synth_normal(key, i) * sigma);
}

#endif
