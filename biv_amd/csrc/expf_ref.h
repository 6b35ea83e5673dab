/* e^x in f32 with the bits glibc's expf returns on the reference's x86-64
 * Linux host: biv's f32::exp (ops::softmax, ops::sigmoid, ops.rs:159-201)
 * calls it there.  This is the published method of glibc's expf (from Arm's
 * optimized-routines): x * 32/ln2 = k + r, 2^(k/32) from a 32-entry table of
 * 2^(i/32) as doubles, 2^(r/32) by a cubic in double, one rounding to f32.
 * Checked against glibc 2.35 over every f32 in (-103, 88): two inputs of
 * 2.2e9 differ by one ulp (tests/test_expf_ref.py).
 *
 * Plain C99 so that the host test compiles the same code with gcc; in HIP
 * device code it is a __device__ function. */
#ifndef BIV_EXPF_REF_H
#define BIV_EXPF_REF_H

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define BIV_EXPF_QUAL __host__ __device__ static inline
#else
#define BIV_EXPF_QUAL static inline
#endif

/* 2^(i/32) rounded to double, minus i << 47 (the exponent added back in
 * biv_expf_finish) */
#define BIV_EXPF_TAB_INIT                                                                              \
    {                                                                                                  \
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,    \
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,    \
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,    \
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,    \
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,    \
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,    \
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,    \
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,    \
    }

/* The two halves of biv_expf_ref, for callers that keep the table
 * elsewhere (in GPU shared memory): the reduction x * 32/ln2 = k + r
 * (returns the table index k % 32; harmless for NaN and out-of-range x),
 * then the cubic and the special cases given tab[k % 32]. */
BIV_EXPF_QUAL uint32_t biv_expf_reduce(float x, double *r, uint64_t *ki)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double z = inv_ln2_n * (double)x;
    double kd = z + shift;
    memcpy(ki, &kd, 8);
    kd -= shift;
    *r = z - kd;
    return (uint32_t)(*ki % 32);
}

BIV_EXPF_QUAL float biv_expf_finish(float x, double r, uint64_t ki, uint64_t entry)
{
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    if (x != x) return x + x;                      /* NaN */
    if (x > 0x1.62e42ep6f) return x * 0x1p127f * 0x1p127f; /* overflow to +inf */
    if (x < -0x1.9fe368p6f) return 0.0f;           /* underflow, -inf included */
    uint64_t t = entry + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double zz = c0 * r + c1;
    const double r2 = r * r;
    double y = c2 * r + 1.0;
    y = zz * r2 + y;
    y = y * s;
    return (float)y;
}

/* biv_expf_finish with no early return: the polynomial is evaluated for
 * every x and the special cases are selected after, so a caller's table
 * read is never behind a branch.  Same bits as biv_expf_finish. */
BIV_EXPF_QUAL float biv_expf_finish_sel(float x, double r, uint64_t ki, uint64_t entry)
{
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint64_t t = entry + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double zz = c0 * r + c1;
    const double r2 = r * r;
    double y = c2 * r + 1.0;
    y = zz * r2 + y;
    y = y * s;
    float res = (float)y;
    res = x < -0x1.9fe368p6f ? 0.0f : res;
    res = x > 0x1.62e42ep6f ? x * 0x1p127f * 0x1p127f : res;
    return x != x ? x + x : res;
}

BIV_EXPF_QUAL float biv_expf_ref(float x)
{
    static const uint64_t tab[32] = BIV_EXPF_TAB_INIT;
    double r;
    uint64_t ki;
    const uint32_t i = biv_expf_reduce(x, &r, &ki);
    return biv_expf_finish(x, r, ki, tab[i]);
}

#endif
