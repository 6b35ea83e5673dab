/* bf16 hi / lo halves of an f32 activation, for the BF16 matrix-core
 * kernels: x = hi + lo + r with hi = bf16(x) (round to nearest, ties to
 * even), lo = bf16(x - hi) and |r| <= 2^-17 |x|, so that w * hi and w * lo
 * are exact f32 products of a bf16 weight w and their sum is w * x to about
 * the rounding of biv's dot_bf16 (quant.rs:1228-1256).
 *
 * Non-finite x: hi = bf16(x) (Inf stays Inf, NaN becomes the quiet NaN
 * 0x7FC0) and lo = 0, so that w * hi + w * lo is w * x as the reference forms
 * it (x - hi would be NaN).  Finite x whose nearest bf16 overflows (|x| >
 * 0x1.fefp127, up to FLT_MAX): hi is x truncated to the largest finite
 * bf16 instead, and lo the rest, so that a finite x keeps finite halves.
 *
 * Plain C99 so that the host test compiles the same code with gcc; in HIP
 * device code it is a __host__ __device__ function. */
#ifndef BIV_BF16_SPLIT_H
#define BIV_BF16_SPLIT_H

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define BIV_BF16_QUAL __host__ __device__ static inline
#else
#define BIV_BF16_QUAL static inline
#endif

BIV_BF16_QUAL uint32_t biv_f32_bits(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

BIV_BF16_QUAL float biv_bits_f32(uint32_t u)
{
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* bf16 bits of x, round to nearest, ties to even; NaN gives 0x7FC0 */
BIV_BF16_QUAL uint32_t bf16_bits(float x)
{
    const uint32_t u = biv_f32_bits(x);
    if (x != x) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

/* the halves of x as bf16 bits */
BIV_BF16_QUAL void bf16_split(float x, uint32_t *hi, uint32_t *lo)
{
    uint32_t h = bf16_bits(x);
    const int finite = (biv_f32_bits(x) & 0x7F800000u) != 0x7F800000u;
    if (finite && (h & 0x7FFFu) == 0x7F80u) h = biv_f32_bits(x) >> 16; /* rounded up to Inf: truncate */
    *hi = h;
    *lo = finite ? bf16_bits(x - biv_bits_f32(h << 16)) : 0u;
}

#endif
