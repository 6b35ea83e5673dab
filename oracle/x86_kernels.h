/* Int8 dot kernels of the CPU oracle, instantiated twice by oracle.c: once for
 * AVX2 (maddubs + madd) and once for AVX-VNNI (dpbusd).  TEST INFRASTRUCTURE
 * ONLY — included by oracle.c, never by the product library.
 *
 * Each kernel follows the accumulation order of biv's x86 int8 kernels so that
 * the f32 result is the one the reference computes on the same x86 host:
 *   dot_q8_0  engine/src/quant.rs:1368-1382  (acc[i&1], sign trick 1294-1299)
 *   dot_q4k   engine/src/quant.rs:1384-1423  (acc_lo / acc_hi, mins subtracted last)
 *   dot_q6k   engine/src/quant.rs:1475-1533  (acc[k&1], i16 sub-scales via madd)
 * The byte-dot primitive is engine/src/quant.rs:1538-1544.
 *
 * Expected macros: SUF (name suffix), TGT (target attribute), DOT_U8_I8(u, s).
 */

#define CAT_(a, b) a##_##b
#define CAT(a, b) CAT_(a, b)

static inline TGT __m256i CAT(dot_u8_i8, SUF)(__m256i u, __m256i s) { return DOT_U8_I8(u, s); }

/* signed x signed bytes: |a| as unsigned times s carrying a's sign */
static inline TGT __m256i CAT(dot_i8_i8, SUF)(__m256i a, __m256i s)
{
    return CAT(dot_u8_i8, SUF)(_mm256_sign_epi8(a, a), _mm256_sign_epi8(s, a));
}

static TGT float CAT(dot_q8_0, SUF)(const uint8_t *w, const int8_t *xq, const float *xd, size_t nb)
{
    __m256 acc[2] = {_mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + 34 * i;
        __m256i p = CAT(dot_i8_i8, SUF)(_mm256_loadu_si256((const __m256i *)(b + 2)),
                                         _mm256_loadu_si256((const __m256i *)(xq + 32 * i)));
        acc[i & 1] = fma_i32(acc[i & 1], p, f16x(b) * xd[i]);
    }
    return hsum(_mm256_add_ps(acc[0], acc[1]));
}

static TGT float CAT(dot_q4k, SUF)(const uint8_t *w, const int8_t *xq, const float *xd, const float *xs,
                                    size_t nb32)
{
    size_t nsb = nb32 / 8;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc_lo = _mm256_setzero_ps(), acc_hi = _mm256_setzero_ps();
    float mins = 0.0f;
    for (size_t i = 0; i < nsb; i++) {
        const uint8_t *b = w + 144 * i;
        float d = f16x(b), dmin = f16x(b + 2);
        const uint8_t *scales = b + 4;
        const int8_t *x = xq + 256 * i;
        for (int j = 0; j < 4; j++) {
            __m256i v = _mm256_loadu_si256((const __m256i *)(b + 16 + 32 * j));
            __m256i lo = _mm256_and_si256(v, m4);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(v, 4), m4);
            uint8_t s1, m1, s2, m2;
            scale_min_k4(2 * j, scales, &s1, &m1);
            scale_min_k4(2 * j + 1, scales, &s2, &m2);
            size_t xa = 8 * i + 2 * j, xb = xa + 1;
            acc_lo = fma_i32(acc_lo,
                             CAT(dot_u8_i8, SUF)(lo, _mm256_loadu_si256((const __m256i *)(x + 64 * j))),
                             d * (float)s1 * xd[xa]);
            acc_hi = fma_i32(acc_hi,
                             CAT(dot_u8_i8, SUF)(hi, _mm256_loadu_si256((const __m256i *)(x + 64 * j + 32))),
                             d * (float)s2 * xd[xb]);
            mins += dmin * ((float)m1 * xs[xa] + (float)m2 * xs[xb]);
        }
    }
    return hsum(_mm256_add_ps(acc_lo, acc_hi)) - mins;
}

static TGT float CAT(dot_q6k, SUF)(const uint8_t *w, const int8_t *xq, const float *xd, size_t nb32)
{
    size_t nsb = nb32 / 8;
    const __m256i m4 = _mm256_set1_epi8(0x0F), m3 = _mm256_set1_epi8(0x03), s32 = _mm256_set1_epi8(32);
    __m256 acc[2] = {_mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t i = 0; i < nsb; i++) {
        const uint8_t *b = w + 210 * i;
        float d = f16x(b + 208);
        const int8_t *x = xq + 256 * i;
        for (int n = 0; n < 2; n++) {
            __m256i ql0 = _mm256_loadu_si256((const __m256i *)(b + 64 * n));
            __m256i ql1 = _mm256_loadu_si256((const __m256i *)(b + 64 * n + 32));
            __m256i qh = _mm256_loadu_si256((const __m256i *)(b + 128 + 32 * n));
            const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
            /* 6-bit values 0..63; the -32 offset comes from the s32 product */
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(ql0, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m3), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(ql1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m3), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m3), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m3), 4));
            for (int k = 0; k < 4; k++) {
                __m256i xv = _mm256_loadu_si256((const __m256i *)(x + 128 * n + 32 * k));
                __m256i p = _mm256_sub_epi16(_mm256_maddubs_epi16(q[k], xv), _mm256_maddubs_epi16(s32, xv));
                __m256i scl = _mm256_set_m128i(_mm_set1_epi16((int16_t)sc[2 * k + 1]),
                                               _mm_set1_epi16((int16_t)sc[2 * k]));
                acc[k & 1] = fma_i32(acc[k & 1], _mm256_madd_epi16(p, scl), d * xd[8 * i + 4 * n + k]);
            }
        }
    }
    return hsum(_mm256_add_ps(acc[0], acc[1]));
}

#undef CAT
#undef CAT_
