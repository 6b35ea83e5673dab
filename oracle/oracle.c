/* CPU oracle for the qwen35moe MoE FFN block of biv.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in C, the arithmetic of biv's
 * Rust CPU path so that the HIP backend can be checked against it and so that
 * bench.py can time the reference algorithm on the host cores.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library never links or calls it.
 *
 * Restated functions (reference file:line, all under engine/src/):
 *   orc_f16_to_f32          quant.rs:114-131   branch-free f16 decode
 *   scale_min_k4            quant.rs:143-153
 *   orc_dequantize_row      quant.rs:156-349   (F32, F16, BF16, Q8_0, Q4_K, Q6_K)
 *   orc_q8act_quantize      quant.rs:368-394   Q8Act::quantize_into
 *   scalar dots             quant.rs:561-687   scalar::dot_q8_0 / dot_q4k / dot_q6k
 *   x86 dots                quant.rs:1043-1545 (x86_kernels.h for the int8 ones)
 *   orc_dot                 quant.rs:413-433   dispatch by type
 *   orc_axpy                quant.rs:470-481, 1209-1226
 *   orc_matmul              ops.rs:84-127      row-chunked, one thread per row
 *   orc_softmax             ops.rs:192-201
 *   sigmoid / silu          ops.rs:159-167
 *   orc_rms_norm            ops.rs:136-144
 *   orc_route               model.rs:256-268
 *   orc_dense_ffn           model.rs:1118-1126
 *   orc_moe                 model.rs:860-898
 *
 * Parity pins (tests/test_oracle.py): the reference's own inline tests
 * (quant.rs:1563-1738, model.rs:1461-1474) restated with their seeds and
 * tolerances, plus brute-force integer block dots, closed forms for the
 * quantiser and route, and float64 dequantise-then-dot for each kernel.
 *
 * Build: oracle/Makefile (gcc, no fast-math, -ffp-contract=off so that no
 * multiply-add is fused unless the reference fuses it with an intrinsic).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <cpuid.h>
#include <immintrin.h>
#include <omp.h>

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4K = 12, T_Q6K = 14, T_BF16 = 30 };
enum { L_SCALAR = 0, L_AVX2 = 1, L_VNNI = 2 };

#define TGT_AVX2 __attribute__((target("avx2,fma,f16c")))
#define TGT_VNNI __attribute__((target("avx2,fma,f16c,avxvnni")))

/* ------------------------------------------------------------------------- */
/* types                                                                      */

/* (elements per block, bytes per block), quant.rs:50-68 */
static int type_block(int ty, size_t *be, size_t *bb)
{
    switch (ty) {
    case T_F32: *be = 1; *bb = 4; return 0;
    case T_F16: case T_BF16: *be = 1; *bb = 2; return 0;
    case T_Q8_0: *be = 32; *bb = 34; return 0;
    case T_Q4K: *be = 256; *bb = 144; return 0;
    case T_Q6K: *be = 256; *bb = 210; return 0;
    default: return -1;
    }
}

size_t orc_row_size(int ty, size_t n)
{
    size_t be, bb;
    if (type_block(ty, &be, &bb)) return 0;
    return n / be * bb;
}

static int uses_f32_act(int ty) { return ty == T_F32 || ty == T_F16 || ty == T_BF16; }

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                         */

static inline float f32_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* quant.rs:114-131: exponent rebias by a multiply, denormals via a magic add */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t w = (uint32_t)h << 16;
    uint32_t sign = w & 0x80000000u;
    uint32_t two_w = w + w;
    float normalized = f32_bits((two_w >> 4) + (0xE0u << 23)) * f32_bits(0x07800000u);
    float denormalized = f32_bits((two_w >> 17) | (126u << 23)) - 0.5f;
    uint32_t b = two_w < (1u << 27) ? bits_f32(denormalized) : bits_f32(normalized);
    return f32_bits(sign | b);
}

float orc_bf16_to_f32(uint16_t h) { return f32_bits((uint32_t)h << 16); }

/* quant.rs:143-153: the 6-bit scale and min of sub-block j of a k4 super-block */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------- */
/* dequantisation, quant.rs:156-349                                           */

int orc_dequantize_row(int ty, const uint8_t *src, float *dst, size_t n)
{
    switch (ty) {
    case T_F32:
        memcpy(dst, src, 4 * n);
        return 0;
    case T_F16:
        for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(rd16(src + 2 * i));
        return 0;
    case T_BF16:
        for (size_t i = 0; i < n; i++) dst[i] = orc_bf16_to_f32(rd16(src + 2 * i));
        return 0;
    case T_Q8_0:
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = src + 34 * b;
            float d = orc_f16_to_f32(rd16(blk));
            for (int j = 0; j < 32; j++) dst[32 * b + j] = (float)(int8_t)blk[2 + j] * d;
        }
        return 0;
    case T_Q4K:
        for (size_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = src + 144 * b;
            float *y = dst + 256 * b;
            float d = orc_f16_to_f32(rd16(blk)), min = orc_f16_to_f32(rd16(blk + 2));
            const uint8_t *scales = blk + 4, *qs = blk + 16;
            for (int j = 0; j < 4; j++) {
                uint8_t s1, m1, s2, m2;
                scale_min_k4(2 * j, scales, &s1, &m1);
                scale_min_k4(2 * j + 1, scales, &s2, &m2);
                float d1 = d * (float)s1, mm1 = min * (float)m1;
                float d2 = d * (float)s2, mm2 = min * (float)m2;
                const uint8_t *q = qs + 32 * j;
                for (int l = 0; l < 32; l++) {
                    y[64 * j + l] = d1 * (float)(q[l] & 0xF) - mm1;
                    y[64 * j + 32 + l] = d2 * (float)(q[l] >> 4) - mm2;
                }
            }
        }
        return 0;
    case T_Q6K:
        for (size_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = src + 210 * b;
            float d = orc_f16_to_f32(rd16(blk + 208));
            for (int h = 0; h < 2; h++) {
                const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h, *sc = blk + 192 + 8 * h;
                float *y = dst + 256 * b + 128 * h;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * (float)(int8_t)sc[is] * (float)q1;
                    y[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
                }
            }
        }
        return 0;
    default:
        return -1;
    }
}

/* ------------------------------------------------------------------------- */
/* Q8 activations, quant.rs:368-394                                           */

void orc_q8act_quantize(const float *x, size_t n, int8_t *qs, float *d, float *s)
{
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        float db = amax / 127.0f;
        float id = db != 0.0f ? 1.0f / db : 0.0f;
        int32_t sum = 0;
        for (int j = 0; j < 32; j++) {
            int32_t r = (int32_t)roundf(xb[j] * id);
            qs[32 * b + j] = (int8_t)r;
            sum += r;
        }
        d[b] = db;
        s[b] = db * (float)sum;
    }
}

/* ------------------------------------------------------------------------- */
/* scalar reference dots, quant.rs:561-687                                    */

static int32_t idot(const int32_t *a, const int8_t *b, int n)
{
    int32_t s = 0;
    for (int i = 0; i < n; i++) s += a[i] * (int32_t)b[i];
    return s;
}

static float sc_dot_q8_0(const uint8_t *w, const int8_t *xq, const float *xd, size_t nb)
{
    float sum = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + 34 * i;
        float d = orc_f16_to_f32(rd16(b));
        int32_t q[32];
        for (int j = 0; j < 32; j++) q[j] = (int8_t)b[2 + j];
        sum += d * xd[i] * (float)idot(q, xq + 32 * i, 32);
    }
    return sum;
}

static void q4k_sub(const uint8_t *b, int sb, int32_t *q)
{
    const uint8_t *q4 = b + 16 + 32 * (sb / 2);
    for (int l = 0; l < 32; l++) q[l] = (q4[l] >> (4 * (sb % 2))) & 0xF;
}

static float sc_dot_q4k(const uint8_t *w, const int8_t *xq, const float *xd, const float *xs, size_t nb32)
{
    float sum = 0.0f;
    for (size_t i = 0; i < nb32 / 8; i++) {
        const uint8_t *b = w + 144 * i;
        float d = orc_f16_to_f32(rd16(b)), min = orc_f16_to_f32(rd16(b + 2));
        for (int sb = 0; sb < 8; sb++) {
            uint8_t sc, m;
            scale_min_k4(sb, b + 4, &sc, &m);
            int32_t q[32];
            q4k_sub(b, sb, q);
            size_t xb = 8 * i + sb;
            sum += d * (float)sc * xd[xb] * (float)idot(q, xq + 32 * xb, 32) - min * (float)m * xs[xb];
        }
    }
    return sum;
}

/* the 256 signed 6-bit values and 16 sub-scales of a q6_K super-block */
static void q6k_unpack(const uint8_t *b, int32_t *q, int32_t *sc16)
{
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            q[128 * n + l] = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            q[128 * n + l + 32] = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            q[128 * n + l + 64] = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            q[128 * n + l + 96] = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            for (int k = 0; k < 4; k++) sc16[8 * n + is + 2 * k] = (int8_t)sc[is + 2 * k];
        }
    }
}

static float sc_dot_q6k(const uint8_t *w, const int8_t *xq, const float *xd, size_t nb32)
{
    float sum = 0.0f;
    for (size_t i = 0; i < nb32 / 8; i++) {
        const uint8_t *b = w + 210 * i;
        float d = orc_f16_to_f32(rd16(b + 208));
        int32_t q[256], sc16[16];
        q6k_unpack(b, q, sc16);
        for (int xb = 0; xb < 8; xb++) {
            int32_t isum = 0;
            for (int half = 0; half < 2; half++) {
                int g = 2 * xb + half, off = 16 * g;
                isum += sc16[g] * idot(q + off, xq + 256 * i + off, 16);
            }
            sum += d * xd[8 * i + xb] * (float)isum;
        }
    }
    return sum;
}

/* The integer of each 32-element activation block, before any float scale:
 *   Q8_0: sum w*x;  Q4_K: sum q4*x (nibble 0..15);  Q6_K: sc[2b]*dot16 + sc[2b+1]*dot16
 * These are the per-block int32 dots of quant.rs:599-607, 609-627, 651-686. */
int orc_block_idots(int ty, const uint8_t *w, const int8_t *xq, size_t nb32, int32_t *out)
{
    int32_t q[256], sc16[16];
    switch (ty) {
    case T_Q8_0:
        for (size_t i = 0; i < nb32; i++) {
            for (int j = 0; j < 32; j++) q[j] = (int8_t)w[34 * i + 2 + j];
            out[i] = idot(q, xq + 32 * i, 32);
        }
        return 0;
    case T_Q4K:
        for (size_t i = 0; i < nb32; i++) {
            q4k_sub(w + 144 * (i / 8), (int)(i % 8), q);
            out[i] = idot(q, xq + 32 * i, 32);
        }
        return 0;
    case T_Q6K:
        for (size_t i = 0; i < nb32 / 8; i++) {
            q6k_unpack(w + 210 * i, q, sc16);
            for (int xb = 0; xb < 8; xb++) {
                int32_t isum = 0;
                for (int half = 0; half < 2; half++) {
                    int g = 2 * xb + half, off = 16 * g;
                    isum += sc16[g] * idot(q + off, xq + 256 * i + off, 16);
                }
                out[8 * i + xb] = isum;
            }
        }
        return 0;
    default:
        return -1;
    }
}

/* orc_block_idots for n_rows consecutive weight rows against one activation
 * row: out is [n_rows][nb32]. */
int orc_block_idots_rows(int ty, const uint8_t *w, size_t n_rows, const int8_t *xq, size_t nb32, int32_t *out)
{
    size_t rb = orc_row_size(ty, nb32 * 32);
    for (size_t r = 0; r < n_rows; r++)
        if (orc_block_idots(ty, w + r * rb, xq, nb32, out + r * nb32)) return -1;
    return 0;
}

/* ------------------------------------------------------------------------- */
/* x86 kernels, quant.rs:1043-1545                                            */

static inline TGT_AVX2 float f16x(const uint8_t *p)
{
    uint16_t h;
    memcpy(&h, p, 2);
    return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h)));
}

/* quant.rs:1149-1153 */
static inline TGT_AVX2 float hsum(__m256 v)
{
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    return _mm_cvtss_f32(_mm_add_ss(s, _mm_movehdup_ps(s)));
}

static inline TGT_AVX2 __m256 fma_i32(__m256 acc, __m256i p, float d)
{
    return _mm256_fmadd_ps(_mm256_cvtepi32_ps(p), _mm256_set1_ps(d), acc);
}

/* quant.rs:1177-1207: four 8-lane accumulators over 32-element steps */
static TGT_AVX2 float x86_dot_f32(const float *a, const float *b, size_t n)
{
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int k = 0; k < 4; k++)
            acc[k] = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8 * k), _mm256_loadu_ps(b + i + 8 * k), acc[k]);
    for (; i + 8 <= n; i += 8) acc[0] = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc[0]);
    float s = hsum(_mm256_add_ps(_mm256_add_ps(acc[0], acc[1]), _mm256_add_ps(acc[2], acc[3])));
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* quant.rs:1209-1226 */
static TGT_AVX2 void x86_axpy(float *y, float a, const float *x, size_t n)
{
    __m256 va = _mm256_set1_ps(a);
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(y + i, _mm256_fmadd_ps(va, _mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i)));
    for (; i < n; i++) y[i] += a * x[i];
}

static inline TGT_AVX2 __m256 bf16_widen(const uint16_t *p)
{
    return _mm256_castsi256_ps(
        _mm256_slli_epi32(_mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)p)), 16));
}

/* quant.rs:1228-1256: two 8-lane accumulators over 16-element steps */
static TGT_AVX2 float x86_dot_bf16(const uint8_t *wb, const float *x, size_t n)
{
    const uint16_t *w = (const uint16_t *)wb;
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 16 <= n; i += 16) {
        acc0 = _mm256_fmadd_ps(bf16_widen(w + i), _mm256_loadu_ps(x + i), acc0);
        acc1 = _mm256_fmadd_ps(bf16_widen(w + i + 8), _mm256_loadu_ps(x + i + 8), acc1);
    }
    if (i + 8 <= n) {
        acc0 = _mm256_fmadd_ps(bf16_widen(w + i), _mm256_loadu_ps(x + i), acc0);
        i += 8;
    }
    float s = hsum(_mm256_add_ps(acc0, acc1));
    for (; i < n; i++) s += orc_bf16_to_f32(rd16(wb + 2 * i)) * x[i];
    return s;
}

#define SUF avx2
#define TGT TGT_AVX2
#define DOT_U8_I8(u, s) _mm256_madd_epi16(_mm256_maddubs_epi16(u, s), _mm256_set1_epi16(1))
#include "x86_kernels.h"
#undef SUF
#undef TGT
#undef DOT_U8_I8

#define SUF vnni
#define TGT TGT_VNNI
#define DOT_U8_I8(u, s) _mm256_dpbusd_avx_epi32(_mm256_setzero_si256(), u, s)
#include "x86_kernels.h"
#undef SUF
#undef TGT
#undef DOT_U8_I8

/* quant.rs:1100-1123: AVX2+FMA+F16C with OS-saved ymm state, then AVX-VNNI */
int orc_detect_level(void)
{
    unsigned a, b, c, d;
    if (!__get_cpuid(1, &a, &b, &c, &d)) return L_SCALAR;
    int fma = (c >> 12) & 1, osxsave = (c >> 27) & 1, avx = (c >> 28) & 1, f16c = (c >> 29) & 1;
    if (!(fma && osxsave && avx && f16c) || __get_cpuid_max(0, 0) < 7) return L_SCALAR;
    unsigned lo, hi;
    __asm__ volatile("xgetbv" : "=a"(lo), "=d"(hi) : "c"(0));
    if ((lo & 6) != 6) return L_SCALAR;
    __cpuid_count(7, 0, a, b, c, d);
    if (!((b >> 5) & 1)) return L_SCALAR;
    __cpuid_count(7, 1, a, b, c, d);
    return ((a >> 4) & 1) ? L_VNNI : L_AVX2;
}

/* detection runs cpuid, which is slow under a hypervisor: cache it, as the
 * reference does (quant.rs:1059-1083) */
static int detected_level = -1;

static int resolve(int level)
{
    int best = detected_level;
    if (best < 0) best = detected_level = orc_detect_level();
    if (level < 0 || level > best) return best;
    return level;
}

/* ------------------------------------------------------------------------- */
/* dispatch, quant.rs:413-433, 459-481                                        */

float orc_dot_f32(const float *a, const float *b, size_t n, int level)
{
    if (resolve(level) >= L_AVX2) return x86_dot_f32(a, b, n);
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

void orc_axpy(float *y, float a, const float *x, size_t n, int level)
{
    if (resolve(level) >= L_AVX2) {
        x86_axpy(y, a, x, n);
        return;
    }
    for (size_t i = 0; i < n; i++) y[i] += a * x[i];
}

/* One weight row against one activation row: xf for F32/F16/BF16 rows,
 * (xq, xd, xs) for quantised rows.  Returns NAN for an unsupported type. */
float orc_dot(int ty, const uint8_t *w, const float *xf, const int8_t *xq, const float *xd, const float *xs,
              size_t n, int level)
{
    int lv = resolve(level);
    switch (ty) {
    case T_F32:
        return orc_dot_f32((const float *)w, xf, n, lv);
    case T_F16: {
        float s = 0.0f; /* only the scalar form: F16 weights are not on the MoE path */
        for (size_t i = 0; i < n; i++) s += orc_f16_to_f32(rd16(w + 2 * i)) * xf[i];
        return s;
    }
    case T_BF16:
        if (lv >= L_AVX2) return x86_dot_bf16(w, xf, n);
        {
            float s = 0.0f;
            for (size_t i = 0; i < n; i++) s += orc_bf16_to_f32(rd16(w + 2 * i)) * xf[i];
            return s;
        }
    case T_Q8_0:
        return lv == L_VNNI ? dot_q8_0_vnni(w, xq, xd, n / 32)
             : lv == L_AVX2 ? dot_q8_0_avx2(w, xq, xd, n / 32)
                            : sc_dot_q8_0(w, xq, xd, n / 32);
    case T_Q4K:
        return lv == L_VNNI ? dot_q4k_vnni(w, xq, xd, xs, n / 32)
             : lv == L_AVX2 ? dot_q4k_avx2(w, xq, xd, xs, n / 32)
                            : sc_dot_q4k(w, xq, xd, xs, n / 32);
    case T_Q6K:
        return lv == L_VNNI ? dot_q6k_vnni(w, xq, xd, n / 32)
             : lv == L_AVX2 ? dot_q6k_avx2(w, xq, xd, n / 32)
                            : sc_dot_q6k(w, xq, xd, n / 32);
    default:
        return NAN;
    }
}

/* ------------------------------------------------------------------------- */
/* matmul, ops.rs:84-127                                                      */

/* out[t*rows + r] = dot(row r, x[t]) for n input rows of `cols`.  Rows are cut
 * into chunks of clamp(rows / (threads*8), 1, 256) and each row is computed
 * whole by one thread, so the result does not depend on the thread count. */
int orc_matmul(int ty, const uint8_t *w, size_t cols, size_t rows, const float *x, size_t n, float *out,
               int threads, int level)
{
    size_t be, bb;
    if (type_block(ty, &be, &bb) || cols % be) return -1;
    size_t row_bytes = orc_row_size(ty, cols);
    int lv = resolve(level);
    if (threads < 1) threads = 1;
    int8_t *qs = NULL;
    float *qd = NULL, *qsum = NULL;
    if (!uses_f32_act(ty)) {
        if (cols % 32) return -1;
        qs = malloc(n * cols);
        qd = malloc(sizeof(float) * n * cols / 32);
        qsum = malloc(sizeof(float) * n * cols / 32);
        if (!qs || !qd || !qsum) { free(qs); free(qd); free(qsum); return -2; }
        /* Input::q8 (ops.rs:63-76): every row quantised, rows block-aligned */
        orc_q8act_quantize(x, n * cols, qs, qd, qsum);
    }
    size_t chunk = rows / ((size_t)threads * 8);
    if (chunk < 1) chunk = 1;
    if (chunk > 256) chunk = 256;
    long n_chunks = (long)((rows + chunk - 1) / chunk);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (long c = 0; c < n_chunks; c++) {
        size_t r0 = (size_t)c * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
        for (size_t r = r0; r < r1; r++)
            for (size_t t = 0; t < n; t++)
                out[t * rows + r] = orc_dot(ty, w + r * row_bytes, x + t * cols, qs ? qs + t * cols : NULL,
                                            qd ? qd + t * cols / 32 : NULL, qsum ? qsum + t * cols / 32 : NULL,
                                            cols, lv);
    }
    free(qs);
    free(qd);
    free(qsum);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* element-wise ops, ops.rs:136-201                                           */

float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float orc_silu(float x) { return x * orc_sigmoid(x); }

void orc_softmax(float *x, size_t n)
{
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

void orc_rms_norm(float *x, const float *w, size_t rows, size_t n, float eps, int level)
{
    for (size_t r = 0; r < rows; r++) {
        float *g = x + r * n;
        float ss = orc_dot_f32(g, g, n, level) / (float)n;
        float scale = 1.0f / sqrtf(ss + eps);
        for (size_t i = 0; i < n; i++) g[i] *= scale * w[i];
    }
}

/* The integer whose signed order is f32::total_cmp's order of x. */
static int32_t total_key(float x)
{
    int32_t b;
    memcpy(&b, &x, sizeof b);
    return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

/* model.rs:256-268: softmax, then the k highest probabilities (the lower
 * index first among equals), weighted by p / max(sum of the k, 1/16384). */
void orc_route(const float *logits, size_t ne, size_t k, int32_t *ids, float *w)
{
    float *p = malloc(sizeof(float) * ne);
    unsigned char *taken = calloc(ne, 1);
    memcpy(p, logits, sizeof(float) * ne);
    orc_softmax(p, ne);
    /* selection by repeated maximum is the first k of the stable sort; the
     * comparison is f32::total_cmp's (model.rs:264): the bits as a signed
     * magnitude, so +NaN ranks above +inf and -NaN below -inf */
    for (size_t j = 0; j < k; j++) {
        size_t best = ne;
        for (size_t i = 0; i < ne; i++) {
            if (taken[i]) continue;
            if (best == ne || total_key(p[i]) > total_key(p[best])) best = i;
        }
        taken[best] = 1;
        ids[j] = (int32_t)best;
    }
    float sum = 0.0f;
    for (size_t j = 0; j < k; j++) sum += p[ids[j]];
    sum = fmaxf(sum, 1.0f / 16384.0f);
    for (size_t j = 0; j < k; j++) w[j] = p[ids[j]] / sum;
    free(p);
    free(taken);
}

/* ------------------------------------------------------------------------- */
/* feed-forwards, model.rs:860-898 and 1118-1126                             */

typedef struct {
    int32_t ty;
    int32_t pad;
    const uint8_t *data;
    uint64_t stride; /* bytes from one expert's matrix to the next */
    uint64_t offset; /* bytes from an expert's matrix to these rows */
} OrcExperts;

typedef struct {
    int32_t ty;
    int32_t pad;
    const uint8_t *data;
} OrcWeight;

typedef struct {
    int32_t n_expert, k, n_embd, n_ff, n_ff_sh, pad;
    OrcWeight router;                 /* [n_expert x n_embd] */
    OrcExperts gate, up, down;        /* [n_ff x n_embd], [n_ff x n_embd], [n_embd x n_ff] */
    OrcWeight sh_gate, sh_up, sh_down, gate_inp; /* when n_ff_sh > 0 */
} OrcMoe;

/* Kernel level for the gate and up matmuls of dense_ffn, -1 (default) for the
 * caller's.  Test-only knob: the scalar level sums each row's block dots in a
 * different order from the x86 kernels, which measures how far a GPU kernel
 * summing in its own order would land from the reference's output. */
static int gu_level = -1;
void orc_set_gu_level(int level) { gu_level = level; }

/* down(silu(gate x) * up x) of n rows; out is [n x e] */
int orc_dense_ffn(int gty, const uint8_t *gate, int uty, const uint8_t *up, int dty, const uint8_t *down,
                  size_t e, size_t ff, const float *x, size_t n, float *out, int threads, int level)
{
    float *g = malloc(sizeof(float) * n * ff), *u = malloc(sizeof(float) * n * ff);
    int rc = -2;
    if (g && u) {
        const int gl = gu_level >= 0 ? gu_level : level;
        rc = orc_matmul(gty, gate, e, ff, x, n, g, threads, gl);
        if (!rc) rc = orc_matmul(uty, up, e, ff, x, n, u, threads, gl);
        if (!rc) {
            for (size_t i = 0; i < n * ff; i++) g[i] = orc_silu(g[i]) * u[i];
            rc = orc_matmul(dty, down, ff, e, g, n, out, threads, level);
        }
    }
    free(g);
    free(u);
    return rc;
}

/* The MoE block of n tokens h [n x e] into out [n x e] (not added to x).
 * Optional taps: ids/weights [n x k], logits [n x n_expert]. */
int orc_moe(const OrcMoe *m, const float *h, size_t n, float *out, int threads, int level, int32_t *ids_out,
            float *w_out, float *logits_out)
{
    size_t e = (size_t)m->n_embd, ne = (size_t)m->n_expert, k = (size_t)m->k, ff = (size_t)m->n_ff;
    int lv = resolve(level);
    float *logits = malloc(sizeof(float) * n * ne);
    int32_t *ids = malloc(sizeof(int32_t) * n * k);
    float *wts = malloc(sizeof(float) * n * k);
    if (!logits || !ids || !wts) { free(logits); free(ids); free(wts); return -2; }
    int rc = orc_matmul(m->router.ty, m->router.data, e, ne, h, n, logits, threads, lv);
    for (size_t t = 0; t < n && !rc; t++) orc_route(logits + t * ne, ne, k, ids + t * k, wts + t * k);
    memset(out, 0, sizeof(float) * n * e);
    size_t grb = orc_row_size(m->gate.ty, e) * ff, urb = orc_row_size(m->up.ty, e) * ff;
    size_t drb = orc_row_size(m->down.ty, ff) * e;
    (void)grb; (void)urb; (void)drb;
    /* experts in ascending id, each over its tokens in ascending order */
    float *x = malloc(sizeof(float) * n * e), *y = malloc(sizeof(float) * n * e);
    size_t *tok = malloc(sizeof(size_t) * n);
    float *tw = malloc(sizeof(float) * n);
    if (!x || !y || !tok || !tw) rc = -2;
    for (size_t i = 0; i < ne && !rc; i++) {
        size_t cnt = 0;
        for (size_t t = 0; t < n; t++)
            for (size_t j = 0; j < k; j++)
                if ((size_t)ids[t * k + j] == i) {
                    tok[cnt] = t;
                    tw[cnt] = wts[t * k + j];
                    cnt++;
                }
        if (!cnt) continue;
        for (size_t c = 0; c < cnt; c++) memcpy(x + c * e, h + tok[c] * e, sizeof(float) * e);
        rc = orc_dense_ffn(m->gate.ty, m->gate.data + i * m->gate.stride + m->gate.offset, m->up.ty,
                           m->up.data + i * m->up.stride + m->up.offset, m->down.ty,
                           m->down.data + i * m->down.stride + m->down.offset, e, ff, x, cnt, y, threads, lv);
        for (size_t c = 0; c < cnt && !rc; c++) orc_axpy(out + tok[c] * e, tw[c], y + c * e, e, lv);
    }
    if (!rc && m->n_ff_sh > 0) {
        rc = orc_dense_ffn(m->sh_gate.ty, m->sh_gate.data, m->sh_up.ty, m->sh_up.data, m->sh_down.ty,
                           m->sh_down.data, e, (size_t)m->n_ff_sh, h, n, y, threads, lv);
        float *g = malloc(sizeof(float) * n);
        if (!g) rc = -2;
        if (!rc) rc = orc_matmul(m->gate_inp.ty, m->gate_inp.data, e, 1, h, n, g, threads, lv);
        for (size_t t = 0; t < n && !rc; t++) orc_axpy(out + t * e, orc_sigmoid(g[t]), y + t * e, e, lv);
        free(g);
    }
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * n * k);
    if (w_out) memcpy(w_out, wts, sizeof(float) * n * k);
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * n * ne);
    free(logits); free(ids); free(wts); free(x); free(y); free(tok); free(tw);
    return rc;
}

int orc_max_threads(void) { return omp_get_num_procs(); }
