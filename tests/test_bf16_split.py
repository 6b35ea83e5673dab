"""The bf16 hi / lo split of the BF16 matrix-core kernels
(biv_amd/csrc/bf16_split.h), compiled by gcc from the same header: ties to
even, non-finite inputs (lo = 0, so that w * hi + w * lo is w * x as the
reference's f32 product), values near FLT_MAX (finite halves), and the
2^-17 bound of x - hi - lo on a sweep of finite inputs."""
import os
import subprocess
import tempfile

from conftest import ROOT

SRC = r'''
#include <math.h>
#include <stdio.h>
#include <float.h>
#include "bf16_split.h"
static float b2f(uint32_t b) { return biv_bits_f32(b << 16); }
static int fails = 0;
#define CHECK(c, ...) do { if (!(c)) { fails++; printf(__VA_ARGS__); printf("\n"); } } while (0)
int main(void) {
    uint32_t h, l;
    /* ties to even: 1 + 2^-8 is halfway between bf16 1 and 1 + 2^-7 */
    CHECK(bf16_bits(1.0f + 0x1p-8f) == 0x3F80u, "tie down");
    CHECK(bf16_bits(1.0f + 3 * 0x1p-8f) == 0x3F82u, "tie up");
    /* infinities and NaN: lo = 0 */
    bf16_split(INFINITY, &h, &l); CHECK(h == 0x7F80u && l == 0, "+inf %x %x", h, l);
    bf16_split(-INFINITY, &h, &l); CHECK(h == 0xFF80u && l == 0, "-inf %x %x", h, l);
    bf16_split(NAN, &h, &l); CHECK((h & 0x7F80u) == 0x7F80u && (h & 0x7Fu) && l == 0, "nan %x %x", h, l);
    /* w * hi + w * lo = w * x for x = +-inf (w = 2) and NaN for w = 0 */
    bf16_split(INFINITY, &h, &l);
    CHECK(2.0f * b2f(h) + 2.0f * b2f(l) == INFINITY, "2 inf");
    CHECK(isnan(0.0f * b2f(h) + 0.0f * b2f(l)), "0 inf");
    /* finite x near FLT_MAX: finite halves summing to x within 2^-16 */
    float big[] = {FLT_MAX, -FLT_MAX, 0x1.fefp127f, 0x1.ff0p127f, 0x1.ffep127f, 0x1.fe8p127f};
    for (int i = 0; i < 6; i++) {
        bf16_split(big[i], &h, &l);
        float fh = b2f(h), fl = b2f(l);
        CHECK(isfinite(fh) && isfinite(fl), "big %a: %a %a", big[i], fh, fl);
        double r = (double)big[i] - (double)fh - (double)fl;
        CHECK(fabs(r) <= 0x1p-16 * fabs((double)big[i]), "big %a: rest %a", big[i], r);
        CHECK(isfinite(2.0f * fh + 2.0f * fl) || fabsf(big[i]) > FLT_MAX / 2, "big sum");
    }
    /* sweep: |x - hi - lo| <= 2^-17 |x| (subnormal x: exact) */
    long n = 0;
    for (uint64_t u = 0; u < 0x100000000ull; u += 7919) {
        float x = biv_bits_f32((uint32_t)u);
        if (!isfinite(x)) continue;
        bf16_split(x, &h, &l);
        double r = (double)x - (double)b2f(h) - (double)b2f(l);
        double bound = fmax(0x1p-17 * fabs((double)x), 0x1p-133);
        n++;
        if (fabs(r) > bound) { CHECK(0, "x %a hi %a lo %a rest %a", x, b2f(h), b2f(l), r); if (fails > 5) break; }
    }
    printf("%ld inputs, %d failures\n", n, fails);
    return fails != 0;
}
'''


def test_bf16_split():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.c"), os.path.join(d, "t")
        with open(src, "w") as f:
            f.write(SRC)
        subprocess.run(["gcc", "-O2", "-std=c99", "-ffp-contract=off", "-I", os.path.join(ROOT, "biv_amd", "csrc"),
                        src, "-o", exe, "-lm"], check=True)
        r = subprocess.run([exe], capture_output=True, text=True)
        print(r.stdout)
        assert r.returncode == 0, r.stdout
