"""The GPU's exp (biv_amd/csrc/expf_ref.h) against the host's glibc expf,
which is what the reference's f32::exp calls on x86-64 Linux.  The header is
plain C; here gcc compiles it into a checker that sweeps the f32 inputs of
(-103, 88) with a stride (every input with stride 1: 2 of 2.2e9 differ, by
one ulp).  The GPU evaluates the same double-precision operations, so the
bits it gets are these."""
import os
import subprocess
import tempfile

from conftest import ROOT

SRC = r'''
#include <math.h>
#include <stdio.h>
#include <string.h>
#include "expf_ref.h"
int main(int argc, char **argv) {
    unsigned stride = 97; long n = 0, bad = 0, sel_bad = 0;
    for (unsigned long long u = 0; u < 0x100000000ull; u += stride) {
        unsigned b = (unsigned)u; float x; memcpy(&x, &b, 4);
        if (!(x > -103.0f && x < 88.0f)) continue;
        float g = expf(x), m = biv_expf_ref(x); n++;
        if (memcmp(&g, &m, 4)) bad++;
        /* the branch-free finish gives the same bits */
        double r; uint64_t ki; uint32_t ti = biv_expf_reduce(x, &r, &ki);
        static const uint64_t tab[32] = BIV_EXPF_TAB_INIT;
        float s = biv_expf_finish_sel(x, r, ki, tab[ti]);
        if (memcmp(&s, &m, 4)) sel_bad++;
    }
    /* the special ranges */
    float sp[] = {-INFINITY, INFINITY, -104.0f, 89.0f, 0.0f, -0.0f};
    for (int i = 0; i < 6; i++) {
        float g = expf(sp[i]), m = biv_expf_ref(sp[i]); if (memcmp(&g, &m, 4)) bad++;
        double r; uint64_t ki; uint32_t ti = biv_expf_reduce(sp[i], &r, &ki);
        static const uint64_t tab[32] = BIV_EXPF_TAB_INIT;
        float s = biv_expf_finish_sel(sp[i], r, ki, tab[ti]);
        if (memcmp(&s, &m, 4)) sel_bad++;
    }
    { float q = __builtin_nanf(""); double r; uint64_t ki; uint32_t ti = biv_expf_reduce(q, &r, &ki);
      static const uint64_t tab[32] = BIV_EXPF_TAB_INIT;
      float s = biv_expf_finish_sel(q, r, ki, tab[ti]); if (s == s) sel_bad++; }
    printf("%ld %ld %ld\n", n, bad, sel_bad);
    return 0;
}
'''


def test_expf_ref_matches_glibc():
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        exe = os.path.join(d, "t")
        open(c, "w").write(SRC)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "biv_amd", "csrc"), c, "-o", exe,
                        "-lm"], check=True)
        n, bad, sel_bad = map(int, subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split())
    assert n > 20_000_000
    assert bad <= 1, f"{bad} of {n} inputs differ from glibc"
    assert sel_bad == 0, f"{sel_bad} inputs where the branch-free finish differs"
