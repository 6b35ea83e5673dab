"""The f32 matrix-core instructions the prefill router uses compute each
output as fmaf(a, b, c) (k = 1: one product, one rounding), bit for bit
against the host's fmaf on random triples with cancellation and subnormal
products, results and accumulators (tests/probes/mfma_fma.cpp, built with the
library).  The router's logits are bit-identical to the reference's
dot_f32 because of it."""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "probes", "mfma_fma")


def test_mfma_f32_k1_is_fmaf():
    if not os.path.exists(EXE):
        pytest.fail("tests/probes/mfma_fma is not built (python -m biv_amd.build)")
    print("case mfma f32 k=1 vs fmaf", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    lines = [l for l in r.stdout.splitlines() if "outputs differ" in l]
    assert len(lines) == 3, r.stdout + r.stderr
    for l in lines:
        assert l.split(":")[1].strip().startswith("0 of"), l
    assert r.returncode == 0, r.stdout + r.stderr
