"""How far from the reference's output would a gate/up kernel land that sums
each row's block dots in an order of its own (as a matrix-core kernel with
whole-block int8 dots would)?  CPU only, with the oracle: the layer is run
once in the x86 order everywhere and once with dense_ffn's gate/up matmuls at
the scalar level (block dots scaled and summed block by block), the rest
unchanged.  The intermediate is quantised again before down, and a value
that lands on the other side of a rounding boundary moves a quant by one
step: the printed max|d|/RMS is what that costs at the configs' sizes.

    python tests/error_budget.py        (about a minute on 8 cores)

Measured (this script, gcc -O2 oracle): Q8_0 T=512 Zipf 9.3e-4 / 2.2e-3 /
4.7e-3 (seeds 1-3); Q4_K/Q6_K T=2048 6.7e-3 / 4.4e-3 (seeds 4-5): beyond the
1e-3 * RMS bar, so gate/up keeps the x86 order (the word-dot kernels)."""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "oracle"))

import numpy as np  # noqa: E402

import oracle as orc  # noqa: E402
from biv_amd import synth  # noqa: E402


def budget(layer, h, label):
    ref = orc.moe(layer, h, threads=8)
    orc.set_gu_level(orc.SCALAR)
    try:
        alt = orc.moe(layer, h, threads=8)
    finally:
        orc.set_gu_level(-1)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    d = np.abs(ref.astype(np.float64) - alt)
    print(f"{label}: max|d|/RMS = {d.max() / rms:.2e}, 99.99th percentile {np.quantile(d, 0.9999) / rms:.2e}",
          flush=True)
    return d.max() / rms


if __name__ == "__main__":
    if not os.path.exists(orc.LIB_PATH):
        orc.build()
    for seed in (1, 2, 3):
        layer = synth.make_layer(seed)
        budget(layer, synth.zipf_bias_tokens(layer, 100 + seed, 512), f"Q8_0 T=512 Zipf, seed {seed}")
    for seed in (4, 5):
        layer = synth.make_layer(seed, types=(synth.Q4K, synth.Q4K, synth.Q6K))
        budget(layer, synth.make_tokens(200 + seed, 2048), f"Q4_K/Q6_K T=2048, seed {seed}")
