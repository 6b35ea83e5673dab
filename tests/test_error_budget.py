"""Error budgets that pin two design decisions of the prefill kernels (CPU only).

1. The exact gate/up keeps the x86 chain order.  A gate/up that sums each
   row's scaled block dots in an order of its own (what a matrix-core kernel
   with whole-block int8 dots would do) is modelled by the oracle's scalar
   level for dense_ffn's gate/up matmuls (quant.rs:599-607 instead of the x86
   chains of 1368-1382).  The intermediate is quantised again before down, and
   a value that lands on the other side of a rounding boundary moves a quant
   by one step: at the Q8_0 T = 512 Zipf config this alone moves the layer's
   output past the north star's bar of 1e-3 * RMS.

2. The BF16 grouped GEMM multiplies the weights by both bf16 halves of the
   f32 activations (hi = bf16(x), lo = bf16(x - hi)).  Dropping the lo half of
   gate/up's input (h) or of down's input (the SwiGLU intermediate) would halve
   that launch's matrix-core work; the test measures what it costs at the
   BF16 config's T = 4096 in a float64 model of the layer (the routing shared
   by both variants, the sums' order immaterial at this scale), and asserts
   that each is above 3e-4 * RMS, the margin a kernel may take out of the
   1e-3 bar and leave room for rounding: so both halves stay.
"""
import numpy as np
import pytest

from biv_amd import synth

BAR = 1e-3


def test_q8_gate_up_needs_the_x86_order(orc):
    layer = synth.make_layer(3)
    h = synth.zipf_bias_tokens(layer, 103, 512)
    ref = orc.moe(layer, h, threads=8)
    orc.set_gu_level(orc.SCALAR)
    try:
        alt = orc.moe(layer, h, threads=8)
    finally:
        orc.set_gu_level(-1)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    rel = float(np.abs(ref.astype(np.float64) - alt).max()) / rms
    print(f"Q8_0 T=512 Zipf, gate/up in the scalar order: max|d|/RMS = {rel:.2e}")
    assert rel > BAR


def _bf16_mats(ex, e):
    u = ex.expert(e).view(np.uint16).astype(np.uint32) << 16
    return u.view(np.float32).reshape(ex.rows, ex.cols).astype(np.float64)


def _bf16_round(x):
    """x (f32) rounded to the nearest bf16, ties to even, as f64."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def _silu(x):
    return x / (1.0 + np.exp(-x))


@pytest.mark.parametrize("seed", [41])
def test_bf16_lo_halves_are_needed(seed):
    T = 4096
    types = (synth.BF16, synth.BF16, synth.BF16)
    layer = synth.make_layer(seed, types=types)
    h32 = synth.make_tokens(500 + seed, T)
    h = h32.astype(np.float64)
    hh = _bf16_round(h32)
    E, ne, k = layer.n_embd, layer.n_expert, layer.k
    R = layer.router.data.view(np.float32).reshape(ne, E).astype(np.float64)
    logits = h @ R.T
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, 1)
    w /= np.maximum(w.sum(1, keepdims=True), 1.0 / 16384)

    # y[variant]: 0 exact, 1 gate/up on bf16(h), 2 down on bf16(intermediate)
    out = np.zeros((3, T, E))

    def ffn(G, U, D, rows, coef):
        g, u = h[rows] @ G.T, h[rows] @ U.T
        gh, uh = hh[rows] @ G.T, hh[rows] @ U.T
        a = (_silu(g) * u).astype(np.float32)  # the f32 intermediate
        ah = (_silu(gh) * uh).astype(np.float32)
        out[0, rows] += coef * (a.astype(np.float64) @ D.T)
        out[1, rows] += coef * (ah.astype(np.float64) @ D.T)
        out[2, rows] += coef * (_bf16_round(a) @ D.T)

    for e in range(ne):
        tok, slot = np.nonzero(ids == e)
        if tok.size:
            ffn(_bf16_mats(layer.gate, e), _bf16_mats(layer.up, e), _bf16_mats(layer.down, e), tok,
                w[tok, slot][:, None])
    sg, su, sd, gi = layer.shared
    mats = [(x.data.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(x.rows, x.cols)
            .astype(np.float64) for x in (sg, su, sd)]
    gate = 1.0 / (1.0 + np.exp(-(h @ gi.data.view(np.float32).astype(np.float64))))
    ffn(*mats, np.arange(T), gate[:, None])

    rms = float(np.sqrt(np.mean(out[0] ** 2)))
    gu = float(np.abs(out[1] - out[0]).max()) / rms
    dn = float(np.abs(out[2] - out[0]).max()) / rms
    print(f"BF16 T={T}: gate/up without lo {gu:.2e} * RMS, down without lo {dn:.2e} * RMS")
    assert gu > 3e-4 and dn > 3e-4
