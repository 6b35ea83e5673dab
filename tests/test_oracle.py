"""Pins of the CPU oracle (oracle/oracle.c).

1. biv's own inline tests, restated with their seeds, generators and
   tolerances: kernels_match_dequantized_dot and vnni_matches_avx2
   (engine/src/quant.rs:1563-1712), bf16_and_f16 (1714-1738) and
   route_picks_and_weighs (engine/src/model.rs:1461-1474).
2. Checks the mathematics fixes: integer block dots against float64 sums of
   the dequantised rows (a second, independent code path), round-half-away
   ties of the quantiser, softmax against float64, route on hand-made cases,
   thread-count invariance of matmul, and the MoE combine reducing to
   dense_ffn when one expert takes every token with weight 1.
"""
import numpy as np
import pytest

from refvectors import Seed, f32_sum_seq, rand_bytes, rand_row, ROW, ref_x

Q8_0, Q4K, Q6K, BF16, F32 = 8, 12, 14, 30, 0
TY = {"Q8_0": Q8_0, "Q4_K": Q4K, "Q6_K": Q6K}


def advance(seed, ty, n):
    be, bb = ROW[ty]
    rand_bytes(n // be * bb, seed)


def kernel_rows(seed0, n=1024, force_m128=False):
    """The rows the reference's kernel tests draw, keyed by type."""
    seed = Seed(seed0)
    rows = {}
    for ty in ("Q4_0", "Q4_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K"):
        if ty in TY:
            w = rand_row(ty, n, seed)
            if force_m128 and ty == "Q8_0":
                w[2] = 0x80  # -128, the weight the sign trick can't negate
            rows[ty] = w
        else:
            advance(seed, ty, n)
    return rows


# ---------------------------------------------------------------------------
# restated reference tests

@pytest.mark.parametrize("ty", ["Q8_0", "Q4_K", "Q6_K"])
def test_kernels_match_dequantized_dot(orc, ty):
    """quant.rs:1651-1712: every kernel within 1e-3*max(|ref|, 1) of the f32
    dot of dequantised weights and dequantised activations."""
    n = 1024
    w = kernel_rows(0x1234_5678_9abc_def1, n)[ty]
    x = ref_x(n)
    qs, d, s = orc.q8act(x)
    xd = (qs.astype(np.float32) * np.repeat(d, 32)).astype(np.float32)
    wd = orc.dequantize_row(TY[ty], w, n)
    ref = f32_sum_seq((wd * xd).astype(np.float32))
    tol = 1e-3 * max(abs(float(ref)), 1.0)
    for level in (orc.AUTO, orc.SCALAR, orc.AVX2, orc.VNNI):
        if level > orc.detect_level():
            continue
        got = orc.dot(TY[ty], w, x, level)
        assert abs(got - ref) < tol, (ty, level, got, ref)


@pytest.mark.parametrize("ty", ["Q8_0", "Q4_K", "Q6_K"])
def test_vnni_matches_avx2(orc, ty):
    """quant.rs:1563-1614: AVX-VNNI and AVX2 kernels agree bit for bit on
    full-range activations, with a -128 Q8_0 weight."""
    if orc.detect_level() < orc.VNNI:
        pytest.skip("no AVX-VNNI on this host")
    n = 1024
    x = ref_x(n)
    xs = []
    for t in range(4):
        v = np.where(np.arange(n) % 5 == t, np.float32(1e3) * np.copysign(np.float32(1), x),
                     x * np.float32(t - 1.5)).astype(np.float32)
        xs.append(v)
    w = kernel_rows(0x0bad_cafe_dead_beef, n, force_m128=True)[ty]
    for v in xs:
        qs, d, s = orc.q8act(v)
        a = np.float32(orc.dot_q(TY[ty], w, qs, d, s, orc.AVX2))
        b = np.float32(orc.dot_q(TY[ty], w, qs, d, s, orc.VNNI))
        assert a.view(np.uint32) == b.view(np.uint32), (ty, a, b)


def f32_to_f16_exact(v):
    """quant.rs:1741-1748"""
    if v == 0.0:
        return 0
    b = int(np.float32(v).view(np.uint32))
    exp = ((b >> 23) & 0xFF) - 127 + 15
    return ((b >> 16) & 0x8000) | (exp << 10) | ((b >> 13) & 0x3FF)


def test_bf16_and_f16(orc):
    """quant.rs:1714-1738"""
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f16_to_f32(0xC000) == -2.0
    assert orc.f16_to_f32(0x0001) == 5.960464477539063e-8
    assert orc.bf16_to_f32(0x3F80) == 1.0
    x = (np.arange(37, dtype=np.float32) * np.float32(0.25)).astype(np.float32)
    want = float(f32_sum_seq(x * x))
    wbf = (x.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    assert abs(orc.dot(BF16, wbf, x) - want) < 1e-3
    w16 = np.array([f32_to_f16_exact(v) for v in x], dtype=np.uint16).view(np.uint8)
    assert abs(orc.dot(1, w16, x) - want) < 1e-3
    assert abs(orc.dot(F32, x.view(np.uint8), x) - want) < 1e-3
    assert abs(orc.dot_f32(x, x) - want) < 1e-3
    y = orc.axpy(x, 2.0, x)
    assert np.array_equal(y, (np.float32(3) * x).astype(np.float32))


def test_route_picks_and_weighs(orc):
    """model.rs:1461-1474"""
    f = np.float32
    l = np.array([np.log(f(2)) + f(1), f(1), np.log(f(0.5)) + f(1), np.log(f(0.5)) + f(1)], dtype=np.float32)
    l = (l - f(1)).astype(np.float32)
    ids, w = orc.route(l, 3)
    assert list(ids) == [0, 1, 2]
    s = 0.5 + 0.25 + 0.125
    for wi, p in zip(w, [0.5, 0.25, 0.125]):
        assert abs(wi - p / s) < 1e-6
    ids, w = orc.route(l, 1)
    assert list(ids) == [0] and list(w) == [1.0]


# ---------------------------------------------------------------------------
# mathematics

def test_f16_decoder_matches_ieee(orc):
    """The branch-free decoder (quant.rs:114-131) against numpy's IEEE half
    for every finite f16, denormals and signed zero included."""
    h = np.arange(1 << 16, dtype=np.uint32)
    finite = (h & 0x7C00) != 0x7C00
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(v)) for v in h[finite][::7]], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want[finite][::7].view(np.uint32))


def test_q8act_closed_form(orc):
    """Q8Act (quant.rs:368-394): |q| <= 127, the block maximum maps to +-127,
    ties round away from zero, a zero block has d = s = 0, s = d * sum(q),
    and dequantisation is within d/2 of the input."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal(32 * 64).astype(np.float32)
    x[32:64] = 0.0
    # amax 127 gives d = 1 and id = 1: +-2.5 and 0.5 are ties
    x[64:96] = 0.0
    x[64], x[65], x[66], x[67] = 127.0, 2.5, -2.5, 0.5
    qs, d, s = orc.q8act(x)
    assert np.abs(qs.astype(np.int32)).max() <= 127
    assert d[1] == 0 and s[1] == 0 and not qs[32:64].any()
    assert d[2] == 1.0 and list(qs[64:68]) == [127, 3, -3, 1]
    xb = x.reshape(-1, 32)
    qb = qs.reshape(-1, 32).astype(np.int32)
    for b in range(xb.shape[0]):
        if d[b] == 0:
            continue
        j = np.argmax(np.abs(xb[b]))
        assert abs(qb[b, j]) == 127
        assert s[b] == np.float32(d[b] * np.float32(qb[b].sum()))
        assert np.all(np.abs(qb[b] * np.float64(d[b]) - xb[b]) <= d[b] * 0.5000001 + 1e-12)


@pytest.mark.parametrize("ty", ["Q8_0", "Q4_K", "Q6_K"])
def test_block_idots_against_dequantised_rows(orc, ty):
    """The per-32-block int32 dots, scaled by their block scales in float64,
    equal the float64 dot of dequantise_row(w) with the int8 activations: a
    wrong nibble, sign, offset or sub-scale index breaks the equality."""
    from biv_amd import synth
    rng = np.random.default_rng(11)
    n = 2048
    w = synth.quantize(TY[ty], rng.standard_normal((1, n)).astype(np.float32) * 0.02).reshape(-1)
    qs, d, s = orc.q8act(rng.standard_normal(n).astype(np.float32))
    idots = orc.block_idots(TY[ty], w, qs).astype(np.float64)
    wd = orc.dequantize_row(TY[ty], w, n).astype(np.float64)
    per_block_want = (wd * qs.astype(np.float64)).reshape(-1, 32).sum(1)
    if ty == "Q8_0":
        dw = np.array([np.frombuffer(w[34 * b:34 * b + 2].tobytes(), np.float16)[0] for b in range(n // 32)],
                      np.float64)
        assert np.allclose(idots * dw, per_block_want, rtol=0, atol=1e-9)
        assert np.array_equal(idots, (w.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
                                      * qs.astype(np.int64)).reshape(-1, 32).sum(1))
    elif ty == "Q4_K":
        # dequantised = d*sc*q - dmin*m: the q part is idot, the min part the block sum
        sb = w.reshape(-1, 144)
        got = []
        for b in range(n // 32):
            blk = sb[b // 8]
            dd = float(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
            dm = float(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
            j = b % 8
            sc_raw = blk[4:16]
            if j < 4:
                sc, m = sc_raw[j] & 63, sc_raw[j + 4] & 63
            else:
                sc = (sc_raw[j + 4] & 0xF) | ((sc_raw[j - 4] >> 6) << 4)
                m = (sc_raw[j + 4] >> 4) | ((sc_raw[j] >> 6) << 4)
            got.append(dd * sc * idots[b] - dm * m * qs[32 * b:32 * b + 32].astype(np.float64).sum())
        assert np.allclose(got, per_block_want, rtol=1e-6, atol=1e-6)
    else:
        sb = w.reshape(-1, 210)
        got = [float(np.frombuffer(sb[b // 8][208:210].tobytes(), np.float16)[0]) * idots[b] for b in range(n // 32)]
        assert np.allclose(got, per_block_want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("ty", ["Q8_0", "Q4_K", "Q6_K"])
def test_dot_against_float64(orc, ty):
    from biv_amd import synth
    rng = np.random.default_rng(3)
    n = 2048
    w = synth.quantize(TY[ty], rng.standard_normal((1, n)).astype(np.float32) * 0.02).reshape(-1)
    x = rng.standard_normal(n).astype(np.float32)
    qs, d, s = orc.q8act(x)
    ref = float(orc.dequantize_row(TY[ty], w, n).astype(np.float64) @ (qs * np.repeat(d, 32)).astype(np.float64))
    for level in range(orc.detect_level() + 1):
        assert abs(orc.dot(TY[ty], w, x, level) - ref) < 1e-4 * max(1.0, abs(ref)), level


def test_softmax_float64(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(256) * 3).astype(np.float32)
    p = orc.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.allclose(p, e / e.sum(), rtol=2e-6, atol=1e-9)
    assert abs(p.astype(np.float64).sum() - 1) < 1e-5


def test_route_cases(orc):
    # ties broken by the lower index, weights renormalised, floor 1/16384
    l = np.array([0.0, 3.0, 3.0, -1.0, 3.0], np.float32)
    ids, w = orc.route(l, 2)
    assert list(ids) == [1, 2] and np.allclose(w, [0.5, 0.5])
    l = np.full(300, -1e4, np.float32)
    l[7] = 0.0
    ids, w = orc.route(l, 3)
    assert ids[0] == 7 and list(ids[1:]) == [0, 1]
    assert w[0] == 1.0 and w[1] == 0.0


def test_matmul_thread_invariance(orc):
    """Rows are computed whole by one thread (ops.rs:95-126): the result does
    not depend on the thread count."""
    from biv_amd import synth
    rng = np.random.default_rng(9)
    w = synth.quantize(Q8_0, rng.standard_normal((96, 512)).astype(np.float32) * 0.02).reshape(-1)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    a = orc.matmul(Q8_0, w, 512, 96, x, threads=1)
    b = orc.matmul(Q8_0, w, 512, 96, x, threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for t in range(5):
        for r in (0, 37, 95):
            assert a[t, r] == np.float32(orc.dot(Q8_0, w[r * 544:(r + 1) * 544], x[t]))


def test_moe_single_expert_is_dense_ffn(orc):
    """With one expert and k = 1 every token goes to it with weight 1:
    fma(1, y, 0) = y, so the block equals dense_ffn bit for bit."""
    from biv_amd import synth
    layer = synth.make_layer(1, n_embd=256, n_expert=1, k=1, n_ff=64, shared=False)
    h = synth.make_tokens(2, 3, 256)
    out, ids, w, _ = orc.moe(layer, h, taps=True)
    assert not ids.any() and np.all(w == 1.0)
    dense = orc.dense_ffn(Q8_0, layer.gate.data, Q8_0, layer.up.data, Q8_0, layer.down.data, 256, 64, h)
    assert np.array_equal(out.view(np.uint32), dense.view(np.uint32))


def test_moe_shared_expert_gate(orc):
    """The shared expert's share is sigmoid(gate_inp . h) * dense_ffn(h),
    added after the routed experts (model.rs:890-896)."""
    from biv_amd import synth
    layer = synth.make_layer(4, n_embd=256, n_expert=8, k=2, n_ff=64, n_ff_sh=64)
    h = synth.make_tokens(5, 2, 256)
    out = orc.moe(layer, h)
    routed = orc.moe(synth.MoeLayer(**{**layer.__dict__, "shared": None, "n_ff_sh": 0}), h)
    sg, su, sd, gi = layer.shared
    ys = orc.dense_ffn(Q8_0, sg.data, Q8_0, su.data, Q8_0, sd.data, 256, 64, h)
    g = h @ gi.data.view(np.float32).astype(np.float64)
    want = routed + (1 / (1 + np.exp(-g)))[:, None] * ys
    assert np.allclose(out, want, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# float64 brute force of the composite functions: rms_norm, the SwiGLU of
# dense_ffn and the weighted combine of the MoE block.  Each expected value is
# built from dequantize_row and q8act only (both pinned above), never from the
# oracle function under test, and each test also shows that a plausible
# mistake (a swapped operand, a dropped term) lands far outside its bar.

def _deq(orc, ty, data, rows, cols):
    rs = orc.row_size(ty, cols)
    return np.stack([orc.dequantize_row(ty, data[r * rs:(r + 1) * rs], cols) for r in range(rows)]).astype(np.float64)


def _q8_f64(orc, x):
    """The Q8 activations of each row of x as float64 values qs * d."""
    x = np.atleast_2d(np.asarray(x, np.float32))
    out = np.empty(x.shape, np.float64)
    for i, row in enumerate(x):
        qs, d, _ = orc.q8act(row)
        out[i] = qs.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
    return out


def _silu64(g):
    return g / (1.0 + np.exp(-g))


def _dense64(orc, Wg, Wu, Wd, x, swap=False):
    """down . q8(silu(gate . q8(x)) * (up . q8(x))) in float64 (model.rs:1118-1126)."""
    xq = _q8_f64(orc, x)
    g, u = xq @ Wg.T, xq @ Wu.T
    if swap:
        g, u = u, g
    a = _silu64(g) * u
    return _q8_f64(orc, a.astype(np.float32)) @ Wd.T


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.sqrt(np.mean(np.asarray(b, np.float64) ** 2)))


@pytest.mark.parametrize("eps", [1e-6, 0.5])
def test_rms_norm_float64(orc, eps):
    """ops::rms_norm (ops.rs:136-144): x / sqrt(mean(x^2) + eps) * w per row.
    eps = 0.5 on rows of small values makes a dropped or misplaced eps, a sum
    instead of a mean, or a missing sqrt fail."""
    rng = np.random.default_rng(21)
    n = 2048
    w = (1 + 0.5 * rng.standard_normal(n)).astype(np.float32)
    x = (rng.standard_normal((7, n)) * (0.3 if eps > 0.1 else 2.0)).astype(np.float32)
    x[3] = 0.0  # zero row: scale 1/sqrt(eps), output 0
    got = orc.rms_norm(x, w, eps)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + eps) * w.astype(np.float64)
    # a few f32 roundings per element: ss, the division, sqrt, 1/., scale*w, v*.
    assert np.all(np.abs(got - want) <= 8 * np.finfo(np.float32).eps * np.abs(want) + 1e-30)
    assert not np.any(got[3])
    if eps > 0.1:
        nz = np.arange(7) != 3
        wrong = x64[nz] / np.sqrt(np.mean(x64[nz] ** 2, axis=1, keepdims=True)) * w  # eps dropped
        assert np.abs(wrong - want[nz]).max() > 1e-2 * np.abs(want).max()


@pytest.mark.parametrize("types", [(Q8_0, Q8_0, Q8_0), (Q4K, Q4K, Q6K)])
def test_dense_ffn_float64(orc, types):
    """dense_ffn (model.rs:1118-1126): down . q8(silu(gate . x) * (up . x))
    with gate and up different matrices.  Against float64 sums of the
    dequantised rows; the bar is a few re-quantisation steps of the
    intermediate (a value near a rounding boundary can land on either side),
    while silu on the wrong matrix misses it by two orders of magnitude."""
    from biv_amd import synth
    rng = np.random.default_rng(33)
    e, ff, n = 512, 256, 6
    gty, uty, dty = types
    gw, uw, dw = (synth.make_weight(rng, gty, e, ff), synth.make_weight(rng, uty, e, ff),
                  synth.make_weight(rng, dty, ff, e))
    x = rng.standard_normal((n, e)).astype(np.float32)
    got = orc.dense_ffn(gty, gw.data, uty, uw.data, dty, dw.data, e, ff, x)
    Wg, Wu, Wd = _deq(orc, gty, gw.data, ff, e), _deq(orc, uty, uw.data, ff, e), _deq(orc, dty, dw.data, e, ff)
    want = _dense64(orc, Wg, Wu, Wd, x)
    assert _rel(got, want) < 5e-4
    assert _rel(_dense64(orc, Wg, Wu, Wd, x, swap=True), want) > 0.3


def test_moe_k3_weighted_combine_float64(orc):
    """Model::moe (model.rs:860-898) with k = 3 distinct weights per token and
    a shared expert: out_t = sum_j w_j * y_{e_j}(h_t) + sigmoid(gate_inp . h_t)
    * y_shared(h_t), with route (model.rs:256-268) redone in float64 (softmax,
    the three highest, p / their sum) and every expert's SwiGLU in float64."""
    from biv_amd import synth
    e, ne, k, ff = 256, 8, 3, 64
    layer = synth.make_layer(41, n_embd=e, n_expert=ne, k=k, n_ff=ff, n_ff_sh=ff)
    h = synth.make_tokens(42, 5, e)
    out, ids, w, _ = orc.moe(layer, h, taps=True)
    R = layer.router.data.view(np.float32).reshape(ne, e).astype(np.float64)
    h64 = h.astype(np.float64)
    logits = h64 @ R.T
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    want_ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
    assert np.array_equal(ids, want_ids)
    want_w = np.take_along_axis(p, want_ids, 1)
    want_w /= want_w.sum(axis=1, keepdims=True)
    assert np.allclose(w, want_w, rtol=1e-5)
    assert all(len(set(np.round(r, 6))) == k for r in want_w), "weights must be distinct to pin the combine"
    ys = []
    for x_ in range(ne):
        Wg = _deq(orc, Q8_0, layer.gate.expert(x_), ff, e)
        Wu = _deq(orc, Q8_0, layer.up.expert(x_), ff, e)
        Wd = _deq(orc, Q8_0, layer.down.expert(x_), e, ff)
        ys.append(_dense64(orc, Wg, Wu, Wd, h))
    sg, su, sd, gi = layer.shared
    ysh = _dense64(orc, _deq(orc, Q8_0, sg.data, ff, e), _deq(orc, Q8_0, su.data, ff, e),
                   _deq(orc, Q8_0, sd.data, e, ff), h)
    gate = 1 / (1 + np.exp(-(h64 @ gi.data.view(np.float32).astype(np.float64))))
    want = np.zeros((h.shape[0], e))
    for t in range(h.shape[0]):
        for j in range(k):
            want[t] += want_w[t, j] * ys[want_ids[t, j]][t]
        want[t] += gate[t] * ysh[t]
    assert _rel(out, want) < 5e-4
    # weights applied in the wrong rank order, or the shared gate dropped, miss the bar
    bad = np.zeros_like(want)
    for t in range(h.shape[0]):
        for j in range(k):
            bad[t] += want_w[t, k - 1 - j] * ys[want_ids[t, j]][t]
        bad[t] += gate[t] * ysh[t]
    assert _rel(bad, want) > 2e-2
    assert _rel(want - gate[:, None] * ysh, want) > 2e-2


def test_route_total_order_nan(orc):
    """route sorts with f32::total_cmp (model.rs:264): +NaN ranks above every
    number and -NaN below.  Logits [-NaN, 1, 2, +NaN]: softmax's max ignores
    NaN (f32::max); the index-order sum takes the first NaN it meets (-NaN) and
    x86 NaN propagation gives p = [-NaN, -NaN, -NaN, +NaN].  So the top 3 are
    expert 3, then 0 and 1 (equal keys, lower index first)."""
    l = np.array([0, 1.0, 2.0, 0], np.float32)
    l.view(np.uint32)[0] = 0xFFC00000
    l.view(np.uint32)[3] = 0x7FC00000
    ids, w = orc.route(l, 3)
    assert list(ids) == [3, 0, 1]
    assert np.all(np.isnan(w))
