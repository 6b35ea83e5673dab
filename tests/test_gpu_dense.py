"""Parity of the dense SwiGLU FFN (Ffn::Dense, model.rs:239-246;
dense_ffn, model.rs:1118-1126) on the GPU with the CPU oracle's dense_ffn.

The rows of a dense FFN are longer than the experts' (n_ff up to 17408 in
the qwen35 dense models), so the kernels stream each row in chunks of 512
elements and carry the reference's 16 x86 chains across the chunks: every
output carries the oracle's bits (the bar asserted is the north star's
max|d| <= 1e-3 * RMS plus >= 99.99% identical bits).
"""
import numpy as np
import pytest

from biv_amd import gguf, synth
from biv_amd.hip import HipError

pytestmark = pytest.mark.gpu

Q8_0, Q4K, Q6K, BF16 = synth.Q8_0, synth.Q4K, synth.Q6K, synth.BF16


@pytest.fixture(scope="module")
def engine():
    from biv_amd import hip
    e = hip.HipEngine(0)
    yield e
    e.close()


_layers = {}


def dense_for(engine, **kw):
    key = tuple(sorted(kw.items()))
    if key not in _layers:
        layer = synth.make_dense(**kw)
        _layers[key] = (layer, engine.dense(layer))
    return _layers[key]


def reference(orc, layer, h):
    g, u, d = layer.gate, layer.up, layer.down
    return orc.dense_ffn(g.ty, g.data, u.ty, u.data, d.ty, d.data, layer.n_embd, layer.n_ff, h, threads=8)


def check(ref, got, min_exact=0.9999):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    err = float(np.abs(ref.astype(np.float64) - got).max())
    exact = float(np.mean(ref.view(np.uint32) == got.view(np.uint32)))
    print(f"max|d|/RMS = {err / rms:.2e}, bit-identical fraction = {exact:.6f}")
    assert err <= 1e-3 * rms
    assert exact >= min_exact


@pytest.mark.parametrize("T", [1, 2, 3, 5, 8, 9, 17, 40, 64, 130])
def test_dense_q8(orc, engine, T):
    print(f"case dense q8 T={T}", flush=True)
    layer, d = dense_for(engine, seed=11, n_embd=2048, n_ff=3584)
    h = synth.make_tokens(600 + T, T, n_embd=2048)
    got = d.ffn(h)
    check(reference(orc, layer, h), got)
    assert np.array_equal(got.view(np.uint32), d.ffn(h).view(np.uint32)), "not bit-identical run to run"


@pytest.mark.parametrize("types", [(Q4K, Q4K, Q6K), (Q6K, Q6K, Q4K), (BF16, BF16, BF16), (Q8_0, Q8_0, BF16)])
def test_dense_types(orc, engine, types):
    print(f"case dense types {types}", flush=True)
    layer, d = dense_for(engine, seed=12, n_embd=1536, n_ff=2560, types=types)
    for T in (1, 6):
        h = synth.make_tokens(700 + T, T, n_embd=1536)
        check(reference(orc, layer, h), d.ffn(h))


def test_dense_large_rows(orc, engine):
    """A qwen35 9B-sized FFN: n_embd 4096, n_ff 12288 (24 chunks per down row),
    at 2, 5 and 8 tokens (each workgroup's tokens and weight ring differ)."""
    print("case dense 4096 x 12288", flush=True)
    layer, d = dense_for(engine, seed=13, n_embd=4096, n_ff=12288)
    for T in (2, 5, 8):
        h = synth.make_tokens(800 + T, T, n_embd=4096)
        check(reference(orc, layer, h), d.ffn(h))


def test_dense_add_and_device(orc, engine):
    """out += ffn(h) (the residual add of Model::layer), through device pointers."""
    print("case dense add", flush=True)
    layer, d = dense_for(engine, seed=11, n_embd=2048, n_ff=3584)
    T = 3
    h = synth.make_tokens(900, T, n_embd=2048)
    x = synth.make_tokens(901, T, n_embd=2048)
    ref = reference(orc, layer, h)
    got = d.ffn(h, out=x.copy(), add=True)
    assert np.array_equal(got.view(np.uint32), (x + ref).view(np.uint32))
    e = engine
    nb = h.nbytes
    hd, od = e.malloc(nb), e.malloc(nb)
    try:
        e.h2d(hd, h)
        e.h2d(od, x)
        d.forward_device(hd, T, od, add=True)
        e.sync()
        back = np.empty_like(x)
        e.d2h(back, od)
    finally:
        e.free(hd)
        e.free(od)
    assert np.array_equal(back.view(np.uint32), got.view(np.uint32))


def test_dense_errors(engine):
    print("case dense errors", flush=True)
    rng = np.random.default_rng(1)
    g = engine.upload_weight(synth.make_weight(rng, Q8_0, 1024, 1536))
    u = engine.upload_weight(synth.make_weight(rng, Q4K, 1024, 1536))
    dn = engine.upload_weight(synth.make_weight(rng, Q8_0, 1536, 1024))
    bad = engine.upload_weight(synth.make_weight(rng, Q8_0, 1024, 1024))
    import ctypes
    out = ctypes.c_void_p()
    rc = engine.L.biv_hip_dense_create(engine.h, g, u, dn, ctypes.byref(out))
    assert rc == -2 and "one type" in engine.L.biv_hip_last_error(engine.h).decode()
    rc = engine.L.biv_hip_dense_create(engine.h, g, g, bad, ctypes.byref(out))
    assert rc == -1 and "shapes" in engine.L.biv_hip_last_error(engine.h).decode()
    layer, d = dense_for(engine, seed=11, n_embd=2048, n_ff=3584)
    assert d.ffn(np.zeros((0, 2048), np.float32)).shape == (0, 2048)


def test_dense_from_gguf(orc, engine, tmp_path):
    """Loader::ffn of a dense layer from a file: the same bits as the layer uploaded directly."""
    print("case dense gguf", flush=True)
    layers = [synth.make_dense(20 + i, n_embd=1024, n_ff=2048, types=(Q4K, Q4K, Q6K)) for i in range(2)]
    p = str(tmp_path / "dense.gguf")
    gguf.write_dense(p, layers)
    h = synth.make_tokens(950, 4, n_embd=1024)
    with gguf.Gguf(p) as g:
        for i, layer in enumerate(layers):
            d = gguf.dense_from_gguf(engine, g, i)
            got = d.ffn(h)
            check(reference(orc, layer, h), got)
        with pytest.raises(HipError) as e:
            gguf.dense_from_gguf(engine, g, 2)
        assert e.value.code == -1
