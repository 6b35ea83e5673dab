"""The entry point that allocates nothing (biv_hip_moe_forward_device_noalloc)
against biv_hip_moe_forward_device, through the C ABI: bit-identical outputs
on two calls in a row, the second with fewer tokens (the fixed scratch keeps
the first call's contents), with and without the residual add, for a Q8_0
layer and a BF16 one (whose matrix-core kernels pass the bf16 halves through
the scratch); a clear error past its size, with stage timing on, and for a
second context on the same GPU while the first holds the buffer."""
import numpy as np
import pytest

from biv_amd import synth

pytestmark = pytest.mark.gpu


def _match(eng, moe, E, cases):
    for T, add in cases:
        print(f"case noalloc T={T} add={add}", flush=True)
        h = synth.make_tokens(50 + T, T, n_embd=E, offsets=True)
        x0 = synth.make_tokens(60 + T, T, n_embd=E)
        hd, ad, bd = eng.malloc(h.nbytes), eng.malloc(h.nbytes), eng.malloc(h.nbytes)
        try:
            eng.h2d(hd, h)
            eng.h2d(ad, x0)
            eng.h2d(bd, x0)
            moe.forward_device(hd, T, ad, add=add)
            moe.forward_device_noalloc(hd, T, bd, add=add)
            eng.sync()
            a = eng.d2h(np.empty_like(h), ad)
            b = eng.d2h(np.empty_like(h), bd)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (T, add)
            assert np.abs(a).max() > 0
        finally:
            for p in (hd, ad, bd):
                eng.free(p)


def test_noalloc_matches_forward_device():
    from biv_amd import hip
    with hip.HipEngine(0) as eng:
        layer = synth.make_layer(1)
        moe = eng.moe(layer)
        E = layer.n_embd
        # T = 256: the prefill pre-pass and the matrix-core router; T <= 3:
        # the routing inside the gate/up launch (its routing workgroup
        # writes the dispatch records into the fixed scratch)
        _match(eng, moe, E, ((256, False), (40, False), (5, False), (3, False), (2, True), (1, True)))
        big = 1000
        hd = eng.malloc(big * E * 4)
        try:
            with pytest.raises(hip.HipError) as e:
                moe.forward_device_noalloc(hd, big, hd)
            assert e.value.code == -1 and "no-allocation" in str(e.value)
            # stage timing creates events: refused
            eng.set_timing(True)
            try:
                with pytest.raises(hip.HipError) as e:
                    moe.forward_device_noalloc(hd, 1, hd)
                assert e.value.code == -1 and "timing" in str(e.value)
            finally:
                eng.set_timing(False)
        finally:
            eng.free(hd)


def test_noalloc_bf16_layer():
    """BF16 experts at T = 256 (pre-pass halves of h, matrix-core gate/up
    writing the intermediate's halves into the scratch for down), then 64
    (the split launch) and 5 (the chain kernels)."""
    from biv_amd import hip
    with hip.HipEngine(0) as eng:
        layer = synth.make_layer(3, n_expert=64, types=(synth.BF16, synth.BF16, synth.BF16))
        moe = eng.moe(layer)
        _match(eng, moe, layer.n_embd, ((256, False), (64, True), (5, False)))


def test_noalloc_one_holder_per_gpu():
    """A second context's call on the GPU whose buffer another holds gets
    BIV_HIP_E_BUSY (-8); once the holder is destroyed it runs."""
    from biv_amd import hip
    layer = synth.make_layer(4, n_expert=16)
    h = synth.make_tokens(7, 2)
    with hip.HipEngine(0) as e1:
        m1 = e1.moe(layer)
        hd = e1.malloc(h.nbytes)
        od = e1.malloc(h.nbytes)
        e1.h2d(hd, h)
        m1.forward_device_noalloc(hd, 2, od)
        e1.sync()
        with hip.HipEngine(0) as e2:
            m2 = e2.moe(layer)
            with pytest.raises(hip.HipError) as e:
                m2.forward_device_noalloc(hd, 2, od)
            assert e.value.code == -8
        e1.sync()
        e1.free(hd)
        e1.free(od)
    with hip.HipEngine(0) as e3:
        m3 = e3.moe(layer)
        hd = e3.malloc(h.nbytes)
        od = e3.malloc(h.nbytes)
        e3.h2d(hd, h)
        m3.forward_device_noalloc(hd, 2, od)
        e3.sync()
        e3.free(hd)
        e3.free(od)
