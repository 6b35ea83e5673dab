"""The entry point that allocates nothing (biv_hip_moe_forward_device_noalloc)
against biv_hip_moe_forward_device, through the C ABI: bit-identical outputs
on two calls in a row, the second with fewer tokens (the fixed scratch keeps
the first call's contents), with and without the residual add; and a clear
error past its size."""
import numpy as np
import pytest

from biv_amd import synth

pytestmark = pytest.mark.gpu


def test_noalloc_matches_forward_device():
    from biv_amd import hip
    with hip.HipEngine(0) as eng:
        layer = synth.make_layer(1)
        moe = eng.moe(layer)
        E = layer.n_embd
        # T = 256: the prefill pre-pass and the matrix-core router
        for T, add in ((256, False), (40, False), (5, False), (1, True)):
            print(f"case noalloc T={T} add={add}", flush=True)
            h = synth.make_tokens(50 + T, T, offsets=True)
            x0 = synth.make_tokens(60 + T, T)
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
        big = 1000
        hd = eng.malloc(big * E * 4)
        try:
            with pytest.raises(hip.HipError) as e:
                moe.forward_device_noalloc(hd, big, hd)
            assert e.value.code == -1 and "no-allocation" in str(e.value)
        finally:
            eng.free(hd)
