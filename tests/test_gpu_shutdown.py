"""moe_shutdown (the API's context destroy): refused while a layer is alive,
frees the library's buffers and stream once every layer is destroyed, and the
next calls initialise the library again with bit-identical results (the
drop-in re-uploads its weights, a new layer forwards as the old one did)."""
import gc

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

MOE_ERR_ARG = 2


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_shutdown_refuses_live_layers_then_reinitialises(moehip):
    gc.collect()   # layers other tests dropped without close()
    L = moehip.lib()
    D, dff, E, T = 256, 128, 16, 3
    ex = O.make_experts(3, E, D, dff, 71)
    rw = O.normal(E * D, 72, 0.0, 0.05).reshape(E, D)
    x = O.normal(T * D, 73, 0.0, 1.0).reshape(T, D)
    want, widx, _, _ = O.moe_block(x, x, rw, None, ex)
    W = O.normal(768 * 2048, 74, 0.0, 0.02).reshape(768, 2048)
    q, s = O.quant_q8(W)
    xv = O.normal(2048, 75, 0.0, 1.0).reshape(1, 2048)
    gwant = O.gemv_q8(xv, q, s, 768, 2048)
    wq = {"q": q, "s": s, "dtype": 2}
    np.testing.assert_array_equal(bits(moehip.matmul_adaptive(xv, None, wq, 768, 2048)), bits(gwant))

    layer = moehip.MoeLayer.from_arrays(3, rw, None, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds)
    got, idx, _ = layer.forward(x, x)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(got), bits(want))

    assert L.moe_shutdown() == MOE_ERR_ARG
    assert b"still alive" in L.moe_last_error()
    # refused means nothing was freed: the layer still forwards
    got, _, _ = layer.forward(x, x)
    np.testing.assert_array_equal(bits(got), bits(want))
    layer.close()
    gc.collect()

    moehip.shutdown()
    moehip.shutdown()   # a second call with nothing initialised is a no-op
    # every entry point initialises device 0 again: the drop-in re-uploads
    np.testing.assert_array_equal(bits(moehip.matmul_adaptive(xv, None, wq, 768, 2048)), bits(gwant))
    layer = moehip.MoeLayer.from_arrays(3, rw, None, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds)
    got, idx, _ = layer.forward(x, x)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(got), bits(want))
    layer.close()
    moehip.init(0)   # already initialised (lazily, on device 0): accepted
