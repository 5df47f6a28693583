"""moe_layer_forward_noalloc (no device allocation; scratch in a file-scope
device array) against moe_layer_forward, which allocates its scratch, on the
same layer and inputs: bit-identical outputs, top-k indices and gates, on
consecutive calls with a smaller T second (the array keeps the previous
call's contents), plus the oracle on the small cases and the size limits."""
import ctypes

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

MOE_ERR_ARG = 2


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _experts(dtype, E, D, dff, seed):
    rg = D if dtype == 2 else D // 2
    rd = dff if dtype == 2 else dff // 2

    def qbytes(n, s):
        u = O.uniform_u32(n, s)
        if dtype == 2:
            return ((u % 255).astype(np.int64) - 127).astype(np.int8)
        return (u & 0xFF).astype(np.uint8)

    return O.ExpertSet(dtype, qbytes(E * dff * rg, seed).reshape(E, dff, rg),
                       np.abs(O.normal(E * dff, seed + 3, 0.0, 2e-4)).reshape(E, dff),
                       qbytes(E * dff * rg, seed + 1).reshape(E, dff, rg),
                       np.abs(O.normal(E * dff, seed + 4, 0.0, 2e-4)).reshape(E, dff),
                       qbytes(E * D * rd, seed + 2).reshape(E, D, rd),
                       np.abs(O.normal(E * D, seed + 5, 0.0, 2e-4)).reshape(E, D), D, dff)


def _run(moehip, layer, x, resid, noalloc):
    T, D = x.shape
    k = layer.top_k
    dx = moehip.DeviceBuffer.from_array(x)
    dr = moehip.DeviceBuffer.from_array(resid) if resid is not None else None
    do, di, dp = (moehip.DeviceBuffer(T * D * 4), moehip.DeviceBuffer(T * k * 4),
                  moehip.DeviceBuffer(T * k * 4))
    fn = moehip.lib().moe_layer_forward_noalloc if noalloc else moehip.lib().moe_layer_forward
    st = fn(layer.h, dx.ptr, None if dr is None else dr.ptr, T, do.ptr, di.ptr, dp.ptr)
    moehip.check(st, "noalloc forward" if noalloc else "forward")
    moehip.synchronize()
    return (do.download((T, D), np.float32), di.download((T, k), np.int32),
            dp.download((T, k), np.float32))


CASES = [
    # dtype, E, D, dff, top_k, bias, T values (consecutive calls)
    (2, 128, 2048, 768, 8, False, (16, 3)),      # configs[2] shape
    (3, 128, 2048, 768, 8, False, (4, 1)),       # Q4 at the config shape, one-token path
    (3, 60, 512, 256, 8, True, (32, 2, 1)),      # the largest T; bias; E not a power of two
    (2, 128, 2048, 768, 8, False, (32, 17)),     # Q8 at the config shape at the largest T
]


@pytest.mark.parametrize("dtype,E,D,dff,top_k,bias,Ts", CASES)
def test_noalloc_matches_allocating_forward(moehip, dtype, E, D, dff, top_k, bias, Ts):
    print("noalloc case", dtype, E, D, dff, top_k, bias, Ts, flush=True)
    seed = 900 + dtype * 10 + E
    ex = _experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 7, 0.0, 0.02).reshape(E, D)
    rb = O.normal(E, seed + 8, 0.0, 0.05) if bias else None
    layer = moehip.MoeLayer.from_arrays(dtype, rw, rb, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds,
                                        top_k=top_k)
    for i, T in enumerate(Ts):
        x = O.normal(T * D, seed + 20 + i, 0.0, 1.0).reshape(T, D)
        r = O.normal(T * D, seed + 40 + i, 0.0, 1.0).reshape(T, D) if i % 2 == 0 else None
        got = _run(moehip, layer, x, r, True)
        ref = _run(moehip, layer, x, r, False)
        np.testing.assert_array_equal(got[1], ref[1], err_msg=f"idx T={T}")
        np.testing.assert_array_equal(bits(got[2]), bits(ref[2]), err_msg=f"p T={T}")
        np.testing.assert_array_equal(bits(got[0]), bits(ref[0]), err_msg=f"out T={T}")
        if T <= 4:
            want, widx, wp, _ = O.moe_block(x, r, rw, rb, ex, top_k)
            np.testing.assert_array_equal(got[1], widx)
            np.testing.assert_array_equal(bits(got[0]), bits(want))
        # and again after the allocating forward reused the layer
        again = _run(moehip, layer, x, r, True)
        np.testing.assert_array_equal(bits(again[0]), bits(got[0]))
    layer.close()


def test_noalloc_limits(moehip):
    """T above 32, or a scratch need above the 4 MiB array, is refused with
    MOE_ERR_ARG and a message; the layer still works afterwards."""
    dtype, E, D, dff, top_k = 3, 16, 512, 2048, 8
    ex = _experts(dtype, E, D, dff, 950)
    rw = O.normal(E * D, 951, 0.0, 0.02).reshape(E, D)
    layer = moehip.MoeLayer.from_arrays(dtype, rw, None, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds,
                                        top_k=top_k)
    L = moehip.lib()
    for T in (33, 32):   # 33: over the token limit; 32 tokens at d_ff 2048: over the array
        dx = moehip.DeviceBuffer(T * D * 4)
        do = moehip.DeviceBuffer(T * D * 4)
        st = L.moe_layer_forward_noalloc(layer.h, dx.ptr, None, T, do.ptr, None, None)
        assert st == MOE_ERR_ARG, T
        assert b"layer_forward_noalloc" in L.moe_last_error()
    x = O.normal(6 * D, 952, 0.0, 1.0).reshape(6, D)
    got = _run(moehip, layer, x, None, True)
    ref = _run(moehip, layer, x, None, False)
    np.testing.assert_array_equal(bits(got[0]), bits(ref[0]))
    np.testing.assert_array_equal(got[1], ref[1])
    layer.close()
