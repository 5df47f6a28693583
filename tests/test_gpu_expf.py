"""The device expf equals the host glibc expf on all 2^32 inputs, and the fused
SiLU*up equals the reference formula bit for bit (test_model_trace.c:229-236,
:500).  The host side of the comparison is the oracle's libm call, run in
threads over 2^26-input chunks."""
import ctypes
import concurrent.futures as cf

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_expf_exhaustive(moehip):
    chunk = 1 << 26
    dy = moehip.DeviceBuffer(chunk * 4)
    total_bad = 0
    first = None
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        futs = []
        for c in range(1 << 6):
            start = c * chunk
            moehip.check(moehip.lib().moe_expf_bits_dev(start, dy.ptr, chunk), "expf_bits")
            y = dy.download((chunk,), np.float32)
            futs.append(ex.submit(O.expf_mismatches, start, y))
            if c % 16 == 15:
                print(f"expf chunks done: {c + 1}/64", flush=True)
            if len(futs) >= 8:
                n, f = futs.pop(0).result()
                total_bad += n
                first = first if (first is not None or n == 0) else f
        for fu in futs:
            n, f = fu.result()
            total_bad += n
            first = first if (first is not None or n == 0) else f
    assert total_bad == 0, f"{total_bad} mismatches, first input bits 0x{first:08x}"


def test_silu_mul_matches_oracle(moehip):
    g = np.concatenate([O.normal(100000, 1, 0.0, 6.0),
                        np.array([0.0, -0.0, 88.0, -88.0, 89.0, -104.0, 1e-30, np.inf, -np.inf, np.nan],
                                 np.float32)])
    u = O.normal(g.size, 2, 0.0, 2.0)
    dg, du, dh = (moehip.DeviceBuffer.from_array(g), moehip.DeviceBuffer.from_array(u),
                  moehip.DeviceBuffer(g.nbytes))
    moehip.check(moehip.lib().moe_silu_mul_dev(dg.ptr, du.ptr, dh.ptr, g.size))
    h = dh.download(g.shape, np.float32)
    want = (O.silu(g) * u).astype(np.float32)
    same = (bits(h) == bits(want)) | (np.isnan(h) & np.isnan(want))
    assert same.all()


@pytest.mark.parametrize("dtype", [2, 3])
def test_epilogue_division_exhaustive(moehip, dtype):
    """The kernels' (float)dot / 127.0f (or 7.0f) equals the IEEE quotient for
    every int32 dot (kernels.c:71, :125)."""
    bad = ctypes.c_ulonglong(123)
    moehip.check(moehip.lib().moe_selfcheck_qdot_dev(dtype, ctypes.byref(bad)), "selfcheck")
    assert bad.value == 0
