"""Device rowwise quantizer (export.py:23-36) equals the oracle's restatement
bit for bit (scales and packed bytes)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,N,K", [(2, 768, 2048), (3, 2048, 768), (2, 5, 33), (3, 7, 10)])
def test_quantize_rows(moehip, dtype, N, K):
    W = O.normal(N * K, 31 * N + K, 0.0, 0.02).reshape(N, K)
    W[0, :] = 0.0  # zero row: scale clamps at 1e-8
    if N > 2:
        W[1, 3] = 1e-3  # a single large entry
    q_want, s_want = (O.quant_q8 if dtype == 2 else O.quant_q4)(W)
    dW = moehip.DeviceBuffer.from_array(W)
    dq = moehip.DeviceBuffer(q_want.nbytes)
    ds = moehip.DeviceBuffer(s_want.nbytes)
    moehip.check(moehip.lib().moe_quantize_rows_dev(dtype, dW.ptr, N, K, dq.ptr, ds.ptr), "quantize")
    q = dq.download(q_want.shape, q_want.dtype)
    s = ds.download(s_want.shape, np.float32)
    np.testing.assert_array_equal(s.view(np.uint32), s_want.view(np.uint32))
    np.testing.assert_array_equal(q, q_want)


@pytest.mark.parametrize("dtype", [2, 3])
def test_quantize_ties(moehip, dtype):
    """Rows whose w/s lands exactly on k + 0.5 round to the even neighbour."""
    if dtype == 2:
        W = np.array([[127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 126.5]], np.float32)
    else:
        W = np.array([[7.0, 2.5, -2.5, 3.5, -6.5, 0.5, -0.5, 1.5]], np.float32)
    q_want, s_want = (O.quant_q8 if dtype == 2 else O.quant_q4)(W)
    dW = moehip.DeviceBuffer.from_array(W)
    dq, ds = moehip.DeviceBuffer(q_want.nbytes), moehip.DeviceBuffer(4)
    moehip.check(moehip.lib().moe_quantize_rows_dev(dtype, dW.ptr, 1, 8, dq.ptr, ds.ptr), "quantize")
    np.testing.assert_array_equal(dq.download(q_want.shape, q_want.dtype), q_want)
    assert ds.download((1,), np.float32)[0] == 1.0


@pytest.mark.parametrize("dtype", [2, 3])
def test_quantize_rows_exact_exporter(moehip, dtype):
    """The device quantizer against the exporter's exact answer
    (quant_pin_cases: RN32 division, half-to-even) on rows where a
    reciprocal multiply, a double-precision scale, an unrounded quotient or
    half-away rounding would each give another integer."""
    import quant_pin_cases as Q
    div = 127 if dtype == 2 else 7
    W, _ = Q.find_rows(div)
    N, K = W.shape
    q_exact, s_want = Q.expected_rows(W, div)
    q_want = q_exact.astype(np.int8) if dtype == 2 else Q.pack_q4(q_exact)
    dW = moehip.DeviceBuffer.from_array(W)
    dq, ds = moehip.DeviceBuffer(q_want.nbytes), moehip.DeviceBuffer(4 * N)
    moehip.check(moehip.lib().moe_quantize_rows_dev(dtype, dW.ptr, N, K, dq.ptr, ds.ptr), "quantize")
    np.testing.assert_array_equal(ds.download((N,), np.float32).view(np.uint32), s_want.view(np.uint32))
    np.testing.assert_array_equal(dq.download(q_want.shape, q_want.dtype), q_want)
