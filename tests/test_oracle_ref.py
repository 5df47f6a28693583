"""Restatement vs the live compiled reference on fresh seeded inputs.

Only in the build container, where oracle/_ref/ is built from /root/reference;
skipped elsewhere (the GPU box has no reference tree).  CPU only.
"""
import ctypes

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def ref_gemv(A, q, s, dtype, M, N, K):
    C = np.empty((M, N), np.float32)
    qw = O.QW(q.ctypes.data, s.ctypes.data, N, K, dtype)
    O.ref_kernels().matmul_adaptive(A.ctypes.data, None, ctypes.addressof(qw), C.ctypes.data,
                                    M, N, K)
    return C


@pytest.mark.parametrize("seed", range(12))
def test_gemv_random_shapes(seed):
    rng = np.random.default_rng(seed)
    for dtype in (2, 3):
        M = int(rng.integers(1, 5))
        N = int(rng.integers(1, 40))
        K = int(rng.integers(1, 300))
        A = O.normal(M * K, 1000 + seed, 0.0, float(rng.choice([0.5, 2.0, 50.0]))).reshape(M, K)
        if dtype == 2:
            q = (O.uniform_u32(N * K, 2000 + seed) & 0xFF).astype(np.uint8).view(np.int8)
            C = O.gemv_q8(A, q, np.ones(N, np.float32) * 0.01, N, K)
        else:
            q = (O.uniform_u32(N * (K // 2) + (K & 1), 3000 + seed) & 0xFF).astype(np.uint8)
            C = O.gemv_q4(A, q, np.ones(N, np.float32) * 0.01, N, K)
        R = ref_gemv(A, q, np.ones(N, np.float32) * 0.01, dtype, M, N, K)
        np.testing.assert_array_equal(bits(C), bits(R))


@pytest.mark.parametrize("seed", range(4))
def test_layer_random(seed):
    dtype = 2 + seed % 2
    T, D, dff, E = 1 + seed, 128, 64, 32
    ex = O.make_experts(dtype, E, D, dff, 9000 + seed)
    x = O.normal(T * D, 9100 + seed, 0.0, 1.0).reshape(T, D)
    rw = O.normal(E * D, 9200 + seed, 0.0, 0.05).reshape(E, D)
    rms2 = O.normal(D, 9300 + seed, 1.0, 0.1)
    xo = x.copy()
    O.ref_trace().ref_moe_layer(xo.ctypes.data, T, D, E, 8, dff, rms2.ctypes.data, rw.ctypes.data,
                                None, ctypes.addressof(ex.Wg), ctypes.addressof(ex.Wu),
                                ctypes.addressof(ex.Wd))
    out, _, _, _ = O.moe_block(O.rmsnorm(x, rms2), x, rw, None, ex)
    np.testing.assert_array_equal(bits(out), bits(xo))


def test_topk_random_ties():
    rng = np.random.default_rng(7)
    for _ in range(300):
        x = np.round(rng.normal(0, 1.5, 128)).astype(np.float32)
        idx_r = np.empty(8, np.int32)
        val_r = np.empty(8, np.float32)
        O.ref_trace().ref_topk_desc(x.ctypes.data, 128, 8, idx_r.ctypes.data, val_r.ctypes.data)
        idx, val = O.topk_desc(x, 8)
        np.testing.assert_array_equal(idx, idx_r)
        np.testing.assert_array_equal(val, val_r)


def test_expf_sampled_matches_host():
    # the restatement calls the same host expf; this guards the test wrapper
    x = O.normal(100000, 77, 0.0, 30.0)
    y = O.expf_array(x)
    s = x.copy()
    O.ref_trace().ref_silu(s.ctypes.data, s.size)
    want = (x / (np.float32(1.0) + O.expf_array(-x))).astype(np.float32)
    np.testing.assert_array_equal(bits(s), bits(want))
    assert np.all(np.isfinite(y) | (x > 88))
