"""Pins the oracle by routes other than its own formulas: numpy library
routines (int64 matmul, stable sort, float64 math), invariants (column
permutation, linearity in the weights, row independence) and special cases.
Each check is chosen so that a plausible slip (a wrong nibble order, a dropped
offset, an off-by-one in K, a transposed operand, a swapped tie rule) fails.
CPU only.
"""
import numpy as np
import pytest

import oracle as O


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def trunc_act(A, mult):
    p = (A.astype(np.float32) * np.float32(mult)).astype(np.float32)
    out = np.full(p.shape, np.iinfo(np.int32).min, dtype=np.int64)
    ok = (p >= -2147483648.0) & (p < 2147483648.0)
    out[ok] = np.trunc(p[ok]).astype(np.int64)
    return out


def epilogue(dot64, div, s):
    d32 = ((dot64 + 2**31) % 2**32 - 2**31).astype(np.int32)   # int32 wrap
    f = d32.astype(np.float32)
    f = (f / np.float32(div)).astype(np.float32)
    return (f * s[None, :].astype(np.float32)).astype(np.float32)


def unpack_q4(q, N, K):
    b = q[: N * (K // 2)].reshape(N, K // 2) if q.ndim == 1 else q
    w = np.empty((N, K), np.int64)
    w[:, 0::2] = (b & 0x0F).astype(np.int64) - 8
    w[:, 1::2] = (b >> 4).astype(np.int64) - 8
    return w


@pytest.mark.parametrize("M,N,K", [(1, 7, 64), (3, 5, 31), (2, 16, 256)])
def test_q8_equals_int64_matmul(M, N, K):
    A = O.normal(M * K, 5 + K, 0.0, 3.0).reshape(M, K)
    q = ((O.uniform_u32(N * K, 6 + K) % 255).astype(np.int64) - 127).astype(np.int8).reshape(N, K)
    s = O.normal(N, 7 + K, 0.0, 0.02)
    want = epilogue(trunc_act(A, 127) @ q.astype(np.int64).T, 127, s)
    np.testing.assert_array_equal(bits(O.gemv_q8(A, q, s, N, K)), bits(want))


@pytest.mark.parametrize("M,N,K", [(1, 7, 64), (3, 5, 30), (2, 16, 256)])
def test_q4_equals_int64_matmul_with_numpy_unpack(M, N, K):
    A = O.normal(M * K, 15 + K, 0.0, 3.0).reshape(M, K)
    q = (O.uniform_u32(N * K // 2, 16 + K) & 0xFF).astype(np.uint8).reshape(N, K // 2)
    s = O.normal(N, 17 + K, 0.0, 0.02)
    want = epilogue(trunc_act(A, 7) @ unpack_q4(q, N, K).T, 7, s)
    np.testing.assert_array_equal(bits(O.gemv_q4(A, q, s, N, K)), bits(want))


def test_q4_nibble_order_single_column():
    # weight nonzero only in column j: the output must equal trunc(7 x_j) * w_j
    N, K = 1, 8
    x = np.arange(1, K + 1, dtype=np.float32).reshape(1, K)
    s = np.ones(1, np.float32)
    for j in range(K):
        w = np.zeros(K, np.int64)
        w[j] = 3
        u = w + 8
        q = (u[0::2] | (u[1::2] << 4)).astype(np.uint8).reshape(1, K // 2)
        C = O.gemv_q4(x, q, s, N, K)
        assert C[0, 0] == np.float32(np.float32(7 * (j + 1) * 3) / np.float32(7))


def test_q4_odd_k_skips_last_high_nibble():
    # K odd: the high nibble of the last byte must not contribute, and row n
    # starts at byte n*(K//2) (rows overlap by one byte).
    N, K = 2, 5
    x = np.ones((1, K), np.float32)
    q = np.array([0x99, 0x99, 0xF9, 0x99, 0x99], np.uint8)  # row0 bytes 0..2, row1 bytes 2..4
    s = np.ones(N, np.float32)
    C = O.gemv_q4(x, q, s, N, K)
    # row 0: columns 0..4 use nibbles (9,9),(9,9),(9) -> w = 1 each, a = 7 -> 35
    # row 1: bytes 2..4: (9, F->skipped? no: byte2 lo=9 hi=F -> cols 0,1), byte3, byte4 lo
    assert C[0, 0] == np.float32(np.float32(35) / np.float32(7))
    want1 = 7 * 1 + 7 * 7 + 7 * 1 + 7 * 1 + 7 * 1
    assert C[0, 1] == np.float32(np.float32(want1) / np.float32(7))


def test_q8_column_permutation_invariance():
    M, N, K = 2, 9, 96
    A = O.normal(M * K, 31, 0.0, 2.0).reshape(M, K)
    q = ((O.uniform_u32(N * K, 32) % 255).astype(np.int64) - 127).astype(np.int8).reshape(N, K)
    s = O.normal(N, 33, 0.0, 0.05)
    perm = np.random.default_rng(0).permutation(K)
    a = O.gemv_q8(A, q, s, N, K)
    b = O.gemv_q8(A[:, perm], np.ascontiguousarray(q[:, perm]), s, N, K)
    np.testing.assert_array_equal(bits(a), bits(b))


def test_q8_truncation_edges_and_x86_conversion():
    assert O.orc().orc_f2i_trunc(2.9999998) == 2
    assert O.orc().orc_f2i_trunc(-2.9999998) == -2
    assert O.orc().orc_f2i_trunc(float("nan")) == -2**31
    assert O.orc().orc_f2i_trunc(3e9) == -2**31
    assert O.orc().orc_f2i_trunc(-2147483648.0) == -2**31
    assert O.orc().orc_f2i_trunc(2147483520.0) == 2147483520
    # a = trunc(x*127) is 0 for |x| < 1/127: such inputs contribute nothing
    K = 16
    x = np.full((1, K), 0.0078, np.float32)
    q = np.full((1, K), 100, np.int8)
    assert O.gemv_q8(x, q, np.ones(1, np.float32), 1, K)[0, 0] == 0.0


def test_topk_equals_stable_sort():
    rng = np.random.default_rng(3)
    for trial in range(200):
        E = int(rng.integers(8, 140))
        x = np.round(rng.normal(0, 2, E)).astype(np.float32)  # ties on purpose
        if trial % 5 == 0:
            x[rng.integers(0, E, 3)] = np.nan
        if trial % 7 == 0:
            x[rng.integers(0, E, 3)] = -np.inf
        idx, val = O.topk_desc(x, 8)
        valid = np.where(~np.isnan(x) & (x > -np.inf))[0]
        order = valid[np.argsort(-x[valid].astype(np.float64), kind="stable")][:8]
        want_idx = np.full(8, -1, np.int32)
        want_idx[: order.size] = order
        np.testing.assert_array_equal(idx, want_idx)
        want_val = np.full(8, -np.inf, np.float32)
        want_val[: order.size] = x[order]
        np.testing.assert_array_equal(val, want_val)


def test_softmax_topk_closed_form():
    for seed in range(20):
        v = np.sort(O.normal(8, 100 + seed, 0.0, 2.0))[::-1].copy()
        p = O.softmax_topk(v)
        e = np.exp(v.astype(np.float64) - v.max())
        want = e / (e.sum() + 1e-9)
        np.testing.assert_allclose(p, want, rtol=2e-6, atol=0)
        assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5


def test_silu_closed_form():
    x = O.normal(4000, 9, 0.0, 5.0)
    y = O.silu(x)
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(y, want, rtol=3e-7, atol=1e-37)


def test_rmsnorm_closed_form():
    x = O.normal(5 * 2048, 10, 0.0, 1.0).reshape(5, 2048)
    w = O.normal(2048, 11, 1.0, 0.1)
    y = O.rmsnorm(x, w)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-7)


def test_matmul_f32_error_bound():
    A = O.normal(3 * 2048, 12, 0.0, 1.0).reshape(3, 2048)
    W = O.normal(128 * 2048, 13, 0.0, 0.02).reshape(128, 2048)
    C = O.matmul_f32(A, W)
    exact = A.astype(np.float64) @ W.astype(np.float64).T
    bound = 2048 * 2.0 ** -24 * (np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T)
    assert np.all(np.abs(C - exact) <= bound)
    # and it is sequential: not equal to a pairwise (numpy float32) sum everywhere
    assert not np.array_equal(C, (A @ W.T).astype(np.float32))


def test_quantizers():
    W = O.normal(64 * 256, 14, 0.0, 0.02).reshape(64, 256)
    q8, s8 = O.quant_q8(W)
    amax = np.abs(W).max(axis=1)
    np.testing.assert_array_equal(s8, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q8).max(axis=1) == 127)
    err = np.abs(W - q8.astype(np.float32) * s8[:, None])
    assert np.all(err <= s8[:, None] * 0.5001)
    q4, s4 = O.quant_q4(W)
    u = unpack_q4(q4, 64, 256) + 8
    assert u.min() >= 0 and u.max() <= 15
    w4 = unpack_q4(q4, 64, 256)
    assert np.all(np.abs(w4).max(axis=1) >= 7)
    err4 = np.abs(W - w4.astype(np.float32) * s4[:, None])
    assert np.all(err4 <= s4[:, None] * 0.5001)
    # a zero row: scale clamps at 1e-8/127 and q is all zero
    Z = np.zeros((1, 8), np.float32)
    qz, sz = O.quant_q8(Z)
    assert not qz.any() and sz[0] == np.float32(np.float32(1e-8) / np.float32(127))


def _small_layer(dtype, T, seed, E=16, D=64, dff=32):
    ex = O.make_experts(dtype, E, D, dff, seed)
    x = O.normal(T * D, seed + 1, 0.0, 1.0).reshape(T, D)
    rw = O.normal(E * D, seed + 2, 0.0, 0.1).reshape(E, D)
    return ex, x, rw


@pytest.mark.parametrize("dtype", [2, 3])
def test_moe_rows_independent_and_residual(dtype):
    ex, x, rw = _small_layer(dtype, 5, 300 + dtype)
    out, idx, p, _ = O.moe_block(x, None, rw, None, ex)
    for t in range(5):
        o1, i1, p1, _ = O.moe_block(x[t:t + 1], None, rw, None, ex)
        np.testing.assert_array_equal(bits(o1[0]), bits(out[t]))
        np.testing.assert_array_equal(i1[0], idx[t])
    out_r, _, _, _ = O.moe_block(x, x, rw, None, ex)
    np.testing.assert_array_equal(bits(out_r), bits((x + out).astype(np.float32)))


@pytest.mark.parametrize("dtype", [2, 3])
def test_moe_equals_composition_of_gemvs(dtype):
    """MoE output == sum_j p_j * down(silu(gate x) * up x), built from the
    oracle's GEMVs, numpy's stable sort and float64-free float32 steps."""
    ex, x, rw = _small_layer(dtype, 2, 400 + dtype)
    out, idx, p, logits = O.moe_block(x, None, rw, None, ex)
    np.testing.assert_array_equal(bits(logits), bits(O.matmul_f32(x, rw)))
    g = O.gemv_q8 if dtype == 2 else O.gemv_q4
    for t in range(2):
        order = np.argsort(-logits[t].astype(np.float64), kind="stable")[:8]
        np.testing.assert_array_equal(idx[t], order)
        acc = np.zeros(64, np.float32)
        for j, e in enumerate(order):
            gg = g(x[t], ex.gq[e], ex.gs[e], 32, 64)[0]
            uu = g(x[t], ex.uq[e], ex.us[e], 32, 64)[0]
            h = (O.silu(gg) * uu).astype(np.float32)
            y = g(h, ex.dq[e], ex.ds[e], 64, 32)[0]
            acc = (acc + (p[t, j] * y).astype(np.float32)).astype(np.float32)
        np.testing.assert_array_equal(bits(acc), bits(out[t]))


def test_moe_dominant_expert():
    ex, x, rw = _small_layer(2, 1, 500)
    rb = np.zeros(16, np.float32)
    rb[11] = 100.0
    _, idx, p, _ = O.moe_block(x, None, rw, rb, ex)
    assert idx[0, 0] == 11
    assert p[0, 0] > 0.999999 and np.all(p[0, 1:] < 1e-20)


def test_quantizer_ties_round_half_even():
    """export.py rounds with torch.round, documented as round-half-to-even.
    Rows built so that fl(w / s) lands exactly on k + 0.5: the oracle must
    pick the even neighbour (a half-away-from-zero rounding would not)."""
    # amax 127 gives s = 1.0 exactly (Q8) and 7 gives s = 1.0 (Q4)
    row8 = np.array([127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 126.5], np.float32)
    q8, s8 = O.quant_q8(row8[None, :])
    assert s8[0] == 1.0
    assert q8[0].tolist() == [127, 2, -2, 4, -4, 0, 0, 126]
    row4 = np.array([7.0, 2.5, -2.5, 3.5, -6.5, 0.5, -0.5, 1.5], np.float32)
    q4, s4 = O.quant_q4(row4[None, :])
    assert s4[0] == 1.0
    w4 = unpack_q4(q4, 1, 8)[0].tolist()
    assert w4 == [7, 2, -2, 4, -6, 0, 0, 2]
