"""The -fopenmp build of the oracle (liboracle_omp.so) against the
single-thread build (liboracle.so), bit for bit.

The threaded build hands whole output rows (GEMV and fp32 product rows),
whole tokens (the MoE block after the router) or whole heads (attention) to
threads; each row is still computed in the reference's order, so its
results must equal the single-thread oracle's exactly.  Its users are the
all-cores CPU baseline of bench.py and the full-shape GPU checks, so this
equality is what lets them stand in for the single-thread restatement.
"""
import numpy as np

import oracle as O


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _both(fn):
    single = fn()
    with O.threaded():
        assert O.orc() is O.orc_omp()
        multi = fn()
    return single, multi


def test_omp_build_is_threaded():
    assert O.orc_single().orc_threads() == 1
    assert O.orc_omp().orc_threads() >= 1


def test_omp_products_equal():
    A = O.normal(3 * 2048, 1, 0.0, 1.0).reshape(3, 2048)
    W = O.normal(768 * 2048, 2, 0.0, 0.02).reshape(768, 2048)
    q8, s8 = O.quant_q8(W)
    q4, s4 = O.quant_q4(W)
    for f in (lambda: O.gemv_q8(A, q8, s8, 768, 2048), lambda: O.gemv_q4(A, q4, s4, 768, 2048),
              lambda: O.matmul_f32(A, W)):
        a, b = _both(f)
        np.testing.assert_array_equal(bits(a), bits(b))


def test_omp_moe_block_equal():
    D, dff, E, T = 256, 128, 16, 9
    ex = O.make_experts(3, E, D, dff, 5)
    x = O.normal(T * D, 6, 0.0, 1.0).reshape(T, D)
    rw = O.normal(E * D, 7, 0.0, 0.05).reshape(E, D)
    (o1, i1, p1, l1), (o2, i2, p2, l2) = _both(lambda: O.moe_block(x, x, rw, None, ex))
    np.testing.assert_array_equal(i1, i2)
    for a, b in ((o1, o2), (p1, p2), (l1, l2)):
        np.testing.assert_array_equal(bits(a), bits(b))


def test_omp_model_forward_equal():
    tm = O.TinyModel(D=128, L=2, hd=32, nq=8, nkv=2, dff=64, E=16, V=200, dtype=3, seed=9)
    ids = (O.uniform_u32(40, 3) % tm.V).astype(np.int32)

    def run():
        cache = tm.new_cache(48)
        out = [tm.forward_kv(ids[:37], 0, cache)]
        for i in range(3):
            out.append(tm.forward_kv(ids[37 + i:38 + i], 37 + i, cache))
        return np.stack(out)

    a, b = _both(run)
    np.testing.assert_array_equal(bits(a), bits(b))
