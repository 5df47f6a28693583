"""GPU parity of the rowwise Q8/Q4 GEMVs (kernels.c:51-181) through the C ABI.

Bar: bit-exact.  The integer dot is exact and the fp32 epilogue is a fixed
sequence of IEEE operations, so every output must equal the oracle's bits.
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def dev_gemv(M_, A, q, s, dtype, N, K):
    A = np.ascontiguousarray(A, np.float32).reshape(-1, K) if K > 0 else np.zeros((A.shape[0], 0), np.float32)
    Mr = A.shape[0]
    dA = M_.DeviceBuffer.from_array(A)
    dq = M_.DeviceBuffer.from_array(q)
    ds = M_.DeviceBuffer.from_array(s)
    dC = M_.DeviceBuffer(Mr * N * 4)
    fn = M_.lib().moe_matmul_q8_dev if dtype == 2 else M_.lib().moe_matmul_q4_dev
    M_.check(fn(dA.ptr, dq.ptr, ds.ptr, dC.ptr, Mr, N, K), "gemv")
    return dC.download((Mr, N), np.float32)


def test_config_shapes_bit_exact(moehip):
    with open(os.path.join(GOLD, "ref_config.json")) as f:
        cfg = json.load(f)
    for c in cfg["cases"]:
        if c["kind"] != "gemv":
            continue
        print("case", c["tag"], flush=True)
        W = O.normal(c["N"] * c["K"], c["seed_w"], 0.0, c["std_w"]).reshape(c["N"], c["K"])
        q, s = (O.quant_q8 if c["dtype"] == 2 else O.quant_q4)(W)
        x = O.normal(c["K"], c["seed_x"], 0.0, 1.0).reshape(1, c["K"])
        C = dev_gemv(moehip, x, q, s, c["dtype"], c["N"], c["K"])
        assert sha(C) == c["sha_C"], c["tag"]


GEMV_TAGS = ["q8_a", "q8_b", "q8_spec", "q4_a", "q4_odd", "q4_spec", "q4_b"]


@pytest.mark.parametrize("tag", GEMV_TAGS)
def test_golden_small_gemvs(moehip, tag):
    with np.load(os.path.join(GOLD, "ref_small.npz")) as z:
        dtype, M, N, K = (int(v) for v in z[f"gemv_{tag}_shape"])
        A, q, s, want = (z[f"gemv_{tag}_{k}"] for k in ("A", "q", "s", "C"))
    C = dev_gemv(moehip, A, q, s, dtype, N, K)
    np.testing.assert_array_equal(bits(C), bits(want))
    # and through the host-pointer drop-in
    C2 = moehip.matmul_adaptive(A, None, {"q": q, "s": s, "dtype": dtype}, N, K)
    np.testing.assert_array_equal(bits(C2), bits(want))


def test_drop_in_f32_and_unknown_dtype(moehip):
    with np.load(os.path.join(GOLD, "ref_small.npz")) as z:
        A, W, want, zero = z["gemv_f32_A"], z["gemv_f32_W"], z["gemv_f32_C"], z["gemv_dtype5_C"]
    C = moehip.matmul_adaptive(A, W, None, 3, 17)
    np.testing.assert_array_equal(bits(C), bits(want))
    q = np.ones((3, 17), np.int8)
    s = np.ones(3, np.float32)
    C = moehip.matmul_adaptive(A, None, {"q": q, "s": s, "dtype": 5}, 3, 17)
    np.testing.assert_array_equal(C, zero)


# every tiled variant (row bytes 384 .. 4096) and the generic path, M = 1..9,
# activation scales that need 1, 2 and 4 limbs
SHAPES = [
    (2, 768, 2048), (2, 2048, 768), (2, 100, 512), (2, 64, 384), (2, 33, 1024), (2, 40, 1536),
    (2, 24, 4096), (2, 17, 100), (2, 5, 7),
    (3, 2048, 768), (3, 768, 2048), (3, 70, 1024), (3, 50, 1536), (3, 64, 3072), (3, 40, 8192),
    (3, 30, 4096), (3, 9, 98), (3, 6, 9),
]


@pytest.mark.parametrize("dtype,N,K", SHAPES)
@pytest.mark.parametrize("M,scale", [(1, 1.0), (3, 30.0), (5, 0.05), (9, 1e5)])
def test_shape_sweep(moehip, dtype, N, K, M, scale):
    seed = dtype * 100000 + N * 31 + K * 7 + M
    A = O.normal(M * K, seed, 0.0, scale).reshape(M, K)
    if dtype == 2:
        q = (O.uniform_u32(N * K, seed + 1) & 0xFF).astype(np.uint8).view(np.int8).reshape(N, K)
        want = O.gemv_q8(A, q, O.normal(N, seed + 2, 0.0, 0.01), N, K)
    else:
        q = (O.uniform_u32(N * (K // 2) + (K & 1), seed + 1) & 0xFF).astype(np.uint8)
        want = O.gemv_q4(A, q, O.normal(N, seed + 2, 0.0, 0.01), N, K)
    C = dev_gemv(moehip, A, q, O.normal(N, seed + 2, 0.0, 0.01), dtype, N, K)
    np.testing.assert_array_equal(bits(C), bits(want))


def test_batched_jobs(moehip):
    for dtype, N, K in [(2, 768, 2048), (3, 2048, 768), (3, 768, 2048), (2, 2048, 768)]:
        nj, M = 6, 2
        qs, ss, As, wants = [], [], [], []
        for j in range(nj):
            W = O.normal(N * K, 500 + j + dtype, 0.0, 0.02).reshape(N, K)
            q, s = (O.quant_q8 if dtype == 2 else O.quant_q4)(W)
            A = O.normal(M * K, 600 + j, 0.0, 1.0).reshape(M, K)
            qs.append(q); ss.append(s); As.append(A)
            wants.append((O.gemv_q8 if dtype == 2 else O.gemv_q4)(A, q, s, N, K))
        bufs = []
        jobs = (moehip.QJob * nj)()
        outs = []
        for j in range(nj):
            dq = moehip.DeviceBuffer.from_array(qs[j]); ds = moehip.DeviceBuffer.from_array(ss[j])
            dA = moehip.DeviceBuffer.from_array(As[j]); dC = moehip.DeviceBuffer(M * N * 4)
            bufs += [dq, ds, dA]
            outs.append(dC)
            jobs[j] = moehip.QJob(dq.ptr, ds.ptr, dA.ptr, dC.ptr)
        djobs = moehip.DeviceBuffer(ctypes.sizeof(jobs))
        moehip.check(moehip.lib().moe_memcpy_h2d(djobs.ptr, ctypes.addressof(jobs), ctypes.sizeof(jobs)))
        moehip.check(moehip.lib().moe_matmul_q_batched_dev(dtype, djobs.ptr, nj, M, N, K), "batched")
        for j in range(nj):
            np.testing.assert_array_equal(bits(outs[j].download((M, N), np.float32)), bits(wants[j]))


def test_variant_selection(moehip):
    assert moehip.gemv_variant(2, 1, 768, 2048).startswith("tiled")
    assert moehip.gemv_variant(3, 1, 2048, 768).startswith("tiled")
    assert moehip.gemv_variant(3, 1, 768, 2048).startswith("tiled")
    assert moehip.gemv_variant(3, 1, 4, 9) == "generic"


@pytest.mark.parametrize("dtype,N,K,M,scale", [(2, 768, 2048, 1, 1.0), (3, 2048, 768, 3, 1.0),
                                               (3, 768, 2048, 5, 40.0), (2, 512, 1024, 2, 400.0),
                                               # one token: the flat stream over all jobs' rows
                                               (3, 2048, 768, 1, 1.0), (3, 768, 2048, 1, 1.0),
                                               (3, 100, 768, 1, 40.0), (2, 77, 2048, 1, 400.0),
                                               (3, 13, 4096, 1, 3000.0)])
def test_prepacked_matches_oracle(moehip, dtype, N, K, M, scale):
    """Pack once, run several products from the same tables.  scale 40 / 400
    pushes Q4 / Q8 activations into the 2- and 4-byte limb ranges (3000:
    4-limb Q4, the exact fallback)."""
    L = moehip.lib()
    nj = 3 if M > 1 else 7
    A = O.normal(M * K, 900 + M, 0.0, scale).reshape(M, K)
    dA = moehip.DeviceBuffer.from_array(A)
    tb = L.moe_act_table_bytes(K)
    assert tb % 16 == 0 and tb >= 16 + K
    tabs = moehip.DeviceBuffer(tb * M)
    moehip.check(L.moe_act_pack_dev(dtype, dA.ptr, M, K, tabs.ptr), "pack")
    jobs = (moehip.QJob * nj)()
    keep, outs, wants = [], [], []
    for j in range(nj):
        W = O.normal(N * K, 910 + j, 0.0, 0.02).reshape(N, K)
        q, s = (O.quant_q8 if dtype == 2 else O.quant_q4)(W)
        wants.append((O.gemv_q8 if dtype == 2 else O.gemv_q4)(A, q, s, N, K))
        dq, ds, dC = (moehip.DeviceBuffer.from_array(q), moehip.DeviceBuffer.from_array(s),
                      moehip.DeviceBuffer(M * N * 4))
        keep += [dq, ds]
        outs.append(dC)
        jobs[j] = moehip.QJob(dq.ptr, ds.ptr, dA.ptr, dC.ptr)
    djobs = moehip.DeviceBuffer(ctypes.sizeof(jobs))
    moehip.check(L.moe_memcpy_h2d(djobs.ptr, ctypes.addressof(jobs), ctypes.sizeof(jobs)))
    moehip.check(L.moe_matmul_q_prepacked_dev(dtype, djobs.ptr, nj, M, N, K, tabs.ptr), "prepacked")
    for j in range(nj):
        np.testing.assert_array_equal(bits(outs[j].download((M, N), np.float32)), bits(wants[j]))


def test_prepacked_rejects_untiled_shapes(moehip):
    L = moehip.lib()
    buf = moehip.DeviceBuffer(4096)
    assert L.moe_act_pack_dev(3, buf.ptr, 1, 9, buf.ptr) != 0        # odd Q4 K
    assert L.moe_matmul_q_prepacked_dev(2, buf.ptr, 1, 1, 4, 100, buf.ptr) != 0
    assert b"tiled" in L.moe_last_error()
    assert L.moe_act_pack_dev(2, buf.ptr, 1, 2048, buf.ptr + 4) != 0  # misaligned tables


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, 3 * (1 << 20) + 48, 64 << 20])
def test_stream_read_ceiling_kernel(moehip, nbytes):
    """The plain read-only stream that bench.py times beside the GEMV reads
    every word once: the XOR of all 32-bit words it folds into the sink
    equals the host's, for spans that split unevenly over the blocks and
    threads."""
    M_ = moehip
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    d = M_.DeviceBuffer.from_array(words)
    sink = M_.DeviceBuffer(16)
    M_.check(M_.lib().moe_memset(sink.ptr, 0, 16), "memset")
    M_.check(M_.lib().moe_stream_read_dev(d.ptr, nbytes, sink.ptr), "stream read")
    got = int(sink.download((4,), np.uint32)[0])
    assert got == int(np.bitwise_xor.reduce(words))
    # sizes that are not whole 16-byte words are rejected
    assert M_.lib().moe_stream_read_dev(d.ptr, nbytes - 4, sink.ptr) != 0


@pytest.mark.parametrize("dtype,N,K,nj", [(3, 2048, 768, 1366), (3, 768, 2048, 5), (2, 768, 2048, 683),
                                          (3, 100, 768, 3), (2, 77, 2048, 9)])
def test_rows_read_reads_every_word_once(moehip, dtype, N, K, nj):
    """moe_rows_read_dev (the GEMV launch's reads without its arithmetic,
    bench.py's read ceiling) reads every weight word and every scale exactly
    once: the XOR it folds into the sink equals the host's XOR of the pool
    (a word read twice or skipped would change it).  Job counts include the
    bench pools' (1366 and 683: 256 / 128-row blocks, 8 row groups a wave)
    and row counts that leave partial row groups."""
    L = moehip.lib()
    rb = K if dtype == 2 else K // 2
    rng = np.random.default_rng(N * 7 + nj)
    q = rng.integers(0, 2**32, size=nj * N * rb // 4, dtype=np.uint32)
    s = rng.integers(0, 2**32, size=nj * N, dtype=np.uint32)
    dq, ds = moehip.DeviceBuffer.from_array(q), moehip.DeviceBuffer.from_array(s)
    jobs = (moehip.QJob * nj)()
    for j in range(nj):
        jobs[j] = moehip.QJob(dq.ptr + j * N * rb, ds.ptr + j * N * 4, None, None)
    djobs = moehip.DeviceBuffer(ctypes.sizeof(jobs))
    moehip.check(L.moe_memcpy_h2d(djobs.ptr, ctypes.addressof(jobs), ctypes.sizeof(jobs)))
    sink = moehip.DeviceBuffer(16)
    want = int(np.bitwise_xor.reduce(q) ^ np.bitwise_xor.reduce(s))
    for cap in (0, 1, 3, 8):   # the GEMV's own blocks-per-CU cap, and others
        moehip.check(L.moe_memset(sink.ptr, 0, 16), "memset")
        moehip.check(L.moe_rows_read_dev(dtype, djobs.ptr, nj, N, K, cap, sink.ptr), "rows read")
        assert int(np.bitwise_xor.reduce(sink.download((4,), np.uint32))) == want, f"cap {cap}"
    assert L.moe_rows_read_dev(dtype, djobs.ptr, nj, N, 100, 0, sink.ptr) != 0   # no tiled geometry
    assert L.moe_rows_read_dev(dtype, djobs.ptr, nj, N, K, 9, sink.ptr) != 0     # cap out of range
