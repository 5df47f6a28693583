"""The C restatement (oracle/) reproduces the compiled reference bit for bit.

Expected values in tests/golden/ were written by tests/golden/make_golden.py
from the reference's own kernels.c and test_model_trace.c compiled in place;
here only the restatement runs.  CPU only.
"""
import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def small():
    with np.load(os.path.join(GOLD, "ref_small.npz")) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def cfg():
    with open(os.path.join(GOLD, "ref_config.json")) as f:
        return json.load(f)


GEMV_TAGS = ["q8_a", "q8_b", "q8_spec", "q4_a", "q4_odd", "q4_spec", "q4_b"]


@pytest.mark.parametrize("tag", GEMV_TAGS)
def test_gemv_small(small, tag):
    dtype, M, N, K = (int(v) for v in small[f"gemv_{tag}_shape"])
    A, q, s = small[f"gemv_{tag}_A"], small[f"gemv_{tag}_q"], small[f"gemv_{tag}_s"]
    C = (O.gemv_q8 if dtype == 2 else O.gemv_q4)(A, q, s, N, K)
    np.testing.assert_array_equal(bits(C), bits(small[f"gemv_{tag}_C"]))


def test_f32_and_unknown_dtype(small):
    C = O.matmul_f32(small["gemv_f32_A"], small["gemv_f32_W"])
    np.testing.assert_array_equal(bits(C), bits(small["gemv_f32_C"]))
    assert not np.any(small["gemv_dtype5_C"])  # reference zero-fills (kernels.c:172-179)
    A = small["gemv_f32_A"]
    q = np.ones((3, 17), np.int8)
    s = np.ones(3, np.float32)
    C = np.full((2, 3), 7.0, np.float32)
    qw = O.QW(q.ctypes.data, s.ctypes.data, 3, 17, 5)
    O.orc().orc_matmul_adaptive(A.ctypes.data, None, ctypes.addressof(qw), C.ctypes.data, 2, 3, 17)
    np.testing.assert_array_equal(C, small["gemv_dtype5_C"])


@pytest.mark.parametrize("i", range(6))
def test_topk_known_answers(small, i):
    idx, val = O.topk_desc(small[f"topk_{i}_x"], 8)
    np.testing.assert_array_equal(idx, small[f"topk_{i}_idx"])
    np.testing.assert_array_equal(bits(val), bits(small[f"topk_{i}_val"]))


def test_silu(small):
    y = O.silu(small["silu_x"])
    np.testing.assert_array_equal(bits(y), bits(small["silu_y"]))


def test_softmax_topk(small):
    for r in range(small["softmax_x"].shape[0]):
        y = O.softmax_topk(small["softmax_x"][r])
        np.testing.assert_array_equal(bits(y), bits(small["softmax_y"][r]))


def test_rmsnorm(small):
    y = O.rmsnorm(small["rms_x"], small["rms_w"])
    np.testing.assert_array_equal(bits(y), bits(small["rms_y"]))
    y = O.rmsnorm(small["rms_x"], None)
    np.testing.assert_array_equal(bits(y), bits(small["rms_y_now"]))


def _experts_from(small, pre, dtype, D, dff):
    return O.ExpertSet(dtype, small[pre + "gq"], small[pre + "gs"], small[pre + "uq"],
                       small[pre + "us"], small[pre + "dq"], small[pre + "ds"], D, dff)


@pytest.mark.parametrize("tag", ["q8", "q4"])
def test_moe_layer_small(small, tag):
    pre = f"layer_{tag}_"
    dtype, T, D, dff, E = (int(v) for v in small[pre + "dims"])
    ex = _experts_from(small, pre, dtype, D, dff)
    x = small[pre + "x"]
    xn = O.rmsnorm(x, small[pre + "rms2"])
    out, idx, p, _ = O.moe_block(xn, x, small[pre + "rw"], small.get(pre + "rb"), ex)
    np.testing.assert_array_equal(bits(out), bits(small[pre + "out"]))


def _gemv_case(c):
    W = O.normal(c["N"] * c["K"], c["seed_w"], 0.0, c["std_w"]).reshape(c["N"], c["K"])
    assert sha(W) == c["sha_w"], "seeded generator drifted"
    q, s = (O.quant_q8 if c["dtype"] == 2 else O.quant_q4)(W)
    x = O.normal(c["K"], c["seed_x"], 0.0, 1.0).reshape(1, c["K"])
    assert sha(x) == c["sha_x"]
    return q, s, x


def test_config_gemvs(cfg):
    for c in cfg["cases"]:
        if c["kind"] != "gemv":
            continue
        q, s, x = _gemv_case(c)
        assert sha(q) == c["sha_q"] and sha(s) == c["sha_s"], c["tag"]
        C = (O.gemv_q8 if c["dtype"] == 2 else O.gemv_q4)(x, q, s, c["N"], c["K"])
        assert sha(C) == c["sha_C"], c["tag"]
        np.testing.assert_array_equal(C[0, c["pick"]], np.array(c["C_pick"], np.float32))


@pytest.mark.parametrize("tag", ["layer_q8_T4", "layer_q4_T2", "layer_q8_T64", "layer_q4_T128"])
def test_config_layers(cfg, tag):
    c = next(c for c in cfg["cases"] if c["tag"] == tag)
    ex = O.make_experts(c["dtype"], c["E"], c["D"], c["d_ff"], c["seed"], c["std_w"])
    assert sha(ex.gq) == c["sha_gq"] and sha(ex.dq) == c["sha_dq"]
    T, D = c["T"], c["D"]
    x = O.normal(T * D, c["seed"] + 1, 0.0, 1.0).reshape(T, D)
    rw = O.normal(c["E"] * D, c["seed"] + 2, 0.0, c["std_w"]).reshape(c["E"], D)
    assert sha(x) == c["sha_x"] and sha(rw) == c["sha_rw"]
    xn = O.rmsnorm(x, np.ones(D, np.float32))
    out, _, _, _ = O.moe_block(xn, x, rw, None, ex)
    assert sha(out) == c["sha_out"]
    np.testing.assert_array_equal(out.reshape(-1)[c["pick"]], np.array(c["out_pick"], np.float32))
