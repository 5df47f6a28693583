"""The C ABI from a compiled C caller (tests/c_caller/moe_caller.c): model.h
QuantizedWeight arrays, matmul_adaptive with host pointers as
test_model_trace.c:496-503 calls it, and moe_layer_create /
moe_layer_forward from QwenConfig / QwenLayerWeights (model.h:9-58).  The
program is plain C built with gcc against include/moehip.h and -lmoehip;
its outputs are compared bit for bit with the oracle."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
CALLER_DIR = os.path.join(HERE, "c_caller")
CALLER = os.path.join(CALLER_DIR, "moe_caller")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _caller():
    if not os.path.exists(CALLER):
        subprocess.run(["make", "-C", CALLER_DIR], check=True)
    return CALLER


@pytest.mark.parametrize("dtype,T", [(2, 3), (3, 5)])
def test_c_caller_matches_oracle(tmp_path, dtype, T):
    D, dff, E, topk = 256, 128, 16, 8
    print("c caller case", dtype, T, flush=True)
    ex = O.make_experts(dtype, E, D, dff, 70 + dtype)
    rw = O.normal(E * D, 71, 0.0, 0.05).reshape(E, D)
    x = O.normal(T * D, 72 + T, 0.0, 1.0).reshape(T, D)
    inp = tmp_path / "in.bin"
    with open(inp, "wb") as f:
        f.write(np.array([dtype, D, dff, E, topk, T], np.int32).tobytes())
        for a in (rw, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds, x):
            f.write(np.ascontiguousarray(a).tobytes())
    out = tmp_path / "out.bin"
    r = subprocess.run([_caller(), str(inp), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    raw = out.read_bytes()
    o = 0

    def take(n, dt):
        nonlocal o
        a = np.frombuffer(raw, dt, n, o)
        o += a.nbytes
        return a

    gemv = O.gemv_q8 if dtype == 2 else O.gemv_q4
    y_gate = take(dff, np.float32)
    y_down = take(D, np.float32)
    y_router = take(E, np.float32)
    y_zero = take(4, np.float32)
    lay = take(T * D, np.float32).reshape(T, D)
    idx = take(T * topk, np.int32).reshape(T, topk)
    p = take(T * topk, np.float32).reshape(T, topk)
    assert o == len(raw)
    np.testing.assert_array_equal(bits(y_gate), bits(gemv(x[0], ex.gq[0], ex.gs[0], dff, D)[0]))
    np.testing.assert_array_equal(bits(y_down), bits(gemv(x[0, :dff], ex.dq[1], ex.ds[1], D, dff)[0]))
    np.testing.assert_array_equal(bits(y_router), bits(O.matmul_f32(x[:1], rw)[0]))
    assert not y_zero.any()
    want, widx, wp, _ = O.moe_block(x, x, rw, None, ex)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(lay), bits(want))
