#!/usr/bin/env python3
"""make_golden.py - writes tests/golden/ fixtures from the compiled reference.

Runs in the build container only: it needs oracle/_ref/ (the reference's
kernels.c and test_model_trace.c compiled from /root/reference by
``make -C oracle ref``).  Inputs come from the seeded generator of
oracle/moe_oracle.c; expected outputs come from the REFERENCE code, never from
the restatement, so the fixtures pin the restatement (tests/test_oracle_*.py)
and through it the GPU path.

Small cases store full inputs and outputs (ref_small.npz).  Cases at the
BASELINE.json shapes store seeds, SHA-256 digests of the inputs and outputs and
a sample of output values (ref_config.json), regenerated at test time.

Tiny whole models (ref_model.json) store the model's seeds and keyword set,
the prompt, the reference's greedy continuation and a digest of every step's
logits (``--model`` writes only this file).

Usage:  python tests/golden/make_golden.py [--model]
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

OUT_DIR = os.path.dirname(os.path.abspath(__file__))


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref_adaptive(A, W_fp32, q, s, dtype, M, N, K):
    """Reference kernels.c matmul_adaptive on host arrays."""
    C = np.full((M, N), np.nan, dtype=np.float32)
    if q is None:
        O.ref_kernels().matmul_adaptive(A.ctypes.data, W_fp32.ctypes.data, None, C.ctypes.data,
                                        M, N, K)
    else:
        qw = O.QW(q.ctypes.data, s.ctypes.data, N, K, dtype)
        O.ref_kernels().matmul_adaptive(A.ctypes.data, None, ctypes.addressof(qw), C.ctypes.data,
                                        M, N, K)
    return C


def special_activations(n: int, seed: int) -> np.ndarray:
    """Activations that exercise the truncation and the limb ranges."""
    base = O.normal(n, seed, 0.0, 1.0)
    extras = np.array([0.0, -0.0, 1.0, -1.0, 0.9999999, -0.9999999, 2.0 / 127.0,
                       1.0 / 127.0 - 1e-9, 300.0, -300.0, 16000.0, -16000.0, 1e6, -1e6,
                       3e7, -3e7, 1e10, -1e10, np.inf, -np.inf, np.nan,
                       18.2857, -18.2857, 18.3, 257.0, -259.0, 0.5 / 127.0, 1e-30],
                      dtype=np.float32)
    out = base.copy()
    out[: min(n, extras.size)] = extras[: min(n, extras.size)]
    return out


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref not built: run `make -C oracle ref` (needs /root/reference)")
    rt = O.ref_trace()
    small = {}

    # ---- a1/a2/a3: GEMVs at tiny shapes, incl. odd K and special values ----
    for tag, dtype, M, N, K, seed in [
        ("q8_a", 2, 3, 5, 7, 11), ("q8_b", 2, 2, 9, 64, 12), ("q8_spec", 2, 2, 4, 33, 13),
        ("q4_a", 3, 2, 4, 10, 21), ("q4_odd", 3, 2, 4, 9, 22), ("q4_spec", 3, 2, 5, 34, 23),
        ("q4_b", 3, 3, 7, 96, 24),
    ]:
        if tag.endswith("spec"):
            A = special_activations(M * K, seed).reshape(M, K)
        else:
            A = O.normal(M * K, seed, 0.0, 1.5).reshape(M, K)
        if dtype == 2:
            q = (O.uniform_u32(N * K, seed + 100) % 255).astype(np.int32) - 127
            q = q.astype(np.int8).reshape(N, K)
            q[0, 0] = -128  # the int8 minimum is legal input for the kernel
        else:
            # row stride K//2; an odd K reads one byte past N*(K//2)
            nbytes = N * (K // 2) + (K & 1)
            q = (O.uniform_u32(nbytes, seed + 100) & 0xFF).astype(np.uint8)
        s = O.normal(N, seed + 200, 0.0, 0.01)
        C = ref_adaptive(A, None, q, s, dtype, M, N, K)
        small[f"gemv_{tag}_A"] = A
        small[f"gemv_{tag}_q"] = q
        small[f"gemv_{tag}_s"] = s
        small[f"gemv_{tag}_C"] = C
        small[f"gemv_{tag}_shape"] = np.array([dtype, M, N, K], np.int32)

    # fp32 path and the unknown-dtype zero fill
    A = O.normal(2 * 17, 31, 0.0, 1.0).reshape(2, 17)
    W = O.normal(3 * 17, 32, 0.0, 0.5).reshape(3, 17)
    small["gemv_f32_A"], small["gemv_f32_W"] = A, W
    small["gemv_f32_C"] = ref_adaptive(A, W, None, None, 0, 2, 3, 17)
    q = np.ones((3, 17), np.int8)
    s = np.ones(3, np.float32)
    small["gemv_dtype5_C"] = ref_adaptive(A, None, q, s, 5, 2, 3, 17)

    # ---- a7: top-k known answers ----
    topk_cases = [
        np.array([0.5, 0.5, 0.5, 0.1, 0.9, 0.5, 0.9, -1.0, 0.5, 0.5, 0.3], np.float32),
        np.array([np.nan, 1.0, np.nan, 2.0, -np.inf, 0.0, -0.0, 3.0, np.inf, 1.0], np.float32),
        np.array([-np.inf, np.nan, 1.0, -np.inf, 2.0, np.nan, -np.inf, -np.inf, 0.5], np.float32),
        np.array([0.0, -0.0, 0.0, -0.0, 0.0, -0.0, 0.0, -0.0, 0.0, -0.0], np.float32),
        O.normal(128, 41, 0.0, 1.0),
        np.round(O.normal(128, 42, 0.0, 2.0)).astype(np.float32),  # many exact ties
    ]
    for i, v in enumerate(topk_cases):
        idx = np.empty(8, np.int32)
        val = np.empty(8, np.float32)
        rt.ref_topk_desc(v.ctypes.data, v.size, 8, idx.ctypes.data, val.ctypes.data)
        small[f"topk_{i}_x"], small[f"topk_{i}_idx"], small[f"topk_{i}_val"] = v, idx, val

    # ---- a8/a9: softmax rows and SiLU over interesting values ----
    sx = np.concatenate([O.normal(200, 51, 0.0, 4.0),
                         np.array([0.0, -0.0, 88.0, -88.0, 89.0, -104.0, -103.9, 1e-30, -1e-30,
                                   20.0, -20.0, np.inf, -np.inf], np.float32)]).astype(np.float32)
    sy = sx.copy()
    rt.ref_silu(sy.ctypes.data, sy.size)
    small["silu_x"], small["silu_y"] = sx, sy
    sm = O.normal(4 * 8, 52, 0.0, 3.0).reshape(4, 8)
    smo = sm.copy()
    rt.ref_softmax_rows(smo.ctypes.data, 4, 8)
    small["softmax_x"], small["softmax_y"] = sm, smo

    # ---- a12: rmsnorm ----
    x = O.normal(3 * 48, 61, 0.0, 2.0).reshape(3, 48)
    w = O.normal(48, 62, 1.0, 0.1)
    y = np.empty_like(x)
    rt.ref_rmsnorm(x.ctypes.data, w.ctypes.data, 3, 48, 1e-6, y.ctypes.data)
    small["rms_x"], small["rms_w"], small["rms_y"] = x, w, y
    y1 = np.empty_like(x)
    rt.ref_rmsnorm(x.ctypes.data, None, 3, 48, 1e-6, y1.ctypes.data)
    small["rms_y_now"] = y1

    # ---- a6-a13: whole MoE layer (norm2 + router + experts + residual) ----
    for tag, dtype, T, D, dff, E, bias, seed in [
        ("q8", 2, 3, 64, 32, 16, False, 71), ("q4", 3, 4, 64, 32, 16, True, 72),
    ]:
        ex = O.make_experts(dtype, E, D, dff, seed)
        x = O.normal(T * D, seed + 1, 0.0, 1.0).reshape(T, D)
        rw = O.normal(E * D, seed + 2, 0.0, 0.1).reshape(E, D)
        rms2 = O.normal(D, seed + 3, 1.0, 0.05)
        rb = O.normal(E, seed + 4, 0.0, 0.1) if bias else None
        xo = x.copy()
        rt.ref_moe_layer(xo.ctypes.data, T, D, E, 8, dff, rms2.ctypes.data, rw.ctypes.data,
                         None if rb is None else rb.ctypes.data,
                         ctypes.addressof(ex.Wg), ctypes.addressof(ex.Wu), ctypes.addressof(ex.Wd))
        pre = f"layer_{tag}_"
        small[pre + "x"], small[pre + "rw"], small[pre + "rms2"], small[pre + "out"] = x, rw, rms2, xo
        if rb is not None:
            small[pre + "rb"] = rb
        small[pre + "gq"], small[pre + "gs"] = ex.gq, ex.gs
        small[pre + "uq"], small[pre + "us"] = ex.uq, ex.us
        small[pre + "dq"], small[pre + "ds"] = ex.dq, ex.ds
        small[pre + "dims"] = np.array([dtype, T, D, dff, E], np.int32)

    np.savez_compressed(os.path.join(OUT_DIR, "ref_small.npz"), **small)

    # ---- BASELINE.json shapes: digests + samples ----
    cfg = {"generator": "orc_fill_normal (splitmix64 -> xoshiro256** -> Box-Muller)",
           "cases": []}
    for tag, dtype, N, K, sw, sx_ in [("q8_768x2048", 2, 768, 2048, 1001, 1002),
                                      ("q4_2048x768", 3, 2048, 768, 1003, 1004),
                                      ("q4_768x2048", 3, 768, 2048, 1005, 1006)]:
        W = O.normal(N * K, sw, 0.0, 0.02).reshape(N, K)
        q, s = (O.quant_q8 if dtype == 2 else O.quant_q4)(W)
        x = O.normal(K, sx_, 0.0, 1.0).reshape(1, K)
        C = ref_adaptive(x, None, q, s, dtype, 1, N, K)
        pick = np.linspace(0, N - 1, 16).astype(int)
        cfg["cases"].append({"kind": "gemv", "tag": tag, "dtype": dtype, "N": N, "K": K,
                             "seed_w": sw, "seed_x": sx_, "std_w": 0.02,
                             "sha_w": sha(W), "sha_q": sha(q), "sha_s": sha(s), "sha_x": sha(x),
                             "sha_C": sha(C), "pick": pick.tolist(),
                             "C_pick": [float(v) for v in C[0, pick]]})
    # layers at the real shape: decode (Q8 T=4, Q4 T=2) and multi-token
    # (Q8 T=64, Q4 T=128: the expert-major kernels)
    for tag, dtype, T, seed in [("layer_q8_T4", 2, 4, 2001), ("layer_q4_T2", 3, 2, 2002),
                                ("layer_q8_T64", 2, 64, 2004), ("layer_q4_T128", 3, 128, 2003)]:
        D, dff, E = 2048, 768, 128
        ex = O.make_experts(dtype, E, D, dff, seed)
        x = O.normal(T * D, seed + 1, 0.0, 1.0).reshape(T, D)
        rw = O.normal(E * D, seed + 2, 0.0, 0.02).reshape(E, D)
        rms2 = np.ones(D, np.float32)
        xo = x.copy()
        rt.ref_moe_layer(xo.ctypes.data, T, D, E, 8, dff, rms2.ctypes.data, rw.ctypes.data, None,
                         ctypes.addressof(ex.Wg), ctypes.addressof(ex.Wu), ctypes.addressof(ex.Wd))
        pick = np.linspace(0, T * D - 1, 32).astype(int)
        cfg["cases"].append({"kind": "layer", "tag": tag, "dtype": dtype, "T": T, "D": D,
                             "d_ff": dff, "E": E, "seed": seed, "std_w": 0.02,
                             "sha_gq": sha(ex.gq), "sha_dq": sha(ex.dq), "sha_x": sha(x),
                             "sha_rw": sha(rw), "sha_out": sha(xo), "pick": pick.tolist(),
                             "out_pick": [float(v) for v in xo.reshape(-1)[pick]]})
    with open(os.path.join(OUT_DIR, "ref_config.json"), "w") as f:
        json.dump(cfg, f, indent=1)
    print("wrote", os.path.join(OUT_DIR, "ref_small.npz"), "and ref_config.json")
    model_fixtures()


# Tiny whole models (oracle.TinyModel keyword sets) for ref_model.json: the
# reference's model_forward_f32 (test_model_trace.c:526-579) on a QW3W file
# written by moe.cc_amd/qw3w.py, greedy over a growing sequence.
MODEL_CASES = [
    ("q4_small", dict(dtype=3, seed=11), 6, 5),
    ("q8_bias_tied", dict(dtype=2, seed=12, bias=True, untied=False), 4, 4),
    ("q4_norms_L3", dict(dtype=3, seed=13, random_norms=True, L=3, D=128, hd=32, nq=4, nkv=2,
                         dff=64, E=16, V=211), 9, 4),
]


def model_fixtures():
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "moe.cc_amd"))
    import qw3w
    rt = O.ref_trace()
    out = {"generator": "oracle.TinyModel (orc_fill_normal seeds), written with qw3w.write",
           "cases": []}
    with tempfile.TemporaryDirectory() as d:
        for tag, kw, n_prompt, steps in MODEL_CASES:
            m = O.TinyModel(**kw)
            path = os.path.join(d, tag + ".bin")
            qw3w.write(path, qw3w.model_entries(m))
            seq = [int(v) for v in (O.uniform_u32(n_prompt, 500 + len(tag)) % m.V)]
            prompt = list(seq)
            logits_sha, picks, choices = [], [], []
            for _ in range(steps + 1):
                ids = np.array(seq, np.int32)
                lg = np.empty(m.V, np.float32)
                assert rt.ref_model_forward_file(path.encode(), ids.ctypes.data, ids.size,
                                                 lg.ctypes.data, m.V) == m.V
                logits_sha.append(sha(lg))
                picks.append([float(v) for v in lg[:8]])
                nxt = int(O.greedy(lg))
                choices.append(nxt)
                seq.append(nxt)
            out["cases"].append({"tag": tag, "model": kw, "prompt": prompt,
                                 "greedy": choices, "logits_sha": logits_sha,
                                 "logits_first8": picks})
    with open(os.path.join(OUT_DIR, "ref_model.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", os.path.join(OUT_DIR, "ref_model.json"))


if __name__ == "__main__":
    if sys.argv[1:] == ["--model"]:
        model_fixtures()
    else:
        main()
