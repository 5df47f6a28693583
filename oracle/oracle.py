"""oracle.py - ctypes wrapper of liboracle.so, the CPU restatement of moe.cc's
quantized expert path (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product (moe.cc_amd/).

Also loads, when present, the compiled reference (oracle/_ref/, built from
/root/reference by ``make -C oracle ref`` in the build container) so that
tests can compare the restatement with the original code.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(_HERE, "liboracle.so")
REF_KERNELS_LIB = os.path.join(_HERE, "_ref", "libref_kernels.so")
REF_TRACE_LIB = os.path.join(_HERE, "_ref", "libref_trace.so")

_P = ctypes.c_void_p
_I = ctypes.c_int


class QW(ctypes.Structure):
    """model.h:26-31 layout."""

    _fields_ = [("q", _P), ("s", _P), ("rows", _I), ("cols", _I), ("dtype", _I)]


_ORC_SIGS = {
    "orc_f2i_trunc": (ctypes.c_int32, [ctypes.c_float]),
    "orc_gemv_q8": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "orc_gemv_q4": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "orc_matmul_adaptive": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "orc_matmul_f32": (None, [_P, _P, _P, _I, _I, _I]),
    "orc_silu": (None, [_P, _I]),
    "orc_rmsnorm": (None, [_P, _P, _I, _I, ctypes.c_float, _P]),
    "orc_topk_desc": (None, [_P, _I, _I, _P, _P]),
    "orc_softmax_topk": (None, [_P, _I]),
    "orc_moe_block": (None, [_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "orc_quant_q8_rows": (None, [_P, _I, _I, _P, _P]),
    "orc_quant_q4_rows": (None, [_P, _I, _I, _P, _P]),
    "orc_fill_normal": (None, [_P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float,
                               ctypes.c_float]),
    "orc_fill_uniform_u32": (None, [_P, ctypes.c_size_t, ctypes.c_uint64]),
    "orc_expf_array": (None, [_P, _P, ctypes.c_size_t]),
    "orc_expf_mismatch_u32range": (ctypes.c_uint64, [ctypes.c_uint32, ctypes.c_uint32, _P,
                                                     ctypes.POINTER(ctypes.c_uint32)]),
}

_orc = None
_refk = None
_reft = None


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"{ORACLE_LIB} not built (make -C oracle)")
        L = ctypes.CDLL(ORACLE_LIB)
        for n, (r, a) in _ORC_SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _orc = L
    return _orc


def ref_available() -> bool:
    return os.path.exists(REF_KERNELS_LIB) and os.path.exists(REF_TRACE_LIB)


def ref_kernels():
    """The reference kernels.c, compiled from /root/reference (build container only)."""
    global _refk
    if _refk is None:
        L = ctypes.CDLL(REF_KERNELS_LIB)
        L.matmul_adaptive.restype = None
        L.matmul_adaptive.argtypes = [_P, _P, _P, _P, _I, _I, _I]
        _refk = L
    return _refk


def ref_trace():
    """The reference test_model_trace.c statics, via oracle/ref_harness.c."""
    global _reft
    if _reft is None:
        L = ctypes.CDLL(REF_TRACE_LIB)
        sigs = {
            "ref_matmul_f32": (None, [_P, _P, _P, _I, _I, _I]),
            "ref_silu": (None, [_P, _I]),
            "ref_rmsnorm": (None, [_P, _P, _I, _I, ctypes.c_float, _P]),
            "ref_topk_desc": (None, [_P, _I, _I, _P, _P]),
            "ref_softmax_rows": (None, [_P, _I, _I]),
            "ref_moe_layer": (None, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
            "ref_model_forward_file": (_I, [ctypes.c_char_p, _P, _I, _P, _I]),
        }
        for n, (r, a) in sigs.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _reft = L
    return _reft


def _c(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------- synthetic data ----------------

def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(n), dtype=np.float32)
    orc().orc_fill_normal(_c(out), out.size, seed, mean, std)
    return out


def uniform_u32(n: int, seed: int) -> np.ndarray:
    out = np.empty(int(n), dtype=np.uint32)
    orc().orc_fill_uniform_u32(_c(out), out.size, seed)
    return out


def quant_q8(W: np.ndarray):
    W = np.ascontiguousarray(W, dtype=np.float32)
    N, K = W.shape
    q = np.empty((N, K), dtype=np.int8)
    s = np.empty(N, dtype=np.float32)
    orc().orc_quant_q8_rows(_c(W), N, K, _c(q), _c(s))
    return q, s


def quant_q4(W: np.ndarray):
    W = np.ascontiguousarray(W, dtype=np.float32)
    N, K = W.shape
    q = np.empty((N, K // 2), dtype=np.uint8)
    s = np.empty(N, dtype=np.float32)
    orc().orc_quant_q4_rows(_c(W), N, K, _c(q), _c(s))
    return q, s


# ---------------- the restated path ----------------

def gemv_q8(A, q, s, N, K):
    A = np.ascontiguousarray(A, dtype=np.float32).reshape(-1, K)
    C = np.empty((A.shape[0], N), dtype=np.float32)
    orc().orc_gemv_q8(_c(A), _c(q), _c(s), _c(C), A.shape[0], N, K)
    return C


def gemv_q4(A, q, s, N, K):
    A = np.ascontiguousarray(A, dtype=np.float32).reshape(-1, K)
    C = np.empty((A.shape[0], N), dtype=np.float32)
    orc().orc_gemv_q4(_c(A), _c(q), _c(s), _c(C), A.shape[0], N, K)
    return C


def matmul_f32(A, W):
    A = np.ascontiguousarray(A, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = A.shape
    N = W.shape[0]
    C = np.empty((M, N), dtype=np.float32)
    orc().orc_matmul_f32(_c(A), _c(W), _c(C), M, N, K)
    return C


def silu(x):
    x = np.array(x, dtype=np.float32, copy=True)
    orc().orc_silu(_c(x), x.size)
    return x


def rmsnorm(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, D = x.shape
    y = np.empty_like(x)
    wp = None if w is None else _c(np.ascontiguousarray(w, dtype=np.float32))
    orc().orc_rmsnorm(_c(x), wp, T, D, eps, _c(y))
    return y


def topk_desc(x, k):
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.empty(k, dtype=np.int32)
    val = np.empty(k, dtype=np.float32)
    orc().orc_topk_desc(_c(x), x.size, k, _c(idx), _c(val))
    return idx, val


def softmax_topk(val):
    v = np.array(val, dtype=np.float32, copy=True)
    orc().orc_softmax_topk(_c(v), v.size)
    return v


class ExpertSet:
    """E experts of one layer: gate/up [d_ff x D], down [D x d_ff], quantized.

    Holds numpy arrays [E, rows, bytes_per_row] plus per-expert QW structs
    pointing into them (the layout model.h binds, one struct per expert)."""

    def __init__(self, dtype: int, gq, gs, uq, us, dq, ds, D: int, d_ff: int):
        self.dtype, self.D, self.d_ff = dtype, D, d_ff
        self.gq, self.gs, self.uq, self.us, self.dq, self.ds = gq, gs, uq, us, dq, ds
        E = gq.shape[0]
        self.E = E
        self.Wg = (QW * E)()
        self.Wu = (QW * E)()
        self.Wd = (QW * E)()
        for e in range(E):
            self.Wg[e] = QW(_c(gq[e]), _c(gs[e]), d_ff, D, dtype)
            self.Wu[e] = QW(_c(uq[e]), _c(us[e]), d_ff, D, dtype)
            self.Wd[e] = QW(_c(dq[e]), _c(ds[e]), D, d_ff, dtype)


def make_experts(dtype: int, E: int, D: int, d_ff: int, seed: int, std: float = 0.02) -> ExpertSet:
    """Synthetic experts: W ~ N(0, std^2) per matrix, then rowwise Q8/Q4."""
    quant = quant_q8 if dtype == 2 else quant_q4
    cols_g = D if dtype == 2 else D // 2
    cols_d = d_ff if dtype == 2 else d_ff // 2
    qdt = np.int8 if dtype == 2 else np.uint8
    gq = np.empty((E, d_ff, cols_g), qdt)
    uq = np.empty((E, d_ff, cols_g), qdt)
    dq = np.empty((E, D, cols_d), qdt)
    gs = np.empty((E, d_ff), np.float32)
    us = np.empty((E, d_ff), np.float32)
    ds = np.empty((E, D), np.float32)
    for e in range(E):
        for j, (qa, sa, n, k) in enumerate(((gq, gs, d_ff, D), (uq, us, d_ff, D), (dq, ds, D, d_ff))):
            W = normal(n * k, seed * 1000003 + e * 7 + j, 0.0, std).reshape(n, k)
            q, s = quant(W)
            qa[e] = q
            sa[e] = s
    return ExpertSet(dtype, gq, gs, uq, us, dq, ds, D, d_ff)


def moe_block(x_norm, x_resid, router_w, router_b, ex: ExpertSet, top_k: int = 8):
    """test_model_trace.c:463-517 -> (out, idx, p, logits)."""
    x_norm = np.ascontiguousarray(x_norm, dtype=np.float32)
    T, D = x_norm.shape
    E = router_w.shape[0]
    out = np.empty((T, D), np.float32)
    idx = np.empty((T, top_k), np.int32)
    p = np.empty((T, top_k), np.float32)
    logits = np.empty((T, E), np.float32)
    rw = np.ascontiguousarray(router_w, dtype=np.float32)
    rb = None if router_b is None else _c(np.ascontiguousarray(router_b, dtype=np.float32))
    xr = None if x_resid is None else _c(np.ascontiguousarray(x_resid, dtype=np.float32))
    orc().orc_moe_block(_c(x_norm), xr, T, D, E, top_k, ex.d_ff, _c(rw), rb,
                        ctypes.addressof(ex.Wg), ctypes.addressof(ex.Wu), ctypes.addressof(ex.Wd),
                        _c(out), _c(idx), _c(p), _c(logits))
    return out, idx, p, logits


def expf_array(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    orc().orc_expf_array(_c(x), _c(y), x.size)
    return y


def expf_mismatches(lo: int, dev: np.ndarray):
    first = ctypes.c_uint32(0)
    dev = np.ascontiguousarray(dev, dtype=np.float32)
    n = orc().orc_expf_mismatch_u32range(lo, dev.size, _c(dev), ctypes.byref(first))
    return int(n), int(first.value)
