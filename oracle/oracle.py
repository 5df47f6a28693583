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
# the same sources built with -fopenmp (rows split over threads, bit-identical)
ORACLE_OMP_LIB = os.path.join(_HERE, "liboracle_omp.so")
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
    "orc_layer_rows": (None, [_P, _P, _P, _I, _I, _P, _P, _I]),
    "orc_model_forward_kv": (None, [_P, _P, _P, _I, _I, _P, _P, _I, _P, _P]),
    "orc_rope_tables": (None, [_I, ctypes.c_float, _I, _P, _P]),
    "orc_greedy": (_I, [_P, _I]),
    "orc_softmax_rows": (None, [_P, _I, _I]),
    "orc_threads": (_I, []),
}

_orc = None
_orc_omp = None
_threaded = False
_refk = None
_reft = None


def _load_orc(path):
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not built (make -C oracle)")
    L = ctypes.CDLL(path)
    for n, (r, a) in _ORC_SIGS.items():
        f = getattr(L, n)
        f.restype = r
        f.argtypes = a
    return L


def orc_single():
    """The single-thread build (liboracle.so)."""
    global _orc
    if _orc is None:
        _orc = _load_orc(ORACLE_LIB)
    return _orc


def orc_omp():
    """The -fopenmp build (liboracle_omp.so): bit-identical, rows on threads."""
    global _orc_omp
    if _orc_omp is None:
        _orc_omp = _load_orc(ORACLE_OMP_LIB)
    return _orc_omp


def orc():
    """The build the wrappers below call: single-thread unless inside
    `threaded()`."""
    return orc_omp() if _threaded else orc_single()


class threaded:
    """Context manager: the wrappers use the -fopenmp build inside it (when
    that build exists; otherwise the single-thread one)."""

    def __enter__(self):
        global _threaded
        self._prev = _threaded
        _threaded = os.path.exists(ORACLE_OMP_LIB)
        return self

    def __exit__(self, *exc):
        global _threaded
        _threaded = self._prev
        return False


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


# ---------------- the whole model (model_oracle.c) ----------------

class OrcConfig(ctypes.Structure):
    """QwenConfig (model.h:9-23) / orc_config."""

    _fields_ = [("d_model", _I), ("n_layers", _I), ("head_dim", _I), ("n_q", _I), ("n_kv", _I),
                ("d_ff", _I), ("n_experts", _I), ("top_k", _I), ("vocab_size", _I),
                ("causal", _I), ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


class OrcLayer(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "q_norm",
                                  "k_norm", "rms1_w", "rms2_w", "router_w", "router_b",
                                  "Wg", "Wu", "Wd")]


class OrcWeights(ctypes.Structure):
    _fields_ = [("tok_emb", _P), ("final_norm_w", _P), ("lm_head", _P), ("layers", _P)]


def _ptr(a):
    return None if a is None else _c(a)


class TinyModel:
    """A seeded synthetic Qwen3-MoE model (config 5's recipe at any size):
    weights ~ N(0, std^2), norm weights 1 (or N(1, 0.1^2) with
    `random_norms`), quantized experts, optional biases and untied head.

    Attributes follow QwenWeights: tok_emb, final_norm_w, lm_head (None =
    tied), layers[L] = dict of numpy arrays plus an ExpertSet."""

    def __init__(self, D=64, L=2, hd=16, nq=4, nkv=2, dff=32, E=16, top_k=8, V=97, dtype=3,
                 seed=1, std=0.02, theta=1e7, eps=1e-6, untied=True, bias=False, qk_norm=True,
                 random_norms=False, expert_std=None):
        self.D, self.L, self.hd, self.nq, self.nkv, self.dff = D, L, hd, nq, nkv, dff
        self.E, self.top_k, self.V, self.expert_dtype = E, top_k, V, dtype
        self.theta, self.eps = float(theta), float(eps)
        self.cfg = OrcConfig(D, L, hd, nq, nkv, dff, E, top_k, V, 1, self.theta, self.eps)
        sd = [seed * 7919]

        def nrm(*shape, mean=0.0, s=std):
            sd[0] += 1
            return normal(int(np.prod(shape)), sd[0], mean, s).reshape(shape)

        def norm_w(n):
            return nrm(n, mean=1.0, s=0.1) if random_norms else np.ones(n, np.float32)

        self.tok_emb = nrm(V, D)
        self.final_norm_w = norm_w(D)
        self.lm_head = nrm(V, D) if untied else None
        Dq, Dkv = nq * hd, nkv * hd
        self.layers = []
        for li in range(L):
            lw = {"Wq": nrm(Dq, D), "Wk": nrm(Dkv, D), "Wv": nrm(Dkv, D), "Wo": nrm(D, Dq),
                  "bq": nrm(Dq, s=0.1) if bias else None, "bk": nrm(Dkv, s=0.1) if bias else None,
                  "bv": nrm(Dkv, s=0.1) if bias else None, "bo": nrm(D, s=0.1) if bias else None,
                  "q_norm": norm_w(hd) if qk_norm else None,
                  "k_norm": norm_w(hd) if qk_norm else None,
                  "rms1_w": norm_w(D), "rms2_w": norm_w(D), "router_w": nrm(E, D),
                  "router_b": nrm(E, s=0.05) if bias else None}
            sd[0] += 1
            lw["experts"] = make_experts(dtype, E, D, dff, sd[0],
                                         std if expert_std is None else expert_std)
            self.layers.append(lw)
        self._build_structs()

    @classmethod
    def from_weights(cls, D, L, hd, nq, nkv, dff, E, V, dtype, tok_emb, final_norm_w, lm_head,
                     layers, top_k=8, theta=1e7, eps=1e-6):
        """A model over given arrays (same attribute layout as __init__
        builds): `layers` = list of dicts with the QwenLayerWeights names and
        an "experts" ExpertSet.  For full-width models whose weights are made
        elsewhere (a seeded generator on the device, downloaded)."""
        self = cls.__new__(cls)
        self.D, self.L, self.hd, self.nq, self.nkv, self.dff = D, L, hd, nq, nkv, dff
        self.E, self.top_k, self.V, self.expert_dtype = E, top_k, V, dtype
        self.theta, self.eps = float(theta), float(eps)
        self.cfg = OrcConfig(D, L, hd, nq, nkv, dff, E, top_k, V, 1, self.theta, self.eps)
        self.tok_emb = np.ascontiguousarray(tok_emb, dtype=np.float32)
        self.final_norm_w = np.ascontiguousarray(final_norm_w, dtype=np.float32)
        self.lm_head = None if lm_head is None else np.ascontiguousarray(lm_head, dtype=np.float32)
        names = ("Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "q_norm", "k_norm", "rms1_w",
                 "rms2_w", "router_w", "router_b")
        self.layers = [dict({k: None for k in names}, **lw) for lw in layers]
        if len(self.layers) != L:
            raise ValueError("from_weights: layer count differs from L")
        self._build_structs()
        return self

    def _build_structs(self):
        self._layers = (OrcLayer * self.L)()
        for i, lw in enumerate(self.layers):
            ex = lw["experts"]
            self._layers[i] = OrcLayer(*[_ptr(lw[k]) for k in (
                "Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "q_norm", "k_norm", "rms1_w",
                "rms2_w", "router_w", "router_b")],
                ctypes.addressof(ex.Wg), ctypes.addressof(ex.Wu), ctypes.addressof(ex.Wd))
        self._w = OrcWeights(_c(self.tok_emb), _c(self.final_norm_w), _ptr(self.lm_head),
                             ctypes.addressof(self._layers))

    def new_cache(self, max_seq):
        shape = (self.L, self.nkv, max_seq, self.hd)
        return np.zeros(shape, np.float32), np.zeros(shape, np.float32)

    def forward_kv(self, ids, pos0, cache, return_x=False):
        """New rows at positions pos0..: returns the last row's logits
        (and the hidden states after the last layer)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        kc, vc = cache
        out = np.empty(self.V, np.float32)
        x = np.empty((ids.size, self.D), np.float32) if return_x else None
        orc().orc_model_forward_kv(ctypes.byref(self.cfg), ctypes.byref(self._w), _c(ids), ids.size,
                                   pos0, _c(kc), _c(vc), kc.shape[2], _c(out), _ptr(x))
        return (out, x) if return_x else out

    def generate(self, prompt, steps, max_seq):
        """Greedy decode: prefill the prompt, then `steps` tokens (greedy)."""
        cache = self.new_cache(max_seq)
        logits = self.forward_kv(prompt, 0, cache)
        out = []
        pos = len(prompt)
        for _ in range(steps):
            nxt = greedy(logits)
            out.append(nxt)
            logits = self.forward_kv([nxt], pos, cache)
            pos += 1
        return np.array(out, np.int32), logits


def greedy(v) -> int:
    """The reference's next-token choice over a logit row
    (test_model_trace.c:735-746): argmax of softmax_rows, first index."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(orc().orc_greedy(_c(v), v.size))


def softmax_rows(m):
    """test_model_trace.c:260-272 on a copy of a 2-D array."""
    m = np.array(m, dtype=np.float32, copy=True, ndmin=2)
    orc().orc_softmax_rows(_c(m), m.shape[0], m.shape[1])
    return m


def rope_tables(hd, theta, n_pos):
    c = np.empty((n_pos, hd // 2), np.float32)
    s = np.empty((n_pos, hd // 2), np.float32)
    orc().orc_rope_tables(hd, float(theta), n_pos, _c(c), _c(s))
    return c, s
