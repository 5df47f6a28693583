"""moehip - Python host binding of libmoehip.so (ctypes; no torch).

Mirrors the reference's call surface for the quantized expert path:
``matmul_adaptive`` (kernels.h:16-17) with its host-pointer semantics, the
device-pointer GEMVs, and the MoE block of one layer
(test_model_trace.c:460-517).  Arrays are numpy; device memory is held by
:class:`DeviceBuffer`.  There is no CPU fallback: if the library is missing or
the GPU runtime fails, every call raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MOEHIP_LIB selects another build of the library (for comparing variants)
LIB_PATH = os.environ.get("MOEHIP_LIB") or os.path.join(_HERE, "libmoehip.so")

_lib: Optional[ctypes.CDLL] = None


class MoeError(RuntimeError):
    pass


class QuantizedWeight(ctypes.Structure):
    """model.h:26-31 layout: {q, s, rows, cols, dtype}."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("s", ctypes.c_void_p),
        ("rows", ctypes.c_int),
        ("cols", ctypes.c_int),
        ("dtype", ctypes.c_int),
    ]


class QJob(ctypes.Structure):
    _fields_ = [
        ("W", ctypes.c_void_p),
        ("S", ctypes.c_void_p),
        ("A", ctypes.c_void_p),
        ("C", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t

_SIGS = {
    "matmul_adaptive": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "moe_init": (_I, [_I]),
    "moe_shutdown": (_I, []),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_version": (ctypes.c_char_p, []),
    "moe_get_stream": (_P, []),
    "moe_synchronize": (_I, []),
    "moe_weight_cache_clear": (_I, []),
    "moe_weight_cache_mode": (_I, [_I]),
    "moe_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "moe_free": (_I, [_P]),
    "moe_memcpy_h2d": (_I, [_P, _P, _SZ]),
    "moe_memcpy_d2h": (_I, [_P, _P, _SZ]),
    "moe_memcpy_d2d": (_I, [_P, _P, _SZ]),
    "moe_memset": (_I, [_P, _I, _SZ]),
    "moe_stream_read_dev": (_I, [_P, _SZ, _P]),
    "moe_event_create": (_I, [ctypes.POINTER(_P)]),
    "moe_event_record": (_I, [_P]),
    "moe_event_elapsed_ms": (_I, [_P, _P, ctypes.POINTER(ctypes.c_float)]),
    "moe_event_destroy": (_I, [_P]),
    "moe_matmul_q8_dev": (_I, [_P, _P, _P, _P, _I, _I, _I]),
    "moe_matmul_q4_dev": (_I, [_P, _P, _P, _P, _I, _I, _I]),
    "moe_matmul_f32_dev": (_I, [_P, _P, _P, _I, _I, _I]),
    "moe_greedy_dev": (_I, [_P, _I, _P]),
    "moe_head_greedy_dev": (_I, [_P, _P, _I, _I, _P, _P]),
    "moe_matmul_adaptive_dev": (_I, [_P, _P, ctypes.POINTER(QuantizedWeight), _P, _I, _I, _I]),
    "moe_matmul_q_batched_dev": (_I, [_I, _P, _I, _I, _I, _I]),
    "moe_gemv_variant": (ctypes.c_char_p, [_I, _I, _I, _I]),
    "moe_act_table_bytes": (_SZ, [_I]),
    "moe_act_pack_dev": (_I, [_I, _P, _I, _I, _P]),
    "moe_matmul_q_prepacked_dev": (_I, [_I, _P, _I, _I, _I, _I, _P]),
    "moe_rows_read_dev": (_I, [_I, _P, _I, _I, _I, _I, _P]),
    "moe_silu_mul_dev": (_I, [_P, _P, _P, _SZ]),
    "moe_expf_dev": (_I, [_P, _P, _SZ]),
    "moe_expf_bits_dev": (_I, [ctypes.c_uint32, _P, _SZ]),
    "moe_selfcheck_qdot_dev": (_I, [_I, ctypes.POINTER(ctypes.c_ulonglong)]),
    "moe_fill_normal_dev": (_I, [_P, _SZ, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
    "moe_quantize_rows_dev": (_I, [_I, _P, ctypes.c_longlong, _I, _P, _P]),
    "moe_layer_create": (_I, [_P, _P, ctypes.POINTER(_P)]),
    "moe_layer_create_raw": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                                  ctypes.POINTER(_P)]),
    "moe_layer_destroy": (_I, [_P]),
    "moe_layer_set_grouped_min_tokens": (_I, [_P, _I]),
    "moe_layer_forward": (_I, [_P, _P, _P, _I, _P, _P, _P]),
    "moe_layer_forward_noalloc": (_I, [_P, _P, _P, _I, _P, _P, _P]),
    "moe_block_forward": (_I, [_P, _P, _I, _P, ctypes.c_float]),
    "moe_rmsnorm_dev": (_I, [_P, _P, _P, _I, _I, ctypes.c_float]),
    "moe_layer_debug_buffers": (_I, [_P, ctypes.POINTER(_P), ctypes.POINTER(_P),
                                     ctypes.POINTER(_P)]),
    "moe_model_create": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "moe_model_load_file": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(_P)]),
    "moe_model_inspect_file": (_I, [ctypes.c_char_p, _P, _P]),
    "moe_model_create_synthetic": (_I, [_P, _I, _I, ctypes.c_uint64, ctypes.c_float, _I,
                                        ctypes.POINTER(_P)]),
    "moe_model_destroy": (_I, [_P]),
    "moe_model_config": (_I, [_P, _P]),
    "moe_model_reset": (_I, [_P]),
    "moe_model_position": (_I, [_P]),
    "moe_model_forward": (_I, [_P, _P, _I, _I, _P, _P]),
    "moe_model_forward_full": (_I, [_P, _P, _I, _I, _P]),
    "moe_model_generate": (_I, [_P, _P, _I, _I, _P, ctypes.POINTER(ctypes.c_float),
                                ctypes.POINTER(ctypes.c_float)]),
}


def exported_symbols():
    """Names the C ABI (include/moehip.h) exports."""
    return list(_SIGS)


def lib() -> ctypes.CDLL:
    """Loads libmoehip.so (built in-tree by ``make -C moe.cc_amd``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MoeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            try:
                fn = getattr(L, name)
            except AttributeError:
                if os.environ.get("MOEHIP_LIB"):
                    continue   # an older build chosen for comparison may predate a symbol
                raise
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().moe_last_error().decode(errors="replace")
        raise MoeError(f"{what}: status {status}: {msg}")


def init(device: int = 0) -> None:
    check(lib().moe_init(device), "moe_init")


def shutdown() -> None:
    """moe_shutdown: frees the library's own device buffers and stream (every
    layer and model must be closed first); the next call re-initialises."""
    check(lib().moe_shutdown(), "moe_shutdown")


def synchronize() -> None:
    check(lib().moe_synchronize(), "moe_synchronize")


class DeviceBuffer:
    """Owned device allocation of `nbytes` bytes."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _P()
        check(lib().moe_malloc(ctypes.byref(p), max(self.nbytes, 1)), "moe_malloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise MoeError("upload past the end of the buffer")
        check(lib().moe_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes), "h2d")

    def download(self, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise MoeError("download past the end of the buffer")
        check(lib().moe_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "d2h")
        return out

    def zero(self) -> None:
        check(lib().moe_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            check(lib().moe_free(self.ptr), "moe_free")
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.moe_free(self.ptr)
        except Exception:
            pass


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def matmul_adaptive(A: np.ndarray, W_fp32: Optional[np.ndarray], W_q: Optional[dict],
                    N: int, K: int) -> np.ndarray:
    """The drop-in entry point on host arrays (kernels.c:149-181).

    ``W_q`` is None for the fp32 path, else a dict with ``q`` (int8 / uint8
    array), ``s`` (fp32 [N]) and ``dtype`` (2 = Q8, 3 = Q4).  Returns C [M, N].
    The host arrays must stay alive while the library caches their upload.
    """
    A = _f32(A)
    M = A.shape[0] if A.ndim == 2 else 1
    C = np.empty((M, N), dtype=np.float32)
    if W_q is None:
        Wf = _f32(W_fp32)
        lib().matmul_adaptive(A.ctypes.data, Wf.ctypes.data, None, C.ctypes.data, M, N, K)
    else:
        qw = QuantizedWeight(W_q["q"].ctypes.data, W_q["s"].ctypes.data, N,
                             K, int(W_q["dtype"]))
        lib().matmul_adaptive(A.ctypes.data, None, ctypes.addressof(qw), C.ctypes.data, M, N, K)
    return C


def gemv_variant(dtype: int, M: int, N: int, K: int) -> str:
    return lib().moe_gemv_variant(dtype, M, N, K).decode()


class Event:
    def __init__(self):
        p = _P()
        check(lib().moe_event_create(ctypes.byref(p)), "event_create")
        self.ptr = p.value

    def record(self) -> None:
        check(lib().moe_event_record(self.ptr), "event_record")

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().moe_event_elapsed_ms(self.ptr, stop.ptr, ctypes.byref(ms)), "elapsed")
        return float(ms.value)

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.moe_event_destroy(self.ptr)
        except Exception:
            pass


class MoeLayer:
    """Device-resident MoE block of one layer (test_model_trace.c:460-517)."""

    def __init__(self, handle, dtype, D, d_ff, E, top_k):
        self.h, self.dtype, self.D, self.d_ff, self.E, self.top_k = handle, dtype, D, d_ff, E, top_k

    @classmethod
    def from_arrays(cls, dtype, router_w, router_b, gq, gs, uq, us, dq, ds, rms2_w=None,
                    top_k=8):
        """Host arrays: router_w [E, D], gq/uq [E, d_ff, rb_g], dq [E, D, rb_d], scales fp32."""
        router_w = _f32(router_w)
        E, D = router_w.shape
        d_ff = gq.shape[1]
        keep = [router_w, np.ascontiguousarray(gq), _f32(gs), np.ascontiguousarray(uq), _f32(us),
                np.ascontiguousarray(dq), _f32(ds)]
        rb = None if router_b is None else _f32(router_b)
        rw2 = None if rms2_w is None else _f32(rms2_w)
        h = _P()
        check(lib().moe_layer_create_raw(
            dtype, D, d_ff, E, top_k, keep[0].ctypes.data,
            None if rb is None else rb.ctypes.data, None if rw2 is None else rw2.ctypes.data,
            keep[1].ctypes.data, keep[2].ctypes.data, keep[3].ctypes.data, keep[4].ctypes.data,
            keep[5].ctypes.data, keep[6].ctypes.data, 0, ctypes.byref(h)), "moe_layer_create_raw")
        return cls(h.value, dtype, D, d_ff, E, top_k)

    def set_grouped_min_tokens(self, min_tokens: int):
        """Token count from which forwards run expert-major (0 = default)."""
        check(lib().moe_layer_set_grouped_min_tokens(self.h, min_tokens),
              "moe_layer_set_grouped_min_tokens")

    def forward_dev(self, x_norm_ptr, x_resid_ptr, T, out_ptr, idx_ptr=None, p_ptr=None):
        check(lib().moe_layer_forward(self.h, x_norm_ptr, x_resid_ptr, T, out_ptr, idx_ptr, p_ptr),
              "moe_layer_forward")

    def forward(self, x_norm: np.ndarray, x_resid: Optional[np.ndarray]):
        """Host-array convenience: returns (out [T, D], idx [T, k], p [T, k])."""
        x_norm = _f32(x_norm)
        T = x_norm.shape[0]
        dx = DeviceBuffer.from_array(x_norm)
        dr = DeviceBuffer.from_array(_f32(x_resid)) if x_resid is not None else None
        do = DeviceBuffer(x_norm.nbytes)
        di = DeviceBuffer(T * self.top_k * 4)
        dp = DeviceBuffer(T * self.top_k * 4)
        self.forward_dev(dx.ptr, None if dr is None else dr.ptr, T, do.ptr, di.ptr, dp.ptr)
        return (do.download((T, self.D), np.float32), di.download((T, self.top_k), np.int32),
                dp.download((T, self.top_k), np.float32))

    def block_forward(self, x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
        x = _f32(x)
        dx = DeviceBuffer.from_array(x)
        do = DeviceBuffer(x.nbytes)
        check(lib().moe_block_forward(self.h, dx.ptr, x.shape[0], do.ptr, eps), "moe_block_forward")
        return do.download(x.shape, np.float32)

    def debug(self, T):
        lg, hh, yy = _P(), _P(), _P()
        check(lib().moe_layer_debug_buffers(self.h, ctypes.byref(lg), ctypes.byref(hh),
                                            ctypes.byref(yy)))
        out = {}
        for name, ptr, shape in (("logits", lg.value, (T, self.E)),
                                 ("h", hh.value, (T * self.top_k, self.d_ff)),
                                 ("y", yy.value, (T * self.top_k, self.D))):
            if not ptr:
                continue
            a = np.empty(shape, np.float32)
            check(lib().moe_memcpy_d2h(a.ctypes.data, ptr, a.nbytes))
            out[name] = a
        return out

    def close(self):
        if self.h:
            check(lib().moe_layer_destroy(self.h), "moe_layer_destroy")
            self.h = None

    def __del__(self):
        try:
            if self.h and _lib is not None:
                _lib.moe_layer_destroy(self.h)
        except Exception:
            pass


# ---------------- the whole model (test_model_trace.c:526-579) ----------------

class QwenConfig(ctypes.Structure):
    """model.h:9-23 layout."""

    _fields_ = [("d_model", _I), ("n_layers", _I), ("head_dim", _I), ("n_q", _I), ("n_kv", _I),
                ("d_ff", _I), ("n_experts", _I), ("top_k", _I), ("vocab_size", _I),
                ("causal", _I), ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


class QwenLayerWeights(ctypes.Structure):
    """model.h:34-58 layout."""

    _fields_ = [(n, _P) for n in ("Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "q_norm",
                                  "k_norm", "rms1_w", "rms2_w", "router_w", "router_b",
                                  "Wg", "bg", "Wu", "bu", "Wd", "bd", "Wg_q", "Wu_q", "Wd_q")] + \
               [("experts_quantized", _I)]


class QwenWeights(ctypes.Structure):
    """model.h:60-69 layout."""

    _fields_ = [("tok_emb", _P), ("final_norm_w", _P), ("lm_head", _P), ("layers", _P)]


def qwen_config(D, L, hd, nq, nkv, dff, E, top_k, V, theta=1e7, eps=1e-6) -> QwenConfig:
    return QwenConfig(D, L, hd, nq, nkv, dff, E, top_k, V, 1, float(theta), float(eps))


class Model:
    """A whole Qwen3-MoE model on the device with a KV cache."""

    def __init__(self, handle):
        self.h = handle
        cfg = QwenConfig()
        check(lib().moe_model_config(self.h, ctypes.byref(cfg)), "moe_model_config")
        self.cfg = cfg
        self.V = cfg.vocab_size

    @classmethod
    def synthetic(cls, cfg: QwenConfig, expert_dtype=3, untied_head=True, seed=1, std=0.02,
                  max_seq=2048):
        h = _P()
        check(lib().moe_model_create_synthetic(ctypes.byref(cfg), expert_dtype, int(untied_head),
                                               seed, std, max_seq, ctypes.byref(h)),
              "moe_model_create_synthetic")
        return cls(h.value)

    @classmethod
    def load_file(cls, path: str, max_seq=2048):
        h = _P()
        check(lib().moe_model_load_file(path.encode(), max_seq, ctypes.byref(h)),
              "moe_model_load_file")
        return cls(h.value)

    @classmethod
    def from_host(cls, cfg: QwenConfig, tok_emb, final_norm_w, lm_head, layers, max_seq=2048):
        """layers: list of dicts of numpy arrays with the QwenLayerWeights
        names (Wq, bq, ..., router_b) plus "experts": an object with gq, gs,
        uq, us, dq, ds arrays [E, rows, bytes] and `dtype` (the oracle's
        ExpertSet has this shape)."""
        keep = []

        def p(a, dt=np.float32):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dt)
            keep.append(a)
            return a.ctypes.data

        n = len(layers)
        lws = (QwenLayerWeights * n)()
        for i, lw in enumerate(layers):
            ex = lw["experts"]
            E = ex.gq.shape[0]
            qdt = np.int8 if ex.dtype == 2 else np.uint8
            arrs = []
            for q, s, rows, cols in ((ex.gq, ex.gs, cfg.d_ff, cfg.d_model),
                                     (ex.uq, ex.us, cfg.d_ff, cfg.d_model),
                                     (ex.dq, ex.ds, cfg.d_model, cfg.d_ff)):
                qa = (QuantizedWeight * E)()
                for e in range(E):
                    qa[e] = QuantizedWeight(p(q[e], qdt), p(s[e]), rows, cols, ex.dtype)
                keep.append(qa)
                arrs.append(ctypes.addressof(qa))
            lws[i] = QwenLayerWeights(*[p(lw.get(k)) for k in (
                "Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "q_norm", "k_norm", "rms1_w",
                "rms2_w", "router_w", "router_b")], None, None, None, None, None, None,
                arrs[0], arrs[1], arrs[2], 1)
        w = QwenWeights(p(tok_emb), p(final_norm_w), p(lm_head), ctypes.addressof(lws))
        h = _P()
        check(lib().moe_model_create(ctypes.byref(cfg), ctypes.byref(w), max_seq, ctypes.byref(h)),
              "moe_model_create")
        return cls(h.value)

    def reset(self):
        check(lib().moe_model_reset(self.h), "moe_model_reset")

    @property
    def position(self) -> int:
        return lib().moe_model_position(self.h)

    def forward(self, ids):
        """New tokens (host ids) at the current position -> (last-row logits, greedy id)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        lg = DeviceBuffer(self.V * 4)
        nx = DeviceBuffer(4)
        check(lib().moe_model_forward(self.h, ids.ctypes.data, ids.size, 0, lg.ptr, nx.ptr),
              "moe_model_forward")
        return lg.download((self.V,), np.float32), int(nx.download((1,), np.int32)[0])

    def forward_full(self, ids, apply_softmax=False):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.V, np.float32)
        check(lib().moe_model_forward_full(self.h, ids.ctypes.data, ids.size, int(apply_softmax),
                                           out.ctypes.data), "moe_model_forward_full")
        return out

    def generate(self, prompt, n_new):
        """-> (ids [n_new], ms_prompt, ms_decode)"""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_new, np.int32)
        a, b = ctypes.c_float(), ctypes.c_float()
        check(lib().moe_model_generate(self.h, prompt.ctypes.data, prompt.size, n_new,
                                       out.ctypes.data, ctypes.byref(a), ctypes.byref(b)),
              "moe_model_generate")
        return out, a.value, b.value

    def close(self):
        if self.h:
            check(lib().moe_model_destroy(self.h), "moe_model_destroy")
            self.h = None

    def __del__(self):
        try:
            if self.h and _lib is not None:
                _lib.moe_model_destroy(self.h)
        except Exception:
            pass


def model_from_tiny(tm, max_seq=64) -> Model:
    """A Model from an object with TinyModel's attributes (oracle test models)."""
    cfg = qwen_config(tm.D, tm.L, tm.hd, tm.nq, tm.nkv, tm.dff, tm.E, tm.top_k, tm.V, tm.theta,
                      tm.eps)
    return Model.from_host(cfg, tm.tok_emb, tm.final_norm_w, tm.lm_head, tm.layers, max_seq)
