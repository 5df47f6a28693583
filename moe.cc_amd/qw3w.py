"""qw3w.py - the reference's QW3W tensor container (all_q8.bin / all_q4.bin).

Layout (export.py:8-21 writes it, io.c:193-285 reads it): little endian, no
padding; magic b"QW3W\\x00\\x01", a u32 entry count, then entries
    u32 name_len, name bytes (no NUL), u32 dtype, u32 ndim, u32 shape[ndim],
    raw data
with dtype 0 = f32, 1 = f16, 2 = int8 (Q8 weights), 3 = uint8 (Q4: two
nibbles per byte, low nibble = even column, value q + 8).  A quantized
weight is two entries, "<name>.scale" (f32 [rows]) and then "<name>.q8" or
"<name>.q4" (export.py:164-171).  The count in the header is the exporter's
tensor count, which undercounts quantized files (merge_dir.py:37); readers
ignore it and read to the end of the file (io.c:212-244), and so does this
one.

Tensor names are the ones model.h:107-323 binds (load_all_weights).
"""
from __future__ import annotations

import mmap
import struct
from typing import Dict, Iterable, Iterator, Tuple

import numpy as np

MAGIC = b"QW3W\x00\x01"
DTYPES = {0: np.float32, 1: np.float16, 2: np.int8, 3: np.uint8}
CODES = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int8): 2,
         np.dtype(np.uint8): 3}


def write(path: str, tensors: Iterable[Tuple[str, np.ndarray]], count: int | None = None) -> int:
    """Writes (name, array) entries in order; `count` is the header's u32
    (default: the number of entries).  Returns the number of entries."""
    items = list(tensors)
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<I", len(items) if count is None else count))
        for name, a in items:
            a = np.ascontiguousarray(a)
            code = CODES.get(a.dtype)
            if code is None:
                raise ValueError(f"{name}: dtype {a.dtype} has no QW3W code")
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)))
            f.write(nb)
            f.write(struct.pack("<II", code, a.ndim))
            f.write(struct.pack("<" + "I" * a.ndim, *a.shape))
            f.write(a.tobytes())
    return len(items)


def iter_entries(buf) -> Iterator[Tuple[str, int, Tuple[int, ...], int, int]]:
    """(name, dtype, shape, data offset, data bytes) of every entry, reading
    to the end of `buf` (io.c:212-271).  Raises ValueError on a bad magic, an
    unknown dtype or a truncated entry."""
    if bytes(buf[:6]) != MAGIC:
        raise ValueError("bad magic (not a QW3W file)")
    off = 10
    n = len(buf)
    while off + 4 <= n:
        (nl,) = struct.unpack_from("<I", buf, off)
        off += 4
        if off + nl + 8 > n:
            raise ValueError("truncated entry header")
        name = bytes(buf[off:off + nl]).decode()
        off += nl
        dt, nd = struct.unpack_from("<II", buf, off)
        off += 8
        if dt not in DTYPES:
            raise ValueError(f"{name}: unknown dtype {dt}")
        shape = struct.unpack_from("<" + "I" * nd, buf, off)
        off += 4 * nd
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(DTYPES[dt]).itemsize
        if off + nbytes > n:
            raise ValueError(f"{name}: truncated data")
        yield name, dt, tuple(shape), off, nbytes
        off += nbytes


class File:
    """A memory-mapped QW3W file with a name index (the reference's bin_find
    is a linear scan, io.c:333-338; this is a dict)."""

    def __init__(self, path: str):
        self._f = open(path, "rb")
        self._m = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        (self.header_count,) = struct.unpack_from("<I", self._m, 6)
        self.index: Dict[str, Tuple[int, Tuple[int, ...], int, int]] = {}
        for name, dt, shape, off, nb in iter_entries(self._m):
            self.index[name] = (dt, shape, off, nb)

    def __contains__(self, name: str) -> bool:
        return name in self.index

    def get(self, name: str) -> np.ndarray:
        dt, shape, off, nb = self.index[name]
        return np.frombuffer(self._m, dtype=DTYPES[dt], count=nb // np.dtype(DTYPES[dt]).itemsize,
                             offset=off).reshape(shape)

    def close(self):
        self._m.close()
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


# ---- names bound by load_all_weights (model.h:107-305) ----

def layer_prefix(L: int) -> str:
    return f"model.layers.{L}."


def expert_name(L: int, e: int, proj: str) -> str:
    return f"model.layers.{L}.mlp.experts.{e}.{proj}_proj.weight"


def model_entries(m) -> Iterator[Tuple[str, np.ndarray]]:
    """Entries of a model object with the attributes of oracle.TinyModel /
    the reference's QwenWeights (numpy arrays), in the exporter's order:
    embedding, final norm, head, then per layer attention, norms, router and
    the experts as .scale then .q8/.q4 pairs."""
    yield "model.embed_tokens.weight", m.tok_emb
    yield "model.norm.weight", m.final_norm_w
    if m.lm_head is not None:
        yield "lm_head.weight", m.lm_head
    suffix = ".q8" if m.expert_dtype == 2 else ".q4"
    for L, lw in enumerate(m.layers):
        p = layer_prefix(L)
        for nm, key in (("q_proj", "Wq"), ("k_proj", "Wk"), ("v_proj", "Wv"), ("o_proj", "Wo")):
            yield p + f"self_attn.{nm}.weight", lw[key]
            b = lw.get("b" + key[1:].lower())
            if b is not None:
                yield p + f"self_attn.{nm}.bias", b
        if lw.get("q_norm") is not None:
            yield p + "self_attn.q_norm.weight", lw["q_norm"]
        if lw.get("k_norm") is not None:
            yield p + "self_attn.k_norm.weight", lw["k_norm"]
        yield p + "input_layernorm.weight", lw["rms1_w"]
        yield p + "post_attention_layernorm.weight", lw["rms2_w"]
        yield p + "mlp.gate.weight", lw["router_w"]
        if lw.get("router_b") is not None:
            yield p + "mlp.gate.bias", lw["router_b"]
        ex = lw["experts"]
        for e in range(ex.E):
            for proj, q, s in (("gate", ex.gq, ex.gs), ("up", ex.uq, ex.us), ("down", ex.dq, ex.ds)):
                yield expert_name(L, e, proj) + ".scale", s[e]
                yield expert_name(L, e, proj) + suffix, q[e]
