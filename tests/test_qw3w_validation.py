"""QW3W files (io.c:193-285) with bad headers or tensors that do not fit
the config load_all_weights infers (model.h:110-163) are rejected by the
library's host-side reader before anything is copied or uploaded:
moe_model_inspect_file (the first half of moe_model_load_file, no GPU call)
returns MOE_ERR_ARG naming the tensor.  The reference reads such files
without checks (a mismatch there is an out-of-bounds read).  CPU only."""
import ctypes
import os
import struct

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "moe.cc_amd", "libmoehip.so")
pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="libmoehip.so not built")

MOE_ERR_ARG = 2


def _tiny(dtype=3, bias=True):
    return O.TinyModel(D=64, L=2, hd=16, nq=4, nkv=2, dff=32, E=8, V=50, dtype=dtype, seed=31,
                       bias=bias)


def _entries(tm):
    import qw3w
    return list(qw3w.model_entries(tm))


def _inspect(path):
    import moehip
    L = moehip.lib()
    cfg = moehip.QwenConfig()
    dt = ctypes.c_int(0)
    st = L.moe_model_inspect_file(str(path).encode(), ctypes.byref(cfg), ctypes.byref(dt))
    msg = L.moe_last_error().decode() if st else ""
    return st, cfg, dt.value, msg


def _write(path, entries, count=None):
    import qw3w
    qw3w.write(str(path), entries, count=count)
    return path


@pytest.mark.parametrize("dtype", [2, 3])
def test_valid_file_config(tmp_path, dtype):
    tm = _tiny(dtype)
    st, cfg, dt, msg = _inspect(_write(tmp_path / "ok.bin", _entries(tm), count=3))
    assert st == 0, msg
    assert dt == dtype
    assert (cfg.d_model, cfg.n_layers, cfg.head_dim, cfg.n_q, cfg.n_kv, cfg.d_ff, cfg.n_experts,
            cfg.top_k, cfg.vocab_size, cfg.causal) == (64, 2, 16, 4, 2, 32, 8, 8, 50, 1)
    assert cfg.rope_theta == np.float32(1e7) and cfg.rms_eps == np.float32(1e-6)


def _replace(entries, name, arr):
    out = [(n, arr if n == name else a) for n, a in entries]
    assert any(n == name for n, _ in entries), name
    return out


BAD = {
    # a q_proj that is a vector
    "q_rank": lambda e: _replace(e, "model.layers.1.self_attn.q_proj.weight", np.zeros(64 * 64, np.float32)),
    # o_proj transposed
    "o_shape": lambda e: _replace(e, "model.layers.0.self_attn.o_proj.weight", np.zeros((64, 32), np.float32)),
    # embedding with the wrong width
    "emb_width": lambda e: _replace(e, "model.embed_tokens.weight", np.zeros((50, 60), np.float32)),
    # untied head with fewer rows than the vocabulary
    "head_rows": lambda e: _replace(e, "lm_head.weight", np.zeros((49, 64), np.float32)),
    # a down projection of layer 1 with half its packed columns
    "down_cols": lambda e: _replace(e, "model.layers.1.mlp.experts.5.down_proj.weight.q4",
                                    np.zeros((64, 8), np.uint8)),
    # a scale vector one short
    "scale_len": lambda e: _replace(e, "model.layers.0.mlp.experts.2.gate_proj.weight.scale",
                                    np.ones(31, np.float32)),
    # the router stored as int8
    "router_dtype": lambda e: _replace(e, "model.layers.1.mlp.gate.weight", np.zeros((8, 64), np.int8)),
    # a bias of the wrong length
    "bias_len": lambda e: _replace(e, "model.layers.0.self_attn.k_proj.bias", np.zeros(33, np.float32)),
    # layer 1 lacks expert 7's up projection
    "missing_expert": lambda e: [(n, a) for n, a in e
                                 if not n.startswith("model.layers.1.mlp.experts.7.up_proj")],
    # layer 0's post-attention norm missing
    "missing_norm": lambda e: [(n, a) for n, a in e
                               if n != "model.layers.0.post_attention_layernorm.weight"],
    # q_norm (which sets head_dim) that does not divide the q rows
    "head_dim": lambda e: _replace(e, "model.layers.0.self_attn.q_norm.weight", np.ones(24, np.float32)),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_misshaped_tensor_rejected(tmp_path, case):
    entries = BAD[case](_entries(_tiny()))
    st, _, _, msg = _inspect(_write(tmp_path / f"{case}.bin", entries))
    assert st == MOE_ERR_ARG, (case, st, msg)
    assert msg.startswith("load:"), msg


def test_truncated_and_corrupt_headers(tmp_path):
    good = _write(tmp_path / "g.bin", _entries(_tiny()))
    raw = good.read_bytes()
    for n in (len(raw) - 1, len(raw) // 2, 11, 9):
        p = tmp_path / f"t{n}.bin"
        p.write_bytes(raw[:n])
        st, _, _, msg = _inspect(p)
        assert st == MOE_ERR_ARG, (n, msg)
    # first entry: its dimensions overwritten with 0, 0xFFFFFFFF, and a pair
    # whose product wraps 64 bits
    nl = struct.unpack_from("<I", raw, 10)[0]
    shape_off = 10 + 4 + nl + 8
    for dims in ((0, 64), (0xFFFFFFFF, 64), (0x7FFFFFFF, 0x7FFFFFFF)):
        b = bytearray(raw)
        struct.pack_into("<II", b, shape_off, *dims)
        p = tmp_path / "dims.bin"
        p.write_bytes(bytes(b))
        st, _, _, msg = _inspect(p)
        assert st == MOE_ERR_ARG, (dims, msg)
    # a dtype code outside 0..3, a rank above 8
    for off, val in ((10 + 4 + nl, 7), (10 + 4 + nl + 4, 9)):
        b = bytearray(raw)
        struct.pack_into("<I", b, off, val)
        p = tmp_path / "hdr.bin"
        p.write_bytes(bytes(b))
        st, _, _, msg = _inspect(p)
        assert st == MOE_ERR_ARG, (off, val, msg)
    p = tmp_path / "magic.bin"
    p.write_bytes(b"QW3X" + raw[4:])
    assert _inspect(p)[0] == MOE_ERR_ARG
    assert _inspect(tmp_path / "absent.bin")[0] == MOE_ERR_ARG
