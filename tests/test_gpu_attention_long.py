"""GPU parity of causal attention at real context lengths
(test_model_trace.c:399-425: the score, softmax and weighted-V loops over
every cached position), through the whole-model C ABI.

The model tests in test_gpu_model.py stay inside one 64-key block.  These
run the kernels' multi-block paths at configs[4]'s head geometry
(head_dim 128, 32 query heads, 4 KV heads) with small D and L:

* a 320-token prompt in one chunk: the query-tiled score kernel over five
  64-key blocks, the query-tiled softmax / V kernel with its V rows staged
  128 positions at a time (three stages);
* 70 single-token decode steps across two more key-block boundaries (320,
  384), each step's logits checked;
* a second prompt chunk at position 390 (query tiles at pos0 > 0);
* the per-row kernels for many rows (MOEHIP_ATTN_ROWWISE), which the
  library takes when the query-tiled kernel's LDS rows do not fit;
* 2060 cached positions (decode's scores no longer fit in registers,
  several 1024-position V chunks) and 4650 (the query-tiled kernel's LDS
  limit: the rowwise kernels take over by themselves), with 4 / 1 query
  heads so that the CPU oracle stays fast.

Bar: bit-exact against oracle/model_oracle.c's KV-cached forward, itself
pinned to the compiled reference's model_forward_f32 (tests/golden/
ref_model.json, tests/test_oracle_model.py).
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _check(got, want, what):
    np.testing.assert_array_equal(bits(got), bits(want), err_msg=what)


GEOM = dict(D=256, L=2, hd=128, nq=32, nkv=4, dff=128, E=16, V=300, dtype=3)


def test_long_prompt_decode_and_second_chunk(moehip):
    """configs[4]'s heads: 320-token prompt, 70 decode steps, a 70-token
    chunk at position 390, then forward_full of the whole sequence."""
    print("attention long: prompt 320 / decode 70 / chunk 70", flush=True)
    tm = O.TinyModel(seed=41, **GEOM)
    max_seq = 512
    m = moehip.model_from_tiny(tm, max_seq=max_seq)
    cache = tm.new_cache(max_seq)
    ids = (O.uniform_u32(320, 141) % tm.V).astype(np.int32)
    want = tm.forward_kv(ids, 0, cache)
    got, nxt = m.forward(ids)
    _check(got, want, "prompt 320")
    assert nxt == O.greedy(want)
    seq = ids.tolist()
    for step in range(70):
        seq.append(nxt)
        want = tm.forward_kv([nxt], len(seq) - 1, cache)
        got, nxt = m.forward([nxt])
        _check(got, want, f"decode step {step} (position {len(seq) - 1})")
        assert nxt == O.greedy(want)
    chunk = (O.uniform_u32(70, 142) % tm.V).astype(np.int32)
    want = tm.forward_kv(chunk, len(seq), cache)
    got, nxt = m.forward(chunk)
    _check(got, want, "chunk at 390")
    seq += chunk.tolist()
    assert m.position == len(seq) == 460
    _check(m.forward_full(seq), got, "forward_full of 460 tokens")
    m.close()


def test_long_rowwise_kernels(moehip, monkeypatch):
    """The per-row score and softmax / V kernels for many rows (the path
    taken when the query-tiled kernel's LDS rows do not fit): a 300-token
    prompt (three 128-position V chunks, the block-parallel exact sum of
    each row's exponentials), then a 9-token chunk and decode steps."""
    print("attention long: rowwise kernels, prompt 300", flush=True)
    monkeypatch.setenv("MOEHIP_ATTN_ROWWISE", "1")
    tm = O.TinyModel(seed=43, **GEOM)
    m = moehip.model_from_tiny(tm, max_seq=400)
    cache = tm.new_cache(400)
    ids = (O.uniform_u32(300, 143) % tm.V).astype(np.int32)
    want = tm.forward_kv(ids, 0, cache)
    got, nxt = m.forward(ids)
    _check(got, want, "rowwise prompt 300")
    chunk = (O.uniform_u32(9, 144) % tm.V).astype(np.int32)
    want = tm.forward_kv(chunk, 300, cache)
    got, nxt = m.forward(chunk)
    _check(got, want, "rowwise chunk at 300")
    pos = 309
    for step in range(12):
        want = tm.forward_kv([nxt], pos, cache)
        got, nxt = m.forward([nxt])
        _check(got, want, f"rowwise decode step {step}")
        pos += 1
    m.close()


def test_context_2060(moehip):
    """2060-token prompt, then decode past 2048 cached positions (the
    decode softmax reads its scores from memory instead of registers; its V
    sums run over three 1024-position chunks)."""
    print("attention long: prompt 2040 / decode to 2060", flush=True)
    tm = O.TinyModel(D=128, L=1, hd=128, nq=4, nkv=1, dff=128, E=16, V=300, dtype=3, seed=44)
    max_seq = 2100
    m = moehip.model_from_tiny(tm, max_seq=max_seq)
    cache = tm.new_cache(max_seq)
    ids = (O.uniform_u32(2040, 145) % tm.V).astype(np.int32)
    want = tm.forward_kv(ids, 0, cache)
    got, nxt = m.forward(ids)
    _check(got, want, "prompt 2040")
    pos = 2040
    for step in range(20):
        want = tm.forward_kv([nxt], pos, cache)
        got, nxt = m.forward([nxt])
        _check(got, want, f"decode at position {pos}")
        pos += 1
    m.close()


def test_context_past_tile_lds(moehip):
    """A 4600-token prompt (query-tiled kernels at their largest), then a
    50-token chunk at position 4600: 8 rows of 4652 scores no longer fit the
    query-tiled kernel's LDS, so the library runs the per-row kernels on
    its own; then decode steps."""
    print("attention long: prompt 4600 / chunk 50 / decode", flush=True)
    tm = O.TinyModel(D=128, L=1, hd=128, nq=1, nkv=1, dff=128, E=16, V=300, dtype=3, seed=45)
    max_seq = 4700
    m = moehip.model_from_tiny(tm, max_seq=max_seq)
    cache = tm.new_cache(max_seq)
    ids = (O.uniform_u32(4600, 146) % tm.V).astype(np.int32)
    want = tm.forward_kv(ids, 0, cache)
    got, nxt = m.forward(ids)
    _check(got, want, "prompt 4600")
    chunk = (O.uniform_u32(50, 147) % tm.V).astype(np.int32)
    want = tm.forward_kv(chunk, 4600, cache)
    got, nxt = m.forward(chunk)
    _check(got, want, "chunk at 4600")
    pos = 4650
    for step in range(4):
        want = tm.forward_kv([nxt], pos, cache)
        got, nxt = m.forward([nxt])
        _check(got, want, f"decode at position {pos}")
        pos += 1
    m.close()
