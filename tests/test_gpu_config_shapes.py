"""GPU parity at the BASELINE configs' own shapes and launch geometry.

* the batch-1 GEMV pools exactly as bench.py times
  them (bench.Pool: 1 GiB of distinct matrices per shape, one shared packed
  activation table, one prepacked launch over all matrices), so the tiled
  kernel runs with the rows per block and row groups per wave the headline
  measures (kernels.c:51-128).
* the prefill layer at its config shape (E = 128, D = 2048,
  d_ff = 768, Q4) at T = 512 (test_model_trace.c:463-517); T = 2048 is
  test_gpu_layer.py's test_grouped_config_shape_T2048.
* a full-width model -- D = 2048, 32 query / 4 KV heads of 128,
  128 Q4 experts of d_ff 768, an untied 151,936-row head -- with two layers,
  a 512-token prompt in one chunk and 8 greedy decode steps, every step's
  logits and greedy choice against the oracle's KV-cached forward
  (test_model_trace.c:526-579, :341-430, :735-746); and the 48-layer model
  bench.py decodes, checked for self-consistency (device-fed generation
  equals step-by-step forwards, and the last step equals a full recompute
  through the prefill kernels).

Bar: bit-exact (the oracle is pinned to the compiled reference: see
tests/test_oracle_model.py and tests/golden/).  The large weights are made
by the library's seeded device generator and quantizer and downloaded, so
both sides read the same bytes; which generator made them does not matter
for parity.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------- the timed GEMV pools ----------------

@pytest.mark.parametrize("dtype,N,K", [(3, 2048, 768), (3, 768, 2048), (2, 768, 2048)])
def test_bench_gemv_pool_bit_exact(moehip, dtype, N, K):
    """bench.py's pool and launch, every output of every matrix checked: the
    pool's matrices stacked are one [count*N x K] matrix against the one x,
    so the oracle checks them in one product."""
    import bench
    count = bench.pool_count(dtype, N, K)
    print("bench pool case", dtype, N, K, count, moehip.gemv_variant(dtype, 1, N, K), flush=True)
    pool = bench.Pool(dtype, N, K, count, seed=1000)
    pool.pack()
    pool.launch()
    moehip.synchronize()
    rb = K if dtype == 2 else K // 2
    q = pool.q.download((count * N, rb), np.int8 if dtype == 2 else np.uint8)
    s = pool.s.download((count * N,), np.float32)
    x = pool.x.download((1, K), np.float32)
    y = pool.y.download((count * N,), np.float32)
    with O.threaded():
        want = (O.gemv_q8 if dtype == 2 else O.gemv_q4)(x, q, s, count * N, K)[0]
    bad = np.flatnonzero(bits(y) != bits(want))
    assert bad.size == 0, f"{bad.size} outputs differ, first at matrix {bad[0] // N} row {bad[0] % N}"
    # a second launch from the same tables (the bench's steady state) is identical
    pool.y.zero()
    pool.launch()
    np.testing.assert_array_equal(bits(pool.y.download((count * N,), np.float32)), bits(want))


# ---------------- the prefill layer at its config shape ----------------

def _random_experts(dtype, E, D, dff, seed):
    rg = D if dtype == 2 else D // 2
    rd = dff if dtype == 2 else dff // 2
    rng = np.random.default_rng(seed)
    gq = rng.integers(0, 256, (E, dff, rg), dtype=np.uint8)
    uq = rng.integers(0, 256, (E, dff, rg), dtype=np.uint8)
    dq = rng.integers(0, 256, (E, D, rd), dtype=np.uint8)
    if dtype == 2:
        gq, uq, dq = (np.where(a == 128, 0, a).view(np.int8) for a in (gq, uq, dq))
    gs = np.abs(O.normal(E * dff, seed + 3, 0.0, 2e-4)).reshape(E, dff)
    us = np.abs(O.normal(E * dff, seed + 4, 0.0, 2e-4)).reshape(E, dff)
    ds = np.abs(O.normal(E * D, seed + 5, 0.0, 2e-4)).reshape(E, D)
    return O.ExpertSet(dtype, gq, gs, uq, us, dq, ds, D, dff)


@pytest.mark.parametrize("T", [512])
def test_prefill_layer_config_shape(moehip, T):
    """configs[3] (Q4, E = 128, D = 2048, d_ff = 768, top-8, x = RMSNorm of
    N(0, 1)) through the default path (expert-major from 32 tokens): T = 512
    selects the 64-pair task shape; against the threaded oracle."""
    dtype, E, D, dff = 3, 128, 2048, 768
    seed = 9900 + T
    print("prefill config-shape case T =", T, flush=True)
    ex = _random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    xr = O.normal(T * D, seed + 13, 0.0, 1.0).reshape(T, D)
    xn = O.rmsnorm(xr, None, 1e-6)
    with O.threaded():
        want, widx, wp, wlog = O.moe_block(xn, xr, rw, None, ex)
    layer = moehip.MoeLayer.from_arrays(dtype, rw, None, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds)
    got, idx, p = layer.forward(xn, xr)
    dbg = layer.debug(T)
    np.testing.assert_array_equal(bits(dbg["logits"]), bits(wlog))
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))
    layer.close()


# ---------------- the model at its own width ----------------

FULL = dict(D=2048, hd=128, nq=32, nkv=4, dff=768, E=128, V=151936)


def _dev_normal(M, shape, seed, mean=0.0, std=0.02):
    n = int(np.prod(shape))
    b = M.DeviceBuffer(n * 4)
    M.check(M.lib().moe_fill_normal_dev(b.ptr, n, seed, mean, std), "fill")
    out = b.download(shape, np.float32)
    b.free()
    return out


def _dev_experts(M, dtype, E, D, dff, seed, tmp):
    """Experts made as the exporter would (N(0, 0.02^2), rowwise Q4/Q8), on
    the device, downloaded."""
    qdt = np.int8 if dtype == 2 else np.uint8
    out = []
    for j, (rows, K) in enumerate(((dff, D), (dff, D), (D, dff))):
        rb = K if dtype == 2 else K // 2
        qb, sb = M.DeviceBuffer(E * rows * rb), M.DeviceBuffer(E * rows * 4)
        M.check(M.lib().moe_fill_normal_dev(tmp.ptr, E * rows * K, seed + j, 0.0, 0.02), "fill")
        M.check(M.lib().moe_quantize_rows_dev(dtype, tmp.ptr, E * rows, K, qb.ptr, sb.ptr), "quant")
        out += [qb.download((E, rows, rb), qdt), sb.download((E, rows), np.float32)]
        qb.free()
        sb.free()
    gq, gs, uq, us, dq, ds = out
    return O.ExpertSet(dtype, gq, gs, uq, us, dq, ds, D, dff)


def _full_width_model(M, L, dtype, seed):
    c = FULL
    D, hd, nq, nkv, dff, E, V = c["D"], c["hd"], c["nq"], c["nkv"], c["dff"], c["E"], c["V"]
    sd = [seed * 1000]

    def nrm(*shape, mean=0.0, std=0.02):
        sd[0] += 1
        return _dev_normal(M, shape, sd[0], mean, std)

    tmp = M.DeviceBuffer(E * dff * D * 4)
    tok, head = nrm(V, D), nrm(V, D)
    ones_d, ones_h = np.ones(D, np.float32), np.ones(hd, np.float32)
    layers = []
    for _ in range(L):
        lw = {"Wq": nrm(nq * hd, D), "Wk": nrm(nkv * hd, D), "Wv": nrm(nkv * hd, D),
              "Wo": nrm(D, nq * hd), "q_norm": ones_h, "k_norm": ones_h, "rms1_w": ones_d,
              "rms2_w": ones_d, "router_w": nrm(E, D)}
        sd[0] += 10
        lw["experts"] = _dev_experts(M, dtype, E, D, dff, sd[0], tmp)
        layers.append(lw)
    tmp.free()
    return O.TinyModel.from_weights(D, L, hd, nq, nkv, dff, E, V, dtype, tok, ones_d, head, layers)


def test_full_width_model_prompt_512_and_decode(moehip):
    """configs[4] at its own width with two layers: a 512-token prompt in one
    chunk (the tile products, the expert-major MoE path, the query-tiled
    attention over eight 64-key blocks), then 8 decode steps (the one-token
    kernels, the fused 151,936-row head and greedy choice at K = 2048), each
    step's logits bit for bit against the oracle; then forward_full of the
    whole 520-token sequence equals the last step."""
    print("full-width model: generating", flush=True)
    tm = _full_width_model(moehip, 2, 3, seed=31)
    max_seq = 2048
    m = moehip.model_from_tiny(tm, max_seq=max_seq)
    ids = (O.uniform_u32(512, 777) % tm.V).astype(np.int32)
    cache = tm.new_cache(max_seq)
    print("full-width model: prompt 512", flush=True)
    got, nxt = m.forward(ids)
    with O.threaded():
        want = tm.forward_kv(ids, 0, cache)
    np.testing.assert_array_equal(bits(got), bits(want), err_msg="prompt 512")
    assert nxt == O.greedy(want)
    seq = ids.tolist()
    for step in range(8):
        seq.append(nxt)
        got, nxt = m.forward([nxt])
        with O.threaded():
            want = tm.forward_kv([seq[-1]], len(seq) - 1, cache)
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=f"decode step {step}")
        assert nxt == O.greedy(want), f"greedy at step {step}"
    print("full-width model: forward_full of", len(seq), flush=True)
    np.testing.assert_array_equal(bits(m.forward_full(seq)), bits(got))
    m.close()


def test_48_layer_model_generate_consistent(moehip):
    """The 48-layer configs[4] model bench.py decodes (same seed and
    construction): generate() with device-fed ids equals step-by-step
    forwards, and the last step's logits equal forward_full of the whole
    sequence (the recompute runs the prefill kernels: tile products,
    expert-major MoE, query-tiled attention)."""
    import bench
    c = bench.QWEN3_30B_A3B
    cfg = moehip.qwen_config(c["D"], c["L"], c["hd"], c["nq"], c["nkv"], c["dff"], c["E"],
                             c["top_k"], c["V"])
    print("48-layer model: building", flush=True)
    m = moehip.Model.synthetic(cfg, expert_dtype=3, untied_head=True, seed=2024, std=0.02,
                               max_seq=2048)
    prompt = np.random.default_rng(512).integers(0, c["V"], 64).astype(np.int32)
    ids, _, _ = m.generate(prompt, 9)
    m.reset()
    lg, nxt = m.forward(prompt)
    seq = prompt.tolist()
    steps = [nxt]
    for _ in range(8):
        seq.append(steps[-1])
        lg, nxt = m.forward([steps[-1]])
        steps.append(nxt)
    assert steps == ids.tolist()
    print("48-layer model: forward_full of", len(seq), flush=True)
    np.testing.assert_array_equal(bits(m.forward_full(seq)), bits(lg))
    m.close()
