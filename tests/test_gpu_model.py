"""GPU parity of the whole model (test_model_trace.c:526-579) and of the
exact fp32 products (test_model_trace.c:213-227, kernels.c:153-165) through
the C ABI.

Bar: bit-exact.  Every fp32 sum is the reference's sequential chain, the
expert dots are exact integers, expf matches glibc and the RoPE tables come
from the same C library calls, so logits, hidden states and greedy tokens
are compared bit for bit with the oracle (oracle/model_oracle.c, itself
pinned to the compiled reference: tests/test_oracle_model.py,
tests/golden/ref_model.json).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_model.json")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def f32_dev(moehip, A, W):
    M, K = A.shape
    N = W.shape[0]
    dA, dW = moehip.DeviceBuffer.from_array(A), moehip.DeviceBuffer.from_array(W)
    dC = moehip.DeviceBuffer(max(1, M * N * 4))
    moehip.check(moehip.lib().moe_matmul_f32_dev(dA.ptr, dW.ptr, dC.ptr, M, N, K), "f32")
    return dC.download((M, N), np.float32)


# (M, N, K): one-wave GEMV with 16 / 32 / 64 rows per wave (chunk tails,
# rows past N), the row kernels (a block per row and token up to 4 tokens;
# four 128-thread token groups per block for 5-16 tokens, a partial last
# group), the LDS tile kernel at both tile sizes (token and row tails;
# 64 x 64 tiles from 1024 blocks: the last shape), and the unaligned
# fallback (K % 4 != 0)
F32_SHAPES = [(1, 37, 2048), (1, 5120, 2048), (3, 100, 4100), (4, 2048, 4096), (2, 33000, 64),
              (1, 70000, 68), (5, 77, 300), (9, 128, 2048), (16, 1024, 4096), (13, 3, 64),
              (40, 130, 2048), (300, 96, 260), (2, 10, 7), (7, 13, 1001), (1, 1, 4),
              (1030, 4100, 260)]


@pytest.mark.parametrize("M,N,K", F32_SHAPES)
def test_f32_products_bit_exact(moehip, M, N, K):
    print("f32 case", M, N, K, flush=True)
    A = O.normal(M * K, 31 + M + K, 0.0, 1.0).reshape(M, K)
    W = O.normal(N * K, 37 + N, 0.0, 0.05).reshape(N, K)
    np.testing.assert_array_equal(bits(f32_dev(moehip, A, W)), bits(O.matmul_f32(A, W)))


def test_f32_special_values(moehip):
    """inf / NaN / huge values propagate exactly as in the sequential loop."""
    A = O.normal(4 * 520, 5, 0.0, 1.0).reshape(4, 520)
    W = O.normal(9 * 520, 6, 0.0, 1.0).reshape(9, 520)
    A[0, 3] = np.inf
    A[1, 100] = np.nan
    A[2, :] *= 1e30
    W[4, 7] = -np.inf
    np.testing.assert_array_equal(bits(f32_dev(moehip, A, W)), bits(O.matmul_f32(A, W)))


def _planted_logits(n, seed, plant):
    """N(0, 0.05) logits (all below 0.3) with `plant` = {index: value}
    written over them."""
    v = O.normal(n, seed, 0.0, 0.05).astype(np.float32)
    for i, x in plant.items():
        v[i] = x
    return v


A03 = np.float32(0.3)
B03 = np.nextafter(A03, np.float32(0.0))          # one ulp under: same probability
GREEDY_CASES = [  # (n, plant)
    (151936, {140000: A03, 70001: B03}),           # tie across blocks: the lower index
    (151936, {9: A03, 5: B03, 151935: B03}),       # tie inside one block
    (151936, {3: A03, 100000: np.float32(np.nan)}),  # NaN anywhere -> 0
    (151936, {77: np.float32(np.inf)}),            # +inf -> 0
    (151936, {}),                                  # plain maximum
    (1000, {999: A03, 500: B03}),
    (1000, {17: np.float32(-np.inf)}),
    (1, {}),
]


@pytest.mark.parametrize("n,plant", GREEDY_CASES)
def test_greedy_dev_and_fused_head(moehip, n, plant):
    """The next-token choice against the oracle's literal softmax + scan
    (test_model_trace.c:735-746): the full-scan kernel on given logits, and
    the head product with its block maxima.  With x = e_0 the product's
    logits are W[:, 0] exactly (the other columns add signed zeros), so the
    planted values reach the choice unchanged."""
    print("greedy case", n, sorted(plant), flush=True)
    v = _planted_logits(n, 60 + n, plant)
    want = O.greedy(v)
    dv = moehip.DeviceBuffer.from_array(v)
    dn = moehip.DeviceBuffer(4)
    moehip.check(moehip.lib().moe_greedy_dev(dv.ptr, n, dn.ptr), "greedy")
    assert int(dn.download((1,), np.int32)[0]) == want
    K = 64
    W = O.normal(n * K, 61 + n, 0.0, 0.05).reshape(n, K)
    W[:, 0] = v
    x = np.zeros(K, np.float32)
    x[0] = 1.0
    dx, dW = moehip.DeviceBuffer.from_array(x), moehip.DeviceBuffer.from_array(W)
    dl = moehip.DeviceBuffer(n * 4)
    moehip.check(moehip.lib().moe_head_greedy_dev(dx.ptr, dW.ptr, n, K, dl.ptr, dn.ptr), "head")
    lg = dl.download((n,), np.float32)
    np.testing.assert_array_equal(bits(lg), bits(O.matmul_f32(x[None, :], W)[0]))
    np.testing.assert_array_equal(bits(lg), bits(v))
    assert int(dn.download((1,), np.int32)[0]) == want


def _golden_cases():
    with open(GOLD) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["tag"])
def test_model_golden_greedy(moehip, case):
    """Prompt then greedy steps: every step's logits equal the oracle's and
    the digest the compiled reference wrote; generate() returns the
    reference's continuation."""
    print("model golden", case["tag"], flush=True)
    tm = O.TinyModel(**case["model"])
    n = len(case["greedy"])
    m = moehip.model_from_tiny(tm, max_seq=len(case["prompt"]) + n + 1)
    cache = tm.new_cache(len(case["prompt"]) + n + 1)
    want = tm.forward_kv(case["prompt"], 0, cache)
    got, nxt = m.forward(case["prompt"])
    pos = len(case["prompt"])
    for step in range(n):
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=f"step {step}")
        assert hashlib.sha256(got.tobytes()).hexdigest() == case["logits_sha"][step]
        assert nxt == case["greedy"][step]
        want = tm.forward_kv([nxt], pos, cache)
        got, nxt = m.forward([nxt])
        pos += 1
    ids, _, _ = m.generate(case["prompt"], n)
    assert ids.tolist() == case["greedy"]
    m.close()


MODEL_CASES = {
    # hd 128 with 8/2 heads; 40-token prompt: tile products and grouped experts
    "q4_hd128": dict(D=256, L=2, hd=128, nq=8, nkv=2, dff=256, E=32, V=300, dtype=3, seed=21),
    "q8_bias_norms": dict(D=256, L=2, hd=64, nq=4, nkv=4, dff=256, E=16, V=257, dtype=2,
                          seed=22, bias=True, random_norms=True, untied=False),
    "q4_gqa_noqk": dict(D=128, L=1, hd=4, nq=32, nkv=4, dff=256, E=16, V=129, dtype=3, seed=23,
                        qk_norm=False),
}


@pytest.mark.parametrize("name", list(MODEL_CASES))
def test_model_prefill_chunks_and_decode(moehip, name):
    """A 40-token prompt in chunks of 3, 32 and 5 tokens (GEMV, tile and
    expert-major paths), then 6 decode steps; logits equal the oracle's at
    every call, and forward_full of the whole sequence equals the last step."""
    print("model case", name, flush=True)
    tm = O.TinyModel(**MODEL_CASES[name])
    m = moehip.model_from_tiny(tm, max_seq=64)
    ids = (O.uniform_u32(40, 99) % tm.V).astype(np.int32)
    cache = tm.new_cache(64)
    seq = []
    for lo, hi in ((0, 3), (3, 35), (35, 40)):
        want = tm.forward_kv(ids[lo:hi], lo, cache)
        got, nxt = m.forward(ids[lo:hi])
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=f"chunk {lo}:{hi}")
        assert nxt == O.greedy(want)
    seq = ids.tolist()
    for step in range(6):
        seq.append(nxt)
        want = tm.forward_kv([nxt], len(seq) - 1, cache)
        got, nxt = m.forward([seq[-1]])
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=f"step {step}")
    full = m.forward_full(seq)
    np.testing.assert_array_equal(bits(full), bits(got))
    probs = m.forward_full(seq, apply_softmax=True)
    np.testing.assert_array_equal(bits(probs), bits(O.softmax_rows(got)[0]))
    assert m.position == len(seq)
    m.close()


def test_model_load_qw3w_file(moehip, tmp_path):
    """moe_model_load_file reads the reference's container (io.c:193-285) and
    infers the config as load_all_weights does (model.h:110-163)."""
    import qw3w
    tm = O.TinyModel(D=64, L=2, hd=16, nq=4, nkv=2, dff=64, E=16, V=97, dtype=3, seed=24, bias=True)
    path = str(tmp_path / "m.bin")
    qw3w.write(path, qw3w.model_entries(tm), count=3)
    m = moehip.Model.load_file(path, max_seq=32)
    assert (m.cfg.d_model, m.cfg.n_layers, m.cfg.head_dim, m.cfg.n_q, m.cfg.n_kv, m.cfg.d_ff,
            m.cfg.n_experts, m.cfg.top_k, m.cfg.vocab_size) == (64, 2, 16, 4, 2, 64, 16, 8, 97)
    ids = (O.uniform_u32(9, 7) % tm.V).astype(np.int32)
    want = tm.forward_kv(ids, 0, tm.new_cache(32))
    np.testing.assert_array_equal(bits(m.forward_full(ids)), bits(want))
    m.close()


def test_model_errors(moehip, tmp_path):
    tm = O.TinyModel(D=64, L=1, hd=16, nq=4, nkv=2, dff=32, E=16, V=50, dtype=3, seed=25)
    m = moehip.model_from_tiny(tm, max_seq=8)
    with pytest.raises(moehip.MoeError):
        m.forward(np.arange(9, dtype=np.int32) % 50)      # past max_seq
    with pytest.raises(moehip.MoeError):
        m.forward([50])                                   # id outside the vocabulary
    m.reset()
    got, _ = m.forward([1, 2])
    want = tm.forward_kv([1, 2], 0, tm.new_cache(8))
    np.testing.assert_array_equal(bits(got), bits(want))
    m.close()
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"QW3X\x00\x01\x00\x00\x00\x00")
    with pytest.raises(moehip.MoeError):
        moehip.Model.load_file(str(bad))


def test_synthetic_model_generate_consistent(moehip):
    """A synthetic model made on the device: generate() (device-fed ids)
    matches step-by-step forwards, and the KV-cached last step equals a full
    recompute of the sequence (the reference's way)."""
    cfg = moehip.qwen_config(512, 2, 128, 8, 2, 256, 32, 8, 1000)
    m = moehip.Model.synthetic(cfg, expert_dtype=3, seed=5, max_seq=128)
    prompt = (O.uniform_u32(50, 3) % 1000).astype(np.int32)
    ids, ms_p, ms_d = m.generate(prompt, 8)
    assert ms_p > 0 and ms_d > 0
    m.reset()
    lg, nxt = m.forward(prompt)
    seq = prompt.tolist()
    steps = [nxt]
    for _ in range(7):
        seq.append(steps[-1])
        lg, nxt = m.forward([steps[-1]])
        steps.append(nxt)
    assert steps == ids.tolist()
    np.testing.assert_array_equal(bits(m.forward_full(seq)), bits(lg))
    m.close()
