"""The KV-cached model restatement (oracle/model_oracle.c) against the
compiled reference's model_forward_f32 (test_model_trace.c:526-579), which
recomputes the whole prefix: tiny synthetic models are written as QW3W files
(moe.cc_amd/qw3w.py) and loaded by the reference's own bin_load +
load_all_weights (io.c:193-285, model.h:107-323).

Bit-exact: the logits of every step, for full prompts, step-by-step decode
and chunked prefill.  Needs oracle/_ref (build container only); the
reference-free checks at the end run everywhere.
"""
import os

import numpy as np
import pytest

import oracle as O
import qw3w

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")

MODELS = {
    # head_dim comes from q_norm's length (model.h:116-118); without q/k norm
    # the reference infers q rows / 32, hence 32 query heads there
    "q4": dict(dtype=3, seed=1),
    "q8_bias_tied": dict(dtype=2, seed=2, bias=True, untied=False),
    "q4_norms": dict(dtype=3, seed=3, random_norms=True, L=3),
    "q8_noqk": dict(dtype=2, seed=4, qk_norm=False, nq=32, hd=4, nkv=4, D=64),
    "q4_gqa8": dict(dtype=3, seed=5, nq=8, nkv=1, hd=8, D=32, dff=64, E=12),
}


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def ref_logits(path, ids, V):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty(V, np.float32)
    n = O.ref_trace().ref_model_forward_file(path.encode(), ids.ctypes.data, ids.size,
                                             out.ctypes.data, V)
    assert n == V
    return out


@pytest.fixture(scope="module")
def written(tmp_path_factory):
    d = tmp_path_factory.mktemp("qw3w")
    out = {}
    for name, kw in MODELS.items():
        m = O.TinyModel(**kw)
        path = str(d / f"{name}.bin")
        qw3w.write(path, qw3w.model_entries(m))
        out[name] = (m, path)
    return out


@needs_ref
@pytest.mark.parametrize("name", list(MODELS))
def test_full_prompt_matches_reference(written, name):
    m, path = written[name]
    ids = (O.uniform_u32(11, 40 + len(name)) % m.V).astype(np.int32)
    want = ref_logits(path, ids, m.V)
    got = m.forward_kv(ids, 0, m.new_cache(32))
    np.testing.assert_array_equal(bits(got), bits(want))


@needs_ref
@pytest.mark.parametrize("name", ["q4", "q8_bias_tied", "q4_gqa8"])
def test_kv_decode_matches_full_recompute(written, name):
    """Prefill 5 tokens, then 6 single-token steps: every step's logits equal
    the reference's recompute of the whole extended sequence."""
    m, path = written[name]
    seq = list((O.uniform_u32(5, 77) % m.V).astype(np.int32))
    cache = m.new_cache(16)
    got = m.forward_kv(seq, 0, cache)
    for step in range(6):
        np.testing.assert_array_equal(bits(got), bits(ref_logits(path, seq, m.V)),
                                      err_msg=f"step {step}")
        nxt = O.greedy(got)
        seq.append(nxt)
        got = m.forward_kv([nxt], len(seq) - 1, cache)


def test_chunked_prefill_equals_one_pass():
    m = O.TinyModel(**MODELS["q4_norms"])
    ids = (O.uniform_u32(9, 5) % m.V).astype(np.int32)
    c1 = m.new_cache(16)
    one, x1 = m.forward_kv(ids, 0, c1, return_x=True)
    c2 = m.new_cache(16)
    m.forward_kv(ids[:3], 0, c2)
    m.forward_kv(ids[3:7], 3, c2)
    two, x2 = m.forward_kv(ids[7:], 7, c2, return_x=True)
    np.testing.assert_array_equal(bits(one), bits(two))
    np.testing.assert_array_equal(bits(x1[7:]), bits(x2))
    np.testing.assert_array_equal(bits(c1[0][:, :, :9]), bits(c2[0][:, :, :9]))


def test_single_layer_attention_closed_form():
    """One position, one head: softmax over a single score is exactly 1, so
    the attention output is the (rotated-free at position 0) V row, and the
    layer's attention part equals Wo (Wv x_norm1) computed by matmul_f32."""
    m = O.TinyModel(D=32, L=1, hd=8, nq=2, nkv=1, dff=32, E=8, dtype=3, seed=9, qk_norm=False)
    lw = m.layers[0]
    x = m.tok_emb[[3]].copy()
    xn1 = O.rmsnorm(x, lw["rms1_w"])
    v = O.matmul_f32(xn1, lw["Wv"])                    # [1, hd]
    h = np.concatenate([v, v], axis=1)                # both query heads read kv head 0
    att = O.matmul_f32(h, lw["Wo"])
    xa = x + att
    want, _, _, _ = O.moe_block(O.rmsnorm(xa, lw["rms2_w"]), xa, lw["router_w"], None,
                                lw["experts"], top_k=8)
    kc, vc = m.new_cache(4)
    xx = x.copy()
    O.orc().orc_layer_rows(O.ctypes.byref(m.cfg), O.ctypes.addressof(m._layers[0]),
                           xx.ctypes.data, 1, 0, kc.ctypes.data, vc.ctypes.data, 4)
    np.testing.assert_array_equal(bits(xx), bits(want))
    np.testing.assert_array_equal(bits(vc[0, 0, 0]), bits(v[0]))


def test_rope_tables_closed_form():
    """Position 0 is the identity rotation; frequency i = 0 turns by exactly
    pos radians; elsewhere the tables agree with float64 trigonometry of the
    exact angle up to the float32 roundings of the frequency and the angle
    (a few ulps of the angle) plus one ulp of the result."""
    c, s = O.rope_tables(128, 1e7, 64)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    pos = np.arange(64, dtype=np.float64)
    np.testing.assert_allclose(c[:, 0], np.cos(pos), rtol=0, atol=2e-7)
    np.testing.assert_allclose(s[:, 0], np.sin(pos), rtol=0, atol=2e-7)
    ang = pos[:, None] * 1e7 ** (-2.0 * np.arange(64)[None, :] / 128.0)
    tol = 3 * np.spacing(ang.astype(np.float32)).astype(np.float64) + 1.2e-7
    assert np.all(np.abs(c - np.cos(ang)) <= tol)
    assert np.all(np.abs(s - np.sin(ang)) <= tol)
    # a wrong pairing (sin for cos) or a dropped factor 2 in the exponent fails
    ang2 = pos[:, None] * 1e7 ** (-1.0 * np.arange(64)[None, :] / 128.0)
    assert not np.all(np.abs(c - np.cos(ang2)) <= tol)


def _ref_probs(v):
    p = np.array(v, np.float32, copy=True)
    O.ref_trace().ref_softmax_rows(p.ctypes.data, 1, p.size)
    return p


def _near_ties(rng, n):
    """Logit rows whose top values sit within a few ulps of each other, so
    that several of them round to the same probability."""
    v = rng.normal(0.0, 1.0, n).astype(np.float32)
    top = np.float32(rng.uniform(0.25, 4.0))
    for j in rng.choice(n, 4, replace=False):
        v[j] = top
        for _ in range(int(rng.integers(0, 6))):
            v[j] = np.nextafter(v[j], np.float32(-np.inf) if rng.random() < 0.5 else np.float32(np.inf))
    return v


@needs_ref
def test_greedy_is_argmax_of_reference_softmax():
    """O.greedy against the compiled reference's softmax_rows (:736) plus the
    first-index scan of :740-746 (numpy's argmax returns the first maximum)."""
    rng = np.random.default_rng(5)
    for trial in range(300):
        n = int(rng.integers(2, 3000))
        v = _near_ties(rng, n) if trial % 2 else rng.normal(0, 3, n).astype(np.float32)
        p = _ref_probs(v)
        assert O.greedy(v) == int(np.argmax(p)), trial


@needs_ref
def test_greedy_known_answers():
    """Logits one ulp apart whose probabilities are equal keep the lower
    index (the logits' argmax would take the other); NaN or +inf anywhere,
    or all -inf, make every probability NaN, and the scan stays at 0."""
    a = np.float32(0.3)
    v = np.array([-1.0, a, np.nextafter(a, np.float32(1.0)), 0.1], np.float32)
    p = _ref_probs(v)
    assert p[1] == p[2] and int(np.argmax(v)) == 2
    assert O.greedy(v) == 1
    for bad in ([1.0, np.nan, 5.0], [1.0, np.inf, 2.0], [-np.inf, -np.inf], [np.nan, 3.0]):
        bad = np.array(bad, np.float32)
        assert np.all(np.isnan(_ref_probs(bad)))
        assert O.greedy(bad) == 0
    assert O.greedy(np.array([-np.inf, 2.0, 3.0, -np.inf], np.float32)) == 2
    assert O.greedy(np.array([0.5, 2.0, -1.0, 2.0, 1.0], np.float32)) == 1


def test_greedy_equals_unit_exponential_rule():
    """The rule the device uses: with m = max (finite), the answer is the
    first i with expf(v_i - m) == 1 (the row maximum has probability
    1 * inv exactly and any e_i < 1 rounds below it), else 0 when a NaN or
    +inf logit is present or every logit is -inf."""
    rng = np.random.default_rng(9)

    def rule(v):
        if np.isnan(v).any() or np.isposinf(v).any() or np.isneginf(v).all():
            return 0
        m = v.max()
        e = np.empty_like(v)
        d = (v - m).astype(np.float32)
        O.orc().orc_expf_array(O._c(d), O._c(e), d.size)
        return int(np.flatnonzero(e == np.float32(1.0))[0])

    for trial in range(400):
        n = int(rng.integers(1, 2000))
        v = _near_ties(rng, n) if (trial % 2 and n >= 4) else rng.normal(0, 1, n).astype(np.float32)
        if trial % 7 == 0:
            v[rng.integers(0, n)] = -np.inf
        assert O.greedy(v) == rule(v), trial


def test_qw3w_round_trip(tmp_path):
    m = O.TinyModel(**MODELS["q8_bias_tied"])
    path = str(tmp_path / "m.bin")
    n = qw3w.write(path, qw3w.model_entries(m), count=7)   # undercounted header is tolerated
    with qw3w.File(path) as f:
        assert f.header_count == 7 and len(f.index) == n
        np.testing.assert_array_equal(f.get("model.embed_tokens.weight"), m.tok_emb)
        ex = m.layers[1]["experts"]
        np.testing.assert_array_equal(f.get(qw3w.expert_name(1, 3, "down") + ".q8"), ex.dq[3])
        np.testing.assert_array_equal(f.get(qw3w.expert_name(1, 3, "down") + ".scale"), ex.ds[3])
        assert "lm_head.weight" not in f


def test_qw3w_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(b"QW3X\x00\x01\x00\x00\x00\x00")
    with pytest.raises(ValueError):
        qw3w.File(str(p))
    good = tmp_path / "t.bin"
    qw3w.write(str(good), [("a", np.ones(4, np.float32))])
    data = good.read_bytes()
    (tmp_path / "trunc.bin").write_bytes(data[:-3])
    with pytest.raises(ValueError):
        qw3w.File(str(tmp_path / "trunc.bin"))


GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_model.json")


def _model_cases():
    import json
    with open(GOLD) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _model_cases(), ids=lambda c: c["tag"])
def test_model_golden(case):
    """The restatement's KV-cached greedy run reproduces the compiled
    reference's logits digests and continuation (tests/golden/ref_model.json)."""
    import hashlib
    m = O.TinyModel(**case["model"])
    cache = m.new_cache(len(case["prompt"]) + len(case["greedy"]) + 1)
    lg = m.forward_kv(case["prompt"], 0, cache)
    pos = len(case["prompt"])
    for step, (want_sha, first8, nxt) in enumerate(zip(case["logits_sha"], case["logits_first8"],
                                                       case["greedy"])):
        np.testing.assert_array_equal(lg[:8], np.array(first8, np.float32), err_msg=f"step {step}")
        assert hashlib.sha256(lg.tobytes()).hexdigest() == want_sha, f"step {step}"
        assert O.greedy(lg) == nxt
        lg = m.forward_kv([nxt], pos, cache)
        pos += 1


@needs_ref
@pytest.mark.parametrize("seed", range(4))
def test_softmax_rows_matches_reference(seed):
    x = O.normal(3 * 1000, 900 + seed, 0.0, 4.0).reshape(3, 1000)
    x[1, 0] = np.nan if seed == 1 else x[1, 0]
    x[2, 5:9] = x[2].max() if seed == 2 else x[2, 5:9]
    want = x.copy()
    O.ref_trace().ref_softmax_rows(want.ctypes.data, 3, 1000)
    np.testing.assert_array_equal(bits(O.softmax_rows(x)), bits(want))


def test_softmax_rows_closed_form():
    """Equal inputs give 1/n each (up to the 1e-9 in the denominator, below
    an ulp here); shifting all inputs by a constant changes nothing."""
    out = O.softmax_rows(np.zeros((1, 8), np.float32))
    np.testing.assert_array_equal(out, np.full((1, 8), np.float32(1.0) / np.float32(8.0 + 1e-9)))
    x = O.normal(64, 3, 0.0, 1.0).reshape(1, 64)
    a, b = O.softmax_rows(x), O.softmax_rows(x + np.float32(0.0))
    np.testing.assert_array_equal(a, b)
    np.testing.assert_allclose(a.sum(), 1.0, rtol=1e-5)
