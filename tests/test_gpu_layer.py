"""GPU parity of the MoE block (test_model_trace.c:460-517) through the C ABI.

Bar: bit-exact outputs, top-k indices and gates.  The router sums in the
reference's order, the expert dots are exact integers, expf matches glibc and
every fp32 step is a separately rounded IEEE operation, so nothing is left to
tolerance.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def random_experts(dtype, E, D, dff, seed):
    """Fast synthetic experts: uniform weight bytes, small normal scales."""
    rg = D if dtype == 2 else D // 2
    rd = dff if dtype == 2 else dff // 2

    def qbytes(n, s):
        u = O.uniform_u32(n, s)
        if dtype == 2:
            return ((u % 255).astype(np.int64) - 127).astype(np.int8)
        return (u & 0xFF).astype(np.uint8)

    gq = qbytes(E * dff * rg, seed).reshape(E, dff, rg)
    uq = qbytes(E * dff * rg, seed + 1).reshape(E, dff, rg)
    dq = qbytes(E * D * rd, seed + 2).reshape(E, D, rd)
    gs = np.abs(O.normal(E * dff, seed + 3, 0.0, 2e-4)).reshape(E, dff)
    us = np.abs(O.normal(E * dff, seed + 4, 0.0, 2e-4)).reshape(E, dff)
    ds = np.abs(O.normal(E * D, seed + 5, 0.0, 2e-4)).reshape(E, D)
    return O.ExpertSet(dtype, gq, gs, uq, us, dq, ds, D, dff)


def make_layer(moehip, dtype, ex, rw, rb=None, rms2=None, top_k=8):
    return moehip.MoeLayer.from_arrays(dtype, rw, rb, ex.gq, ex.gs, ex.uq, ex.us, ex.dq, ex.ds,
                                       rms2_w=rms2, top_k=top_k)


@pytest.mark.parametrize("tag", ["q8", "q4"])
def test_golden_small_layers(moehip, tag):
    with np.load(os.path.join(GOLD, "ref_small.npz")) as z:
        pre = f"layer_{tag}_"
        dtype, T, D, dff, E = (int(v) for v in z[pre + "dims"])
        ex = O.ExpertSet(dtype, z[pre + "gq"], z[pre + "gs"], z[pre + "uq"], z[pre + "us"],
                         z[pre + "dq"], z[pre + "ds"], D, dff)
        x, rw, rms2, want = z[pre + "x"], z[pre + "rw"], z[pre + "rms2"], z[pre + "out"]
        rb = z[pre + "rb"] if (pre + "rb") in z.files else None
    layer = make_layer(moehip, dtype, ex, rw, rb, rms2)
    got = layer.block_forward(x)
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("tag", ["layer_q8_T4", "layer_q4_T2", "layer_q8_T64", "layer_q4_T128"])
def test_config_layers_vs_reference_digest(moehip, tag):
    with open(os.path.join(GOLD, "ref_config.json")) as f:
        c = next(c for c in json.load(f)["cases"] if c["tag"] == tag)
    print("case", tag, flush=True)
    ex = O.make_experts(c["dtype"], c["E"], c["D"], c["d_ff"], c["seed"], c["std_w"])
    assert sha(ex.gq) == c["sha_gq"]
    T, D = c["T"], c["D"]
    x = O.normal(T * D, c["seed"] + 1, 0.0, 1.0).reshape(T, D)
    rw = O.normal(c["E"] * D, c["seed"] + 2, 0.0, c["std_w"]).reshape(c["E"], D)
    layer = make_layer(moehip, c["dtype"], ex, rw, None, np.ones(D, np.float32))
    out = layer.block_forward(x)
    assert sha(out) == c["sha_out"]


CASES = [  # dtype, T, E, D, d_ff, bias, resid
    (2, 1, 128, 2048, 768, False, True),
    (2, 4, 128, 2048, 768, True, True),
    (2, 16, 128, 2048, 768, False, False),
    (3, 1, 128, 2048, 768, False, True),
    (3, 5, 128, 2048, 768, True, True),
    (3, 16, 128, 2048, 768, False, True),
    (2, 37, 64, 1024, 512, True, True),
    (3, 9, 32, 512, 384, False, True),
    (2, 3, 16, 96, 64, False, True),     # generic (untiled) expert rows
    # one token: the gate/up blocks rank the logits (E <= 256: 4, 2, 1 key
    # parts; E a power of two or not); E > 256 keeps the selection kernel
    (3, 1, 60, 512, 256, False, True),
    (2, 1, 200, 512, 256, True, True),
    (3, 1, 256, 512, 256, False, True),
    (3, 1, 300, 512, 256, True, True),
    # two tokens: each gate/up block ranks its own token's logits and
    # reduces that token's x-table partials ([token][router row] layout)
    (2, 2, 128, 2048, 768, True, True),
    (3, 2, 60, 512, 256, False, True),
    # few tokens, 8 experts: every token takes all 8, so each expert's
    # gate/up stream serves every token (up to 31 slots)
    (3, 20, 8, 512, 256, False, True),
    (2, 31, 8, 256, 128, True, True),
]


@pytest.mark.parametrize("dtype,T,E,D,dff,bias,resid", CASES)
def test_layer_vs_oracle(moehip, dtype, T, E, D, dff, bias, resid):
    seed = 7000 + dtype * 100 + T
    print("case", dtype, T, E, D, dff, bias, resid, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    rb = O.normal(E, seed + 11, 0.0, 0.05) if bias else None
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    xr = O.normal(T * D, seed + 13, 0.0, 1.0).reshape(T, D) if resid else None
    want, widx, wp, wlog = O.moe_block(xn, xr, rw, rb, ex)
    layer = make_layer(moehip, dtype, ex, rw, rb)
    got, idx, p = layer.forward(xn, xr)
    dbg = layer.debug(T)
    np.testing.assert_array_equal(bits(dbg["logits"]), bits(wlog))
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("T", [3, 2, 1])
def test_router_ties_and_nan(moehip, T):
    """Equal logits keep the lower expert first; NaN logits are never chosen."""
    dtype, E, D, dff = 2, 32, 256, 128
    ex = random_experts(dtype, E, D, dff, 99)
    rw = O.normal(E * D, 98, 0.0, 0.02).reshape(E, D)
    rw[5] = rw[17]          # experts 5 and 17 tie exactly
    rw[9] = rw[17]
    rw[3, 0] = np.nan       # expert 3's logit is NaN for every token
    xn = O.normal(T * D, 97, 0.0, 1.0).reshape(T, D)
    xn[:, :] += rw[17] * 50  # push the tied experts to the top
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex)
    layer = make_layer(moehip, dtype, ex, rw)
    got, idx, p = layer.forward(xn, xn)
    assert 3 not in idx
    np.testing.assert_array_equal(idx, widx)
    assert list(idx[0][:3]) == [5, 9, 17]
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("T", [1, 2, 3, 16])
def test_decode_dead_slots(moehip, T):
    """Per-pair kernels with router rows 6-15 NaN (16 experts): every
    token's slots 6 and 7 hold -1, so their gate/up blocks (which select
    for themselves up to two tokens) and their down terms drop out."""
    dtype, E, D, dff = 3, 16, 512, 256
    seed = 9600 + T
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    rw[6:, 3] = np.nan
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex)
    assert (widx[:, 6:] == -1).all() and (widx[:, :6] >= 0).all()
    layer = make_layer(moehip, dtype, ex, rw)
    got, idx, p = layer.forward(xn, xn)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dtype", [3, 2])
@pytest.mark.parametrize("case", ["plain", "big_rows", "dead_slots", "top4"])
def test_fused_one_token_gate_up_down(moehip, dtype, case):
    """One token at E = 128, D = 2048, d_ff = 768.  Q4: gate/up and down
    share one launch -- the down blocks select for themselves and take h's
    tables, limb counts and sums from the gate/up blocks' tagged words; Q8
    (two launches at this shape) as the per-pair reference point.  big_rows:
    gate/up row scales of d_ff rows 0-63 x 1000, so h needs two limbs there
    (Q4: the down blocks' exact fallback on the tagged fp32 h; Q8: two
    planes, or four where |h| passes 257); dead_slots: router rows 5-127
    NaN, so ranks 5-7 hold -1 (their down terms drop out, waves 1-3's
    second rank is dead); top4: top-k 4 (every wave's second rank is past
    k).  Each case runs twice, the first call on 1000x larger activations,
    so that a word left by an earlier launch would show."""
    E, D, dff = 128, 2048, 768
    seed = {"plain": 9700, "big_rows": 9710, "dead_slots": 9720, "top4": 9730}[case] + dtype
    top_k = 4 if case == "top4" else 8
    print("fused one-token case", dtype, case, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    if case == "big_rows":
        ex.gs[:, :64] *= 1000.0
        ex.us[:, :64] *= 1000.0
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    if case == "dead_slots":
        rw[5:, 7] = np.nan
    xn = O.normal(D, seed + 12, 0.0, 1.0).reshape(1, D)
    big = np.ascontiguousarray(xn * np.float32(1000.0))
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex, top_k=top_k)
    want_big, widx_big, _, _ = O.moe_block(big, xn, rw, None, ex, top_k=top_k)
    if case == "dead_slots":
        assert (widx[:, 5:] == -1).all() and (widx[:, :5] >= 0).all()
    layer = make_layer(moehip, dtype, ex, rw, top_k=top_k)
    got_big, idx_big, _ = layer.forward(big, xn)
    np.testing.assert_array_equal(idx_big, widx_big)
    np.testing.assert_array_equal(bits(got_big), bits(want_big))
    got, idx, p = layer.forward(xn, xn)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


def test_fused_one_token_deadline(moehip, monkeypatch):
    """The fused launch's bounded waits, forced from the host: with a wait
    limit of 0 a down block that does not find its words at the first look
    gives up and writes NaN for its rows.  Every output row is then either
    the oracle's bits or NaN -- never a wrong number -- and the launch
    completes; with the limit back every row is exact again."""
    dtype, E, D, dff = 3, 128, 2048, 768
    seed = 9770
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    layer = make_layer(moehip, dtype, ex, rw)
    xn = O.normal(D, seed + 12, 0.0, 1.0).reshape(1, D)
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex)
    monkeypatch.setenv("MOEHIP_FUSE_WAIT_US", "0")
    nan_rows = 0
    for _ in range(4):
        got, idx, p = layer.forward(xn, xn)
        np.testing.assert_array_equal(idx, widx)
        bad = ~np.isnan(got[0])
        np.testing.assert_array_equal(bits(got[0][bad]), bits(want[0][bad]))
        nan_rows += int(np.isnan(got[0]).sum())
    print("outputs given up at the deadline:", nan_rows, "of", 4 * D, flush=True)
    monkeypatch.delenv("MOEHIP_FUSE_WAIT_US")
    got, idx, p = layer.forward(xn, xn)
    np.testing.assert_array_equal(bits(got), bits(want))


def test_fused_one_token_between_other_paths(moehip):
    """The fused one-token launch between calls on the other paths (T = 1,
    3, 1, 40, 1, 2, 1 at the Q4 fused shape: per-pair kernels at 2-3 tokens,
    expert-major at 40): its tags come from an epoch only its own router
    launches advance, so the words the earlier fused calls left are never
    current in a later one; each call against the oracle."""
    dtype, E, D, dff = 3, 128, 2048, 768
    seed = 9750
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    layer = make_layer(moehip, dtype, ex, rw)
    for i, T in enumerate((1, 3, 1, 40, 1, 2, 1)):
        print("fused-shape sequence call", i, "T", T, flush=True)
        xn = O.normal(T * D, seed + 20 + i, 0.0, 1.0).reshape(T, D)
        xr = O.normal(T * D, seed + 40 + i, 0.0, 1.0).reshape(T, D)
        want, widx, wp, _ = O.moe_block(xn, xr, rw, None, ex)
        got, idx, p = layer.forward(xn, xr)
        np.testing.assert_array_equal(idx, widx)
        np.testing.assert_array_equal(bits(p), bits(wp))
        np.testing.assert_array_equal(bits(got), bits(want))


def test_router_block_sum_special_rows(moehip):
    """The one-token router's product sums at D = 2048 (block-parallel
    candidate segments) against the oracle's loop, bit for bit, on rows
    built to stress them: partial sums that cross zero often (alternating
    +-c pairs with a small drift, where segment estimates miss and the
    sequential fallback runs), exact cancellation to zero, 1e30 / 1e-30
    terms side by side, an overflow to inf and then NaN, a NaN term,
    all-zero and all-equal rows, and plain random rows."""
    dtype, E, D, dff = 3, 16, 2048, 256
    seed = 9800
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    k = np.arange(D)
    rw[0] = np.where(k % 2 == 0, 1.0, -1.0) * (1.0 + 1e-3 * (k % 7))
    rw[1, : D // 2] = 0.5
    rw[1, D // 2:] = -0.5
    rw[2] = np.where(k % 3 == 0, 1e30, np.where(k % 3 == 1, 1e-30, -1e30))
    rw[3, :] = 3e38
    rw[3, D // 2:] = -3e38
    rw[4, 1000] = np.nan
    rw[5] = 0.0
    rw[6] = 0.25
    rw[7] = np.sin(k * 0.37) * np.exp(-k / 700.0)
    xn = np.abs(O.normal(D, seed + 12, 0.0, 1.0)).reshape(1, D) + np.float32(0.5)
    want, widx, wp, wlog = O.moe_block(xn, xn, rw.astype(np.float32), None, ex)
    layer = make_layer(moehip, dtype, ex, rw.astype(np.float32))
    got, idx, p = layer.forward(xn, xn)
    dbg = layer.debug(1)
    np.testing.assert_array_equal(bits(dbg["logits"]), bits(wlog))
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


def test_rmsnorm_dev(moehip):
    for T, D in ((3, 2048), (2, 100)):
        x = O.normal(T * D, 5 + D, 0.0, 2.0).reshape(T, D)
        w = O.normal(D, 6 + D, 1.0, 0.1)
        dx, dw, dy = (moehip.DeviceBuffer.from_array(x), moehip.DeviceBuffer.from_array(w),
                      moehip.DeviceBuffer(x.nbytes))
        moehip.check(moehip.lib().moe_rmsnorm_dev(dx.ptr, dw.ptr, dy.ptr, T, D, 1e-6))
        np.testing.assert_array_equal(bits(dy.download((T, D), np.float32)), bits(O.rmsnorm(x, w)))


def _seq_sum_rows():
    """Rows whose sequential sum of squares defeats the segment estimates of
    block_seq_sum in different ways (every path of its stitching runs)."""
    rng = np.random.default_rng(77)
    D = 2048
    rows = [rng.normal(0, 1, D),                                  # the common case
            rng.normal(0, 1, D) * 10.0 ** rng.integers(-18, 18, D),   # huge dynamic range
            np.where(np.arange(D) % 97 == 0, 3e18, 1e-3),          # a few huge squares: far estimates
            rng.normal(0, 1, D), rng.normal(0, 1, D), rng.normal(0, 1e19, D)]   # overflow to inf
    rows[3][1000] = np.nan
    rows[4][5] = np.inf
    return np.array(rows, np.float32)


def test_rmsnorm_parallel_sum_paths(moehip):
    """The block-parallel sequential sum of squares (candidate segments with a
    sequential fallback) against the oracle's loop, bit for bit, through both
    users: the RMSNorm kernel and the norm fused into the router product."""
    x = _seq_sum_rows()
    T, D = x.shape
    for w in (None, O.normal(D, 78, 1.0, 0.1)):
        dx, dy = moehip.DeviceBuffer.from_array(x), moehip.DeviceBuffer(x.nbytes)
        dw = moehip.DeviceBuffer.from_array(w) if w is not None else None
        moehip.check(moehip.lib().moe_rmsnorm_dev(dx.ptr, dw.ptr if dw else None, dy.ptr, T, D, 1e-6))
        np.testing.assert_array_equal(bits(dy.download((T, D), np.float32)), bits(O.rmsnorm(x, w)))
    # fused into the router (one token and four tokens at a time)
    dtype, E, dff = 3, 16, 256
    ex = random_experts(dtype, E, D, dff, 79)
    rw = O.normal(E * D, 80, 0.0, 0.02).reshape(E, D)
    rms2 = O.normal(D, 81, 1.0, 0.1)
    layer = make_layer(moehip, dtype, ex, rw, None, rms2)
    finite = x[np.isfinite(x).all(axis=1)][:3]
    for rows in (finite[:1], finite[:3]):
        want = O.moe_block(O.rmsnorm(rows, rms2), rows, rw, None, ex)[0]
        np.testing.assert_array_equal(bits(layer.block_forward(rows)), bits(want))


@pytest.mark.parametrize("dtype,E,bias", [(3, 60, False), (2, 200, True), (3, 300, False)])
def test_block_forward_one_token(moehip, dtype, E, bias):
    """One token through rmsnorm fused into the router: the x tables' headers
    come from the router blocks' partials, reduced where the experts are
    selected (inside the gate/up blocks for E <= 256, a kernel of its own
    above)."""
    D, dff = 512, 256
    seed = 4100 + E
    print("case", dtype, E, bias, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 1, 0.0, 0.02).reshape(E, D)
    rb = O.normal(E, seed + 2, 0.0, 0.05) if bias else None
    x = O.normal(D, seed + 4, 0.0, 1.0).reshape(1, D)
    for wscale in (1.0, 40.0):   # one- and two-limb activations
        rms2 = (O.normal(D, seed + 3, 1.0, 0.1) * wscale).astype(np.float32)
        layer = make_layer(moehip, dtype, ex, rw, rb, rms2)
        want = O.moe_block(O.rmsnorm(x, rms2), x, rw, rb, ex)[0]
        np.testing.assert_array_equal(bits(layer.block_forward(x)), bits(want))


def test_repeated_forward_and_growing_T(moehip):
    """Scratch reuse: T grows and shrinks between calls; results stay exact."""
    dtype, E, D, dff = 3, 64, 1024, 512
    ex = random_experts(dtype, E, D, dff, 55)
    rw = O.normal(E * D, 56, 0.0, 0.02).reshape(E, D)
    layer = make_layer(moehip, dtype, ex, rw)
    for T in (2, 11, 1, 11):
        xn = O.normal(T * D, 60 + T, 0.0, 1.0).reshape(T, D)
        want, widx, _, _ = O.moe_block(xn, xn, rw, None, ex)
        got, idx, _ = layer.forward(xn, xn)
        np.testing.assert_array_equal(idx, widx)
        np.testing.assert_array_equal(bits(got), bits(want))


GROUPED = [  # dtype, T, E, D, d_ff, bias, resid, x scale
    (2, 1, 128, 2048, 768, False, True, 1.0),
    (3, 3, 128, 2048, 768, True, True, 1.0),
    (2, 40, 128, 2048, 768, False, True, 1.0),
    (3, 96, 128, 2048, 768, False, False, 1.0),
    (2, 21, 32, 1024, 512, True, True, 1.0),
    (3, 130, 16, 512, 256, False, True, 1.0),    # > 64 pairs per expert: several passes
    (3, 17, 64, 1024, 512, False, True, 40.0),   # 2-limb Q4 activations
    (2, 9, 64, 1024, 256, True, True, 400.0),    # 4-limb Q8 activations (and h)
    (3, 70, 8, 512, 256, False, True, 3000.0),   # 4-limb Q4, > 32 pairs per expert
    # E = top-k: every expert takes every token, > 256 pairs each, so each
    # expert's pairs split into several tasks (blocks)
    (3, 300, 8, 512, 256, False, True, 1.0),
    (3, 520, 8, 256, 256, False, True, 40.0),    # split, 2-limb Q4
    (2, 280, 8, 512, 256, True, True, 0.3),      # split, one-limb Q8
    (3, 2048, 8, 256, 256, False, True, 1.0),    # 2048 tokens, router blocks cut to E = 8 experts
    # the config shape's D = 2048 and d_ff = 768 (16 and 6 stages of the LDS
    # ring), 16 experts so that 128 pairs per expert on average select the
    # four-tile, eight-wave blocks (the prefill bench's T = 2048 shape)
    (3, 256, 16, 2048, 768, False, True, 1.0),
    # Q8 at D = 2048, d_ff = 768: x ~ N(0, 1) needs two limbs, so every task
    # runs limb passes folded into one dot (two-tile blocks)
    (2, 128, 16, 2048, 768, True, True, 1.0),
    # D = 384: three down row tiles of 128 in one block (two-tile shape), a
    # partial last tile of 256 rows (four-tile shape, one tile per block)
    (3, 96, 16, 384, 256, False, True, 1.0),
    (3, 256, 16, 384, 256, False, True, 1.0),
    # x tables packed by 16 router blocks per token group, 24 units a token
    # (uneven shares), two-limb activations, a partial last token group
    (3, 50, 128, 384, 256, False, True, 40.0),
]


@pytest.mark.parametrize("dtype,T,E,D,dff,bias,resid,scale", GROUPED)
def test_grouped_vs_oracle(moehip, dtype, T, E, D, dff, bias, resid, scale):
    """The expert-major kernels (forced at every T) against the oracle."""
    seed = 8100 + dtype * 100 + T
    print("grouped case", dtype, T, E, D, dff, bias, resid, scale, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    rb = O.normal(E, seed + 11, 0.0, 0.05) if bias else None
    xn = O.normal(T * D, seed + 12, 0.0, scale).reshape(T, D)
    xr = O.normal(T * D, seed + 13, 0.0, 1.0).reshape(T, D) if resid else None
    want, widx, wp, wlog = O.moe_block(xn, xr, rw, rb, ex)
    layer = make_layer(moehip, dtype, ex, rw, rb)
    layer.set_grouped_min_tokens(1)
    got, idx, p = layer.forward(xn, xr)
    dbg = layer.debug(T)
    np.testing.assert_array_equal(bits(dbg["logits"]), bits(wlog))
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dtype,T", [(3, 24), (3, 96), (3, 256), (2, 24), (2, 96), (2, 256)])
def test_grouped_mixed_limb_segments(moehip, dtype, T):
    """h rows 0-63 of every expert scaled up (gate and up row scales x 1000):
    those h values need 2 (Q4) or 4 (Q8) limbs, the other rows one, so the
    gate/up blocks write different limb planes per row segment and down's
    limb passes read zeros for the segments that wrote fewer.  A first call
    on 1000x larger activations (h of every row needs 2 or 4 limbs) leaves
    the upper h planes nonzero, so that a plane read where it was not
    written this call shows.  16 experts: T = 24 / 96
    / 256 select the 1-, 2- and 4-tile block shapes."""
    E, D, dff = 16, 512, 768
    seed = 8800 + dtype * 10 + T
    print("mixed-limb case", dtype, T, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    ex.gs[:, :64] *= 1000.0
    ex.us[:, :64] *= 1000.0
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex)
    layer = make_layer(moehip, dtype, ex, rw)
    layer.set_grouped_min_tokens(1)
    big = np.ascontiguousarray(xn * np.float32(1000.0))
    want_big, _, _, _ = O.moe_block(big, xn, rw, None, ex)
    got_big, _, _ = layer.forward(big, xn)
    np.testing.assert_array_equal(bits(got_big), bits(want_big))
    got, idx, p = layer.forward(xn, xn)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dtype,top_k,T,grouped", [(3, 4, 64, True), (2, 6, 48, True), (3, 2, 40, True),
                                                    (3, 4, 5, False), (2, 6, 3, False), (2, 2, 1, False)])
def test_layer_other_top_k(moehip, dtype, top_k, T, grouped):
    """A top-k other than 8 (model.h keeps it a config value): the
    selection, the gates and the combine over k ranks (the expert-major
    path's runtime-k combine kernels, fp32 y for Q8 and int16 dots for Q4;
    the per-pair kernels below 32 tokens), bit for bit against the oracle."""
    E, D, dff = 32, 512, 256
    seed = 9100 + dtype * 10 + top_k + T
    print("top-k case", dtype, top_k, T, grouped, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    ex.gs[:] *= np.float32(60.0)
    ex.us[:] *= np.float32(60.0)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    xr = O.normal(T * D, seed + 13, 0.0, 1.0).reshape(T, D)
    want, widx, wp, wlog = O.moe_block(xn, xr, rw, None, ex, top_k)
    layer = make_layer(moehip, dtype, ex, rw, top_k=top_k)
    layer.set_grouped_min_tokens(1 if grouped else 1000)
    got, idx, p = layer.forward(xn, xr)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))
    layer.close()


def _q4_down_dots(ex, xn, widx):
    """The Q4 down products' int32 dots of every live (token, rank) pair,
    from the oracle's expert GEMVs (kernels.c:96-128) and SwiGLU."""
    D, dff = ex.D, ex.d_ff
    out = []
    for t in range(xn.shape[0]):
        for e in widx[t]:
            if e < 0:
                continue
            g = O.gemv_q4(xn[t:t + 1], ex.gq[e], ex.gs[e], dff, D)
            u = O.gemv_q4(xn[t:t + 1], ex.uq[e], ex.us[e], dff, D)
            h = (O.silu(g) * u).astype(np.float32).reshape(-1)
            a = np.trunc((h * np.float32(7.0)).astype(np.float64)).astype(np.int64)
            w = ex.dq[e].astype(np.int64)
            wu = np.empty((D, dff), np.int64)
            wu[:, 0::2] = (w & 0xF) - 8
            wu[:, 1::2] = (w >> 4) - 8
            out.append(wu @ a)
    return np.concatenate(out)


@pytest.mark.parametrize("factor", [40.0, 300.0, 3000.0])
def test_grouped_q4_int16_down_dots(moehip, factor):
    """The expert-major Q4 down kernel hands the combine each output's int32
    dot as int16 when it lies in [-32767, 32767], else a marker and the fp32
    value: gate/up row scales x factor put the down dots inside int16
    (1), across its edge within one pair (300) and mostly past it (3000);
    the host counts the dots of each case from the oracle's own GEMVs so
    that both paths are known to run, and the layer stays bit-identical."""
    dtype, E, D, dff, T = 3, 16, 512, 768, 48
    seed = 8900 + int(factor)
    print("int16 dots case", factor, flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    ex.gs[:] *= np.float32(factor)
    ex.us[:] *= np.float32(factor)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    xr = O.normal(T * D, seed + 13, 0.0, 1.0).reshape(T, D)
    want, widx, wp, _ = O.moe_block(xn, xr, rw, None, ex)
    big = np.abs(_q4_down_dots(ex, xn, widx)) > 32767
    if factor == 40.0:
        assert not big.any() and np.abs(_q4_down_dots(ex, xn, widx)).max() > 1000
    elif factor == 300.0:
        assert 0.05 < big.mean() < 0.95, big.mean()
    else:
        assert big.mean() > 0.95, big.mean()
    layer = make_layer(moehip, dtype, ex, rw)
    layer.set_grouped_min_tokens(1)
    got, idx, p = layer.forward(xn, xr)
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))
    layer.close()


def test_grouped_config_shape_T2048(moehip):
    """The prefill bench's layer shape (configs[3]: Q4, E = 128, D = 2048,
    d_ff = 768, top-8) at T = 2048: eight-wave router blocks, x tables
    packed by the router blocks, one 256-pair task per expert, the many-pair
    grouping, two down row tiles per block -- bit for bit against the
    oracle (its threaded build: 77 G multiply-adds)."""
    dtype, T, E, D, dff = 3, 2048, 128, 2048, 768
    seed = 9900
    print("config-shape case T=2048", flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    xr = O.normal(T * D, seed + 13, 0.0, 1.0).reshape(T, D)
    with O.threaded():
        want, widx, wp, wlog = O.moe_block(xn, xr, rw, None, ex)
    layer = make_layer(moehip, dtype, ex, rw)
    got, idx, p = layer.forward(xn, xr)
    dbg = layer.debug(T)
    np.testing.assert_array_equal(bits(dbg["logits"]), bits(wlog))
    np.testing.assert_array_equal(idx, widx)
    np.testing.assert_array_equal(bits(p), bits(wp))
    np.testing.assert_array_equal(bits(got), bits(want))


def test_grouped_many_pairs_dead_slots(moehip):
    """More pairs than one grouping block takes (700 tokens x top-8 = 5600
    pairs: 22 blocks of 255, the last 245) with router rows 6-15 NaN, so
    that only 6 experts are live and every token's slots 6 and 7 hold -1:
    the selection's per-block counts skip dead slots and the scatter gets
    exactly the live pairs."""
    dtype, T, E, D, dff = 3, 700, 16, 256, 256
    seed = 9700
    print("many-pairs dead-slots case", flush=True)
    ex = random_experts(dtype, E, D, dff, seed)
    rw = O.normal(E * D, seed + 10, 0.0, 0.02).reshape(E, D)
    rw[6:, 1] = np.nan
    xn = O.normal(T * D, seed + 12, 0.0, 1.0).reshape(T, D)
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex)
    assert (widx[:, 6:] == -1).all() and (widx[:, :6] >= 0).all()
    layer = make_layer(moehip, dtype, ex, rw)
    layer.set_grouped_min_tokens(1)
    for _ in range(2):
        got, idx, p = layer.forward(xn, xn)
        np.testing.assert_array_equal(idx, widx)
        np.testing.assert_array_equal(bits(p), bits(wp))
        np.testing.assert_array_equal(bits(got), bits(want))


def test_grouped_and_decode_agree_ties_nan(moehip):
    """Both paths on the same layer and tokens: tied and NaN router logits."""
    dtype, T, E, D, dff = 2, 12, 32, 256, 128
    ex = random_experts(dtype, E, D, dff, 77)
    rw = O.normal(E * D, 78, 0.0, 0.02).reshape(E, D)
    rw[5] = rw[17]
    rw[3, 0] = np.nan
    xn = O.normal(T * D, 79, 0.0, 1.0).reshape(T, D)
    xn[:, :] += rw[17] * 50
    want, widx, wp, _ = O.moe_block(xn, xn, rw, None, ex)
    layer = make_layer(moehip, dtype, ex, rw)
    outs = []
    for mt in (1, 1000):
        layer.set_grouped_min_tokens(mt)
        got, idx, p = layer.forward(xn, xn)
        np.testing.assert_array_equal(idx, widx)
        np.testing.assert_array_equal(bits(p), bits(wp))
        np.testing.assert_array_equal(bits(got), bits(want))
        outs.append(got)
    assert 3 not in widx
