"""The oracle's restatement of the exporter's rowwise quantizer
(export.py:23-36, orc_quant_q8_rows / orc_quant_q4_rows) pinned by exact
arithmetic.

export.py runs in torch fp32: s = amax.clamp(1e-8) / 127 (or / 7) and
q = torch.round(w / s).  IEEE-754 fixes both steps: a correctly rounded
fp32 division, then half-to-even integer rounding (torch.round's documented
rule).  quant_pin_cases.expected evaluates that with Python Fractions.  The
rows are chosen (quant_pin_cases.find_rows) so that each plausible mistake
-- a reciprocal multiply, a scale kept in double, a quotient not rounded to
fp32, half-away-from-zero rounding -- gives another integer on at least one
of their weights; the oracle must match the exact answer on all of them.
tests/test_gpu_quant.py holds the device quantizer to the same rows.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O
import quant_pin_cases as Q


def test_rn32_against_ieee_hardware():
    """The exact helper agrees with the host's IEEE fp32 division and
    multiplication (correct rounding) on random operands, and rounds ties
    to even."""
    rng = np.random.default_rng(3)
    a = rng.normal(0, 1, 3000).astype(np.float32)
    b = rng.uniform(1e-4, 3, 3000).astype(np.float32)
    for x, y in zip(a, b):
        assert Q.rn32(Fraction(float(x)) / Fraction(float(y))) == Fraction(float(x / y))
        assert Q.rn32(Fraction(float(x)) * Fraction(float(y))) == Fraction(float(x * y))
    one = Fraction(1)
    ulp = Fraction(1, 2 ** 23)
    assert Q.rn32(one + ulp / 2) == one               # tie to even (down)
    assert Q.rn32(one + 3 * ulp / 2) == one + 2 * ulp  # tie to even (up)
    assert Q.rn32(Fraction(1, 3)) == Fraction(float(np.float32(1) / np.float32(3)))
    assert Q.rn32(Fraction(1, 2 ** 149)) == Fraction(1, 2 ** 149)   # smallest subnormal


@pytest.mark.parametrize("div", [127, 7])
def test_rows_discriminate_every_mistake(div):
    W, counts = Q.find_rows(div)
    assert all(c > 0 for c in counts.values()), counts
    # and each mistake changes at least one quantized value of the rows
    lo, hi = (-127, 127) if div == 127 else (-8, 7)
    for kind in counts:
        hit = False
        for row in W:
            amax = np.float32(np.max(np.abs(row)))
            s = Q.scale_of(amax, div)
            for w in row:
                if Q.mistakes(w, amax, div, lo, hi)[kind] != Q.expected(w, s, lo, hi):
                    hit = True
                    break
            if hit:
                break
        assert hit, kind


def test_oracle_q8_matches_exact_exporter():
    W, _ = Q.find_rows(127)
    q_want, s_want = Q.expected_rows(W, 127)
    q, s = O.quant_q8(W)
    np.testing.assert_array_equal(s.view(np.uint32), s_want.view(np.uint32))
    np.testing.assert_array_equal(q.astype(np.int64), q_want)


def test_oracle_q4_matches_exact_exporter():
    W, _ = Q.find_rows(7)
    q_want, s_want = Q.expected_rows(W, 7)
    q, s = O.quant_q4(W)
    np.testing.assert_array_equal(s.view(np.uint32), s_want.view(np.uint32))
    np.testing.assert_array_equal(q, Q.pack_q4(q_want))


@pytest.mark.parametrize("div", [127, 7])
def test_oracle_scale_clamp_and_extremes(div):
    """amax below 1e-8 clamps to the fp32 value 1e-8; tiny and subnormal
    weights; the row maximum itself maps to +-127 (+-7)."""
    W = np.zeros((3, 8), np.float32)
    W[1, :] = [3e-9, -1e-9, 1e-45, 0.0, -3e-9, 2e-9, 5e-10, -7e-9]
    W[2, :] = [0.05, -0.05, 0.025, -0.0125, 1e-30, -1e-30, 0.049999, 0.0]
    q_want, s_want = Q.expected_rows(W, div)
    if div == 127:
        q, s = O.quant_q8(W)
        np.testing.assert_array_equal(q.astype(np.int64), q_want)
    else:
        q, s = O.quant_q4(W)
        np.testing.assert_array_equal(q, Q.pack_q4(q_want))
    np.testing.assert_array_equal(s.view(np.uint32), s_want.view(np.uint32))
    assert s_want[0] == np.float32(float(Q.rn32(Fraction(float(np.float32(1e-8))) / div)))
