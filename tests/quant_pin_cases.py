"""Rows that pin the exporter's rowwise quantizer (export.py:23-36) by
exact arithmetic, shared by the CPU test of the oracle and the GPU test of
moe_quantize_rows_dev.

export.py computes, in torch fp32:
    s = amax.clamp(1e-8) / 127      (Q4: / 7)
    q = round(w / s)                (torch.round: half to even; Q4 then
                                     clamped to [-8, 7] and offset by +8)
IEEE fp32 division is correctly rounded, so the exporter's answer is
    s = RN32(amax / 127),  q = rhe(RN32(w / s))
with RN32 the round-to-nearest-even of the exact rational value and rhe the
half-to-even integer rounding.  `expected` evaluates exactly that with
Python Fractions, with no floating-point step of its own.

`find_rows` searches the fp32 neighbours of the rounding boundaries
(k + 1/2) * s for weights on which plausible mistakes give another integer:
  recip   q = rhe(RN32(w * RN32(1 / s)))      (reciprocal multiply)
  double  s, w / s in float64, then rint       (scale kept in double)
  exact   q = rhe(w / s) without rounding the quotient to fp32
  away    half away from zero instead of half to even
Every mistake is represented by at least one weight of the returned rows,
so an oracle or kernel that makes any of them fails the comparison.
"""
from __future__ import annotations

import functools
import math
from fractions import Fraction

import numpy as np

_F32_MIN_EXP = -126
_F32_MANT = 23


def rn32(x: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp32 value (ties to even)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # correct the floating log estimate
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, _F32_MIN_EXP)
    quantum = Fraction(2) ** (e - _F32_MANT)
    m = a / quantum
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * quantum
    if v >= Fraction(2) ** 128:
        raise OverflowError("fp32 overflow")
    return sign * v


def rhe(x: Fraction) -> int:
    """Round half to even (Python's round on a Fraction is exactly this)."""
    return round(x)


def away(x: Fraction) -> int:
    f = math.floor(abs(x) + Fraction(1, 2))
    return f if x >= 0 else -f


def f32(x) -> Fraction:
    return Fraction(float(np.float32(x)))


def scale_of(amax: np.float32, div: int) -> Fraction:
    return rn32(f32(max(amax, np.float32(1e-8))) / div)


def expected(w: np.float32, s: Fraction, lo: int, hi: int) -> int:
    return min(hi, max(lo, rhe(rn32(f32(w) / s))))


def mistakes(w: np.float32, amax: np.float32, div: int, lo: int, hi: int) -> dict:
    s = scale_of(amax, div)
    fw = f32(w)
    clamp = lambda q: min(hi, max(lo, q))  # noqa: E731
    r = rn32(1 / s)
    sd = float(np.float32(amax)) / div           # the scale in double
    qd = float(np.float32(w)) / sd
    return {"recip": clamp(rhe(rn32(fw * r))),
            "double": clamp(int(np.rint(qd))),
            "exact": clamp(rhe(fw / s)),
            "away": clamp(away(rn32(fw / s)))}


def _screen(amax: np.float32, div: int, lo: int, hi: int, n_nb: int):
    """Fast numpy screen of the neighbours of every boundary (k + 1/2) s:
    the weights on which some mistake's integer differs from the exporter's
    (each is confirmed afterwards with exact arithmetic)."""
    s32 = np.float32(float(scale_of(amax, div)))
    ks = np.arange(lo, hi, dtype=np.float64)
    w = ((ks + 0.5) * float(s32)).astype(np.float32)
    cand = [w]
    up, dn = w, w
    for _ in range(n_nb):
        up = np.nextafter(up, np.float32(np.inf))
        dn = np.nextafter(dn, np.float32(-np.inf))
        cand += [up, dn]
    w = np.concatenate(cand)
    w = w[np.abs(w) < amax]
    with np.errstate(all="ignore"):
        true = np.clip(np.rint(w / s32), lo, hi)
        recip = np.clip(np.rint(w * (np.float32(1) / s32)), lo, hi)
        dbl = np.clip(np.rint(w.astype(np.float64) / (float(amax) / div)), lo, hi)
        q32 = (w / s32).astype(np.float64)
        awayq = np.clip(np.sign(q32) * np.floor(np.abs(q32) + 0.5), lo, hi)
    differs = (recip != true) | (dbl != true) | (awayq != true)
    # unrounded quotient: only where the fp32 quotient is exactly a half
    halves = (q32 - np.floor(q32)) == 0.5
    return w[differs | halves]


@functools.lru_cache(maxsize=None)
def find_rows(div: int, K: int = 64, n_rows: int = 6, seed: int = 5):
    """-> (W [n_rows x K] fp32, counts of weights per mistake kind).
    Row r has amax at column 0 (a positive or negative weight), the
    discriminating weights found for that amax (each confirmed with exact
    arithmetic), and N(0, (amax/4)^2) filler clipped to |w| < amax."""
    lo, hi = (-127, 127) if div == 127 else (-8, 7)
    rng = np.random.default_rng(seed + div)
    rows = []
    counts = {"recip": 0, "double": 0, "exact": 0, "away": 0}
    tries = 0
    while len(rows) < n_rows:
        tries += 1
        assert tries < 200, "no discriminating weights found"
        amax = np.float32(rng.uniform(0.01, 0.09))
        s = scale_of(amax, div)
        found = []
        kinds_row = set()
        for w in _screen(amax, div, lo, hi, 24):
            want = expected(w, s, lo, hi)
            bad = [n for n, q in mistakes(w, amax, div, lo, hi).items() if q != want]
            if not bad:
                continue
            if any(n not in kinds_row for n in bad) or len(found) < K // 2:
                found.append(w)
                kinds_row.update(bad)
                for n in bad:
                    counts[n] += 1
            if len(found) >= K - 1:
                break
        if not found:
            continue
        row = np.clip(rng.normal(0.0, float(amax) / 4, K), -0.99 * float(amax),
                      0.99 * float(amax)).astype(np.float32)
        row[0] = amax if len(rows) % 2 == 0 else -amax
        row[1:1 + len(found)] = np.array(found[:K - 1], np.float32)
        rows.append(row)
    assert all(v > 0 for v in counts.values()), counts
    return np.stack(rows), counts


def expected_rows(W: np.ndarray, div: int):
    """Exact exporter answer for each row: (q int [N x K], s fp32 [N])."""
    lo, hi = (-127, 127) if div == 127 else (-8, 7)
    N, K = W.shape
    q = np.empty((N, K), np.int64)
    s_out = np.empty(N, np.float32)
    for n in range(N):
        amax = np.float32(np.max(np.abs(W[n])))
        s = scale_of(amax, div)
        s_out[n] = np.float32(float(s))
        for k in range(K):
            q[n, k] = expected(W[n, k], s, lo, hi)
    return q, s_out


def pack_q4(q: np.ndarray) -> np.ndarray:
    """export.py:32-35: +8, low nibble = even column, high = odd column."""
    u = (q + 8).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)
