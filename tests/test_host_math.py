"""Host-side checks of arithmetic shortcuts the HIP kernels take, against the oracle's restatement of the
reference rule they replace."""

import numpy as np

from oracle import bxref as R


def _div_round_short(a, p, r):
    """The kernels' short form of ops.div_round (csrc/bx_rows.hip div_round64) for 0 <= p <= 62, r < 2^34 and
    |a 2^p / r| < 2^51: float64 estimate (same operation order), wrapping remainder, one correction each way,
    round half up. Returns (value, taken)."""
    qd = a.astype(np.float64) * np.ldexp(1.0, p) * (1.0 / r.astype(np.float64))
    taken = (p >= 0) & (p <= 62) & (r < (1 << 34)) & (np.abs(qd) < 2.0 ** 51)
    q = np.floor(np.where(taken, qd, 0.0)).astype(np.int64)
    with np.errstate(over="ignore"):
        rem = (a.astype(np.uint64) << p.astype(np.uint64)).astype(np.int64) - q * r
    lo = rem < 0
    q, rem = np.where(lo, q - 1, q), np.where(lo, rem + r, rem)
    hi = rem >= r
    q, rem = np.where(hi, q + 1, q), np.where(hi, rem - r, rem)
    return q + (2 * rem >= r), taken


def test_div_round_short_form_matches_long_division():
    g = np.random.default_rng(0)
    n = 400_000
    ab = g.integers(0, 63, n)
    a = (g.integers(0, 1 << 62, n, dtype=np.int64) >> (62 - ab)) * g.choice([-1, 1], n)
    rb = g.integers(1, 35, n)
    r = np.maximum(g.integers(0, 1 << 62, n, dtype=np.int64) >> (62 - rb), 1)
    p = g.integers(0, 63, n)
    a[:4] = [np.iinfo(np.int64).max, np.iinfo(np.int64).min + 1, 0, -1]
    got, taken = _div_round_short(a, p, r)
    assert taken.sum() > n // 4
    ref = R.div_round(a[taken], p[taken], r[taken])
    assert np.array_equal(got[taken], ref)


