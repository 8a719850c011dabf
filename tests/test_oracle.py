"""Pins the CPU oracle (oracle/bxref.py) against closed forms, the reference's own fixtures and brute force.

Mirrors the reference's CPU tests (tests/test_exact_ops.py, tests/test_intops.py, tests/test_int8_ops.py,
tests/test_model_bounds.py) and its self-check hash (docs/REPRODUCING.md:26, src/bitexact/repro.py:144-187).
"""

import hashlib
import json
import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import bxref as R

SELF_CHECK_SHA = "5053b757aad61165cb7d22d271f6b87acbc0edbd29ec06f352f1f4e022b1b214"


def rnd(v):
    return (Fraction(v) + Fraction(1, 2)).__floor__()


def bf16_bits(vals):
    return torch.tensor(vals, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy()


def rand_bf16_bits(N, K, seed, force=True):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    if force:
        w[0, :5] = torch.tensor([1e-9, -3e-8, 0.0, 2.0, -0.5]).to(torch.bfloat16)
    return w.view(torch.int16).numpy()


def test_self_check_hash():
    """Recompute the reference's 8 self-check fixtures with the oracle; the transcript hash must match."""
    vectors = {}
    values = [-(1 << 50) + 3, -17, -1, 0, 1, 17, (1 << 50) - 3]
    for shift in [-3, 0, 1, 7, 31]:
        got = R.rsh(np.array(values), shift).tolist()
        assert got == [rnd(Fraction(v) / Fraction(2) ** shift) for v in values]
        vectors[f"round_shift_{shift}"] = got
    denom = [3, 7, 11, 13, 17, 19, 23]
    vectors["floor_division"] = R.fdiv(np.array(values), np.array(denom)).tolist()
    assert vectors["floor_division"] == [a // b for a, b in zip(values, denom)]
    squares = [0, 1, 2, 3, 4, 17, (1 << 60) - 1]
    vectors["integer_sqrt"] = R.isqrt(np.array(squares)).tolist()
    assert vectors["integer_sqrt"] == [math.isqrt(x) for x in squares]
    wv = [[1.0, -0.5, 2 ** -30, -2 ** -28, 0.125, 0.0, 0.75, -0.25],
          [-0.25, 0.5, -0.125, 1.0, -2 ** -29, 2 ** -31, -0.75, 0.0]]
    bits = bf16_bits(wv)
    dec = R.decompose(bits)
    assert len(dec["rr"]) > 0
    q = np.array([[13, -7, 3, 11, 0, -5, 17, -19], [-2, 5, 7, -11, 3, 0, 1, 4]])
    shifts = np.array([-10, -6])
    y, bad = R.exact_linear(q, dec, shifts, checked=True)
    assert not bad
    expected = [[rnd(sum(Fraction(w) * int(x) for w, x in zip(row, qs)) * Fraction(2) ** (int(s) + R.FR))
                 for row in wv] for qs, s in zip(q.tolist(), shifts)]
    assert y.tolist() == expected
    vectors["bf16_linear_with_sparse_residual"] = y.tolist()
    enc = json.dumps(vectors, sort_keys=True, separators=(",", ":")).encode()
    assert hashlib.sha256(enc).hexdigest() == SELF_CHECK_SHA


def test_rshc_and_rsh():
    xs = [0, 1, -1, 5, -5, 6, -6, 7, -7, (1 << 50) + 3, -(1 << 50) - 3]
    for s in (-3, 0, 1, 2, 7, 40, 62):
        ref = [rnd(Fraction(x) / Fraction(2) ** s) for x in xs]
        assert R.rshc(np.array(xs), np.full(len(xs), s)).tolist() == ref
        assert R.rshc(np.array(xs), s).tolist() == ref
        assert R.rsh(np.array(xs), np.full(len(xs), s)).tolist() == ref
    # clamp: shifts beyond 62 act as 62 (exact 0 for |x| < 2^61)
    assert R.rshc(np.array([(1 << 60), -(1 << 60)]), 90).tolist() == [0, 0]


def test_bitlen_isqrt_fdiv():
    v = [0, 1, 2, 3, 255, 256, (1 << 40) - 1, 1 << 40, (1 << 62) + 5]
    assert R.bitlen(np.array(v)).tolist() == [x.bit_length() for x in v]
    x = np.concatenate([(np.int64(1) << np.arange(0, 62)) - 1, np.int64(1) << np.arange(0, 62)])
    assert R.bitlen(x).tolist() == [int(t).bit_length() for t in x]
    xs = [0, 1, 2, 3, 4, 15, 16, 17, (1 << 60) - 1, 1 << 60, (1 << 62) - 1, 12345678987654321]
    assert R.isqrt(np.array(xs)).tolist() == [math.isqrt(t) for t in xs]
    rg = random.Random(5)
    a = [rg.randrange(-(1 << 62), 1 << 62) for _ in range(5000)]
    b = [rg.randrange(1 << 11, 1 << rg.choice([12, 31, 34])) for _ in range(5000)]
    assert R.fdiv(np.array(a), np.array(b)).tolist() == [p // q for p, q in zip(a, b)]
    a2 = [t >> 2 for t in a]
    assert R.rdiv(np.array(a2), np.array(b)).tolist() == [rnd(Fraction(p, q)) for p, q in zip(a2, b)]


def test_div_round():
    rg = random.Random(0)
    a, p, r = [], [], []
    for _ in range(4000):
        rr = rg.randrange(1 << 11, 1 << rg.choice([12, 20, 31, 33]))
        pp = rg.randrange(-70, 60)
        lim = (1 << 61) if pp <= 0 else max(1, (rr << 61) >> (pp + 1)) // max(1, rr) * rr
        a.append(rg.randrange(-min(lim, 1 << 61), min(lim, 1 << 61) + 1))
        p.append(pp)
        r.append(rr)
    got = R.div_round(np.array(a), np.array(p), np.array(r)).tolist()
    assert got == [rnd(Fraction(x) * Fraction(2) ** pp / rr) for x, pp, rr in zip(a, p, r)]


def test_combine_shift_round():
    rg = random.Random(1)
    n = 4000
    T = [rg.randrange(-(1 << 58), 1 << 58) for _ in range(n)]
    d = [rg.choice([0, 0, 1, 7, 16, 30]) for _ in range(n)]
    B = [rg.randrange(-(1 << 50), 1 << 50) if dd else 0 for dd in d]
    p = [rg.randrange(-100, 3) for _ in range(n)]
    H, L = R.combine(np.array(T), np.array(d), np.array(B))
    assert all(h * (1 << 32) + lo == t * (1 << dd) + b
               for h, lo, t, dd, b in zip(H.tolist(), L.tolist(), T, d, B))
    got = R.shift_round_hl(H, L, np.array(p)).tolist()
    ref = [rnd(Fraction(t * (1 << dd) + b) * Fraction(2) ** pp) for t, dd, b, pp in zip(T, d, B, p)]
    inside = [abs(x) < 1 << 61 for x in ref]
    assert sum(inside) > n // 2
    assert [x for x, k in zip(got, inside) if k] == [x for x, k in zip(ref, inside) if k]


def test_quant():
    g = np.random.default_rng(0)
    P = g.integers(-(1 << 44), 1 << 44, (6, 64))
    P[1] //= 1 << 40
    P[2] = 0
    q, sh = R.quant(P, -40)
    assert int(np.abs(q).max()) <= 1 << 22
    for i in range(6):
        for j in range(64):
            assert int(q[i, j]) == rnd(Fraction(int(P[i, j])) * Fraction(2) ** (-40 - int(sh[i])))
        nz = P[i] != 0
        if nz.any():   # the row exponent is minimal: the largest |q| needs the 23rd bit
            assert int(np.abs(q[i]).max()) >= 1 << 21


def test_limbs_roundtrip():
    g = np.random.default_rng(0)
    for n in (1, 2, 3):
        x = g.integers(-R.LIM[n], R.LIM[n] + 1, (5, 40))
        x[0, 0], x[0, 1] = R.LIM[n], -R.LIM[n]
        lo, r = R.split_limbs(x, n)
        assert not r.any() and all(int(np.abs(t).max()) <= 128 for t in lo)
        assert (sum(t << (8 * i) for i, t in enumerate(lo)) == x).all()
        a = R.stack_limbs(x, n)
        assert a.dtype == np.int8 and a.shape[0] % 8 == 0 and a.shape[0] >= 24
        w = g.integers(-127, 128, (40, 7))
        assert (R.join_limbs(a.astype(np.int64) @ w, 5, n) == x @ w).all()
    _, r = R.split_limbs(np.array([R.LIM[2] + 1]), 2)
    assert r.any()


def test_decompose_invariants():
    bits = rand_bf16_bits(48, 256, 2)
    dec = R.decompose(bits)
    w = R.bf16_to_f64(bits)
    W, g, d = dec["W"], dec["g"], dec["d"]
    rec = W.astype(np.float64) * np.power(2.0, g.astype(np.float64))[:, None]
    gf = g - d
    rec[dec["rr"], dec["rc"]] += dec["rv"].astype(np.float64) * np.power(2.0, gf[dec["rr"]].astype(np.float64))
    assert (rec == w).all() and len(dec["rr"]) > 0
    assert int(np.abs(W).max()) <= R.LIM3
    # minimality of g: one grid step finer would overflow 3 limbs (rows with any weight)
    nzrow = (W != 0).any(1)
    assert (np.abs(W[nzrow]).max(1) > R.LIM3 // 2).all()
    # minimality of the residual grid gf = g - d: in every row with residual entries some rv is odd (a coarser
    # grid would lose that bit; a finer one would change d, rv and the model digest while keeping the value)
    for r in np.unique(dec["rr"]):
        assert (dec["rv"][dec["rr"] == r] & 1).any(), r
    assert (d[np.setdiff1d(np.arange(len(d)), dec["rr"])] == 0).all()   # rows without residual: d = 0


def test_emb_fixed_closed_form():
    """The embedding rounding (src/bitexact/exact/consts.py:131-135) against the exact rational rule
    floor(w 2^FR + 1/2) for every bf16 value of a sample that covers ties, tiny values and both signs."""
    from fractions import Fraction
    g = np.random.default_rng(11)
    bits = rand_bf16_bits(6, 64, 5)
    extra = np.array([0x0000, 0x8000, 0x3F80, 0xBF80, 0x3300, 0xB300, 0x3380, 0xB380, 0x3340, 0xB340, 0x2F80,
                      0x0001, 0x8001, 0x42FE, 0xC2FE], dtype=np.uint16).view(np.int16)
    bits = np.concatenate([bits.reshape(-1), extra, g.integers(0x2E00, 0x3E00, 64).astype(np.int16)])[None, :]
    m = R.engine_constants(bits, {}, {}, np.zeros((1, 32), np.int64), np.zeros((1, 32), np.int64), 0)
    sm, ex = R.bf16_parts(bits)
    for i in range(bits.shape[1]):
        w = Fraction(int(sm[0, i])) * (Fraction(2) ** int(ex[0, i]))
        ref = (w * (1 << R.FR) + Fraction(1, 2)).__floor__()
        assert int(m["emb"][0, i]) == ref, (hex(int(bits[0, i]) & 0xFFFF), int(m["emb"][0, i]), ref)


def test_linear_closed_form():
    """decompose + wmm + residual + epilogue against the exact rational sum over bf16 weights
    (reference tests/test_exact_ops.py:118-134)."""
    bits = rand_bf16_bits(48, 256, 2)
    dec = R.decompose(bits)
    g = np.random.default_rng(3)
    q = g.integers(-(1 << 22), (1 << 22) + 1, (5, 256))
    T = R.wmm_f64(q, dec["W"])
    assert T.tolist() == R.brute_matmul(q, dec["W"].T)
    sh = np.array([-30, -10, 0, -25, -18])
    y, flag = R.exact_linear(q, dec, sh)
    wf = [[Fraction(float(v)) for v in row] for row in R.bf16_to_f64(bits)]
    for m in range(5):
        for n in range(48):
            exact = sum(int(q[m, k]) * wf[n][k] for k in range(256)) * Fraction(2) ** (int(sh[m]) + R.FR)
            assert int(y[m, n]) == rnd(exact)


@pytest.mark.parametrize("shift", [-90, -33, -32, -31, -1, 0, 1, 20, 30])
def test_checked_epilogue_valid(shift):
    for value in [-1234567, -1, 0, 1, 1234567]:
        y, flag, _ = R.epilogue(np.array([[value]]), np.zeros((1, 1), np.int64), [0], [shift - R.FR], [0],
                                R.FR, True)
        assert int(y[0, 0]) == rnd(Fraction(value) * Fraction(2) ** shift) and not flag


def test_checked_epilogue_big_integer_oracle():
    rg = random.Random(19)
    cases = [(rg.randrange(-(1 << 59), 1 << 59), rg.randrange(-(1 << 50), 1 << 50),
              rg.randrange(31), rg.randrange(-100, 31)) for _ in range(2000)]
    t, b, d, shifts = (np.array(x) for x in zip(*cases))
    y, flag, bad = R.epilogue(t[None], b[None], d, shifts + d - R.FR, np.zeros(1, np.int64), R.FR, True)
    want = [rnd(Fraction(v * (1 << dd) + rs) * Fraction(2) ** s) for v, rs, dd, s in cases]
    assert flag
    for i, w in enumerate(want):
        assert bool(bad[0, i]) == (abs(w) >= 1 << 62)
        if not bad[0, i]:
            assert int(y[0, i]) == w
    for value in (-1, 1):   # unsupported positive shift fails closed
        _, f, _ = R.epilogue(np.array([[value]]), np.zeros((1, 1), np.int64), [0], [31 - R.FR], [0], R.FR, True)
        assert f


def test_int8_quant_rows_imm():
    g = np.random.default_rng(0)
    for nl in (1, 2, 3):
        z = g.integers(-(1 << 44), 1 << 44, (5, 64))
        z[1] //= 1 << 40
        q, as_, sh = R.quant_rows(z, nl)
        assert int(np.abs(q).max()) <= R.qmax(nl)
        assert ((as_ >= 1 << 29) & (as_ <= 1 << 30)).all()
        for i in range(5):      # closed form: q = round(rsh(z, sh) qmax / as_)
            for j in range(0, 64, 7):
                s = int(sh[i])
                zs = rnd(Fraction(int(z[i, j])) / Fraction(2) ** s) if s > 0 else int(z[i, j]) << -s
                assert int(q[i, j]) == rnd(Fraction(zs * R.qmax(nl), int(as_[i])))
        w = g.integers(-127, 128, (7, 64))
        assert R.imm(q, w).tolist() == R.brute_matmul(q, w.T)


def test_bmm_brute():
    g = np.random.default_rng(0)
    for Z, M, K, N in [(3, 5, 64, 7), (2, 4, 70, 9)]:
        a = g.integers(-R.LIM3, R.LIM3 + 1, (Z, M, K))
        b = g.integers(-R.LIM3, R.LIM3 + 1, (Z, K, N))
        got = R.bmm(a, b)
        for z in range(Z):
            assert got[z].tolist() == R.brute_matmul(a[z], b[z])


def test_exp2_and_softmax_precision():
    lut = R.exp2_table()
    g = np.random.default_rng(0)
    t = g.integers(0, 30 << R.FT2, 10000)
    v = R.exp2neg_lut(t, lut, 40).astype(np.float64) / 2 ** 40
    assert float(np.abs(v - np.power(2.0, -t / 2 ** R.FT2)).max()) < 3e-10
    # table endpoints: 2^0 and 2^-1 at 2^60
    assert int(lut[0]) == 1 << 60 and int(lut[-1]) == 1 << 59
    # a row whose max key gets weight exactly 2^FP, masked keys weight 0
    raw = np.array([[5 << 20, 3 << 20, 7 << 20, 1 << 20]])
    ok = np.array([[True, True, True, False]])
    p, den = R.softmax_w(raw, ok, np.array([[-1]]), R.FK, lut, R.FP)   # score = raw 2^-21
    assert int(p[0, 2]) == 1 << R.FP and int(p[0, 3]) == 0 and int(den[0, 0]) == int(p.sum())
    assert (np.diff([p[0, 1], p[0, 0], p[0, 2]]) > 0).all()


def test_rms_precision():
    g = np.random.default_rng(1)
    for width in (512, 2048, 4096):
        x = g.integers(-(200 << R.FR), 200 << R.FR, (4, width))
        x[1] //= 1 << 12
        x[2] = (1 << 40) - 1
        r, er = R.rms(x)
        assert ((r >= 1 << 30) & (r < 1 << 31)).all()
        ref = np.sqrt(((x.astype(np.float64) / 2 ** R.FR) ** 2).mean(-1) + 1e-5)
        assert np.allclose(r.astype(np.float64) * np.power(2.0, er.astype(np.float64)), ref, rtol=1e-7)


def test_paged_layout_roundtrip():
    g = np.random.default_rng(2)
    c = g.integers(-R.LIM3, R.LIM3 + 1, (3, 2, 16, 2 * 64))
    lim = R.to_limbs(c).astype(np.int64)
    k = lim[..., :64] + (lim[..., 64:128] << 8) + (lim[..., 128:192] << 16)
    v = lim[..., 192:256] + (lim[..., 256:320] << 8) + (lim[..., 320:384] << 16)
    assert (k == c[..., :64]).all() and (v == c[..., 64:]).all() and (lim[..., 384:] == 0).all()


def test_rope_inv_freq_llama3():
    """Pinned against transformers' own llama3 rule (the reference's dependency) where it imports."""
    try:
        import torch
        from transformers import LlamaConfig
        from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    except ImportError:
        ROPE_INIT_FUNCTIONS = None
    if ROPE_INIT_FUNCTIONS is not None:
        for hd in (64, 128):
            cfg = LlamaConfig(hidden_size=hd * 32, num_attention_heads=32, num_key_value_heads=8, head_dim=hd,
                              rope_theta=500000.0, max_position_embeddings=131072,
                              rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                            "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
            try:
                want = ROPE_INIT_FUNCTIONS["llama3"](cfg, "cpu")[0]
            except TypeError:
                want = ROPE_INIT_FUNCTIONS["llama3"](cfg, torch.device("cpu"), None)[0]
            assert np.array_equal(R.llama3_inv_freq(hd), want.double().numpy())
    inv = R.llama3_inv_freq()
    base = 1.0 / 500000.0 ** (np.arange(0, 64, 2) / 64)
    assert inv[0] == np.float32(base[0])           # high frequency: unscaled
    assert np.isclose(inv[-1], base[-1] / 32)      # low frequency: divided by the factor
    c, s = R.rope_tables(16, R.FT, inv)
    assert (c[0] == 1 << 30).all() and (s[0] == 0).all()


def test_rope_position_zero_is_a_scale():
    """At position 0 the tables are cos = 2^FT, sin = 0: rope is a plain scale, so q = y 2^FT and k, v are
    single roundings of y (closed forms independent of the rope formula)."""
    cos, sin = R.rope_tables(4, R.FT_ROPE, R.llama3_inv_freq(64))
    assert cos[0].tolist() == [1 << R.FT_ROPE] * 32 and not sin[0].any()
    rng = np.random.default_rng(3)
    B, T, H, HKV, HD = 1, 1, 4, 2, 64
    y = rng.integers(-(1 << 30), 1 << 30, (1, (H + 2 * HKV) * HD))
    Pq, k, v = R.rope_y(y, np.zeros((1, 1), np.int64), cos, sin, B, T, (H, HKV, HD))
    yy = [int(x) for x in y[0]]
    assert [int(x) for x in Pq.reshape(-1)] == [x << R.FT_ROPE for x in yy[:H * HD]]
    rnd = lambda x, s: math.floor(Fraction(x, 1 << s) + Fraction(1, 2))
    assert [int(x) for x in k.reshape(-1)] == [rnd(x << R.FT_ROPE, R.FR + R.FT_ROPE - R.FK) for x in yy[H * HD:(H + HKV) * HD]]
    assert [int(x) for x in v.reshape(-1)] == [rnd(x, R.FR - R.FV) for x in yy[(H + HKV) * HD:]]


def test_rope_is_a_rotation():
    """The integer rope of (x1, x2) by (c, s) preserves x1^2 + x2^2 up to c^2 + s^2 (a rotation scaled by the
    table's modulus), for every position of the tables."""
    cos, sin = R.rope_tables(64, R.FT_ROPE, R.llama3_inv_freq(64))
    rng = np.random.default_rng(4)
    y = rng.integers(-(1 << 20), 1 << 20, (64, 3 * 64))
    pos = np.arange(64).reshape(1, 64)
    Pq, _, _ = R.rope_y(y, pos, cos, sin, 1, 64, (1, 1, 64))
    for t in range(64):
        x = [int(a) for a in y[t, :64]]
        p = [int(a) for a in Pq[0, t, 0]]
        for d in range(32):
            c, s = int(cos[t, d]), int(sin[t, d])
            assert p[d] ** 2 + p[d + 32] ** 2 == (x[d] ** 2 + x[d + 32] ** 2) * (c * c + s * s)


def test_norm24_and_int8_post_closed_forms():
    rng = np.random.default_rng(5)
    rnd = lambda x, s: math.floor(Fraction(x, 1 << s) + Fraction(1, 2)) if s > 0 else x << -s
    mant0 = rng.integers(1, 1 << 40, 200)
    e0 = rng.integers(-50, 10, 200)
    mant, e = R.norm24(mant0, e0)
    for a, b, mm, ee in zip(mant0.tolist(), e0.tolist(), mant.tolist(), e.tolist()):
        assert (1 << 23) <= mm <= (1 << 24)
        assert abs(Fraction(mm) * Fraction(2) ** ee - Fraction(a) * Fraction(2) ** b) <= Fraction(2) ** (ee - 1)
    acc = rng.integers(-(1 << 38), 1 << 38, (3, 50))
    m = rng.integers(-(1 << 20), 1 << 20, 50)
    mant = rng.integers(1 << 23, (1 << 24) + 1, 3)
    e = rng.integers(-40, -10, 3)
    y, flag = R.int8_post(acc, m, 40, mant, e)
    for i in range(3):
        for j in range(50):
            t = rnd(int(acc[i, j]) * int(m[j]), 40)
            assert int(y[i, j]) == rnd(t * int(mant[i]), 24 - R.FR8 - int(e[i]))


def test_silu_mul_closed_forms():
    """silu(g) u: the sigmoid is within a few units of 2^30 / (1 + e^-g), sig(g) + sig(-g) = 2^30 +- 1, and
    s = silu(g) at FR is within 2^-20 relative (plus 1 unit) of the real value; P = s u exactly."""
    import math
    lut = R.exp2_table()
    rng = np.random.default_rng(7)
    g = np.concatenate([rng.integers(-(20 << 24), 20 << 24, 4000), np.array([0, 1, -1, 64 << 24, -(64 << 24)])])
    u = rng.integers(-(1 << 28), 1 << 28, g.shape[0])
    P, eps, ok = R.silu_mul(g, u, lut)
    assert ok and eps == -2 * R.FR
    Pp, _, _ = R.silu_mul(g, np.ones_like(g), lut)
    Pn, _, _ = R.silu_mul(-g, np.ones_like(g), lut)
    assert np.array_equal(P, Pp * u)                        # s u exactly
    # silu(g) - silu(-g) = g exactly in the reals; the integer rule keeps it within 2 units + g 2^-29
    assert np.all(np.abs(Pp - Pn - g) <= 2 + np.abs(g) // (1 << 29))
    for gi, si in zip(g[:500].tolist(), Pp[:500].tolist()):
        x = gi / 2.0 ** 24
        want = x / (1.0 + math.exp(-x)) * 2.0 ** 24
        assert abs(si - want) <= 1 + abs(want) * 2.0 ** -20, (gi, si, want)
    assert Pp[g.shape[0] - 5] == 0                          # silu(0) = 0
    # a gate beyond 2^32 or a product beyond 2^62 bits is flagged
    assert not R.silu_mul(np.array([(1 << 32) + 1]), np.array([1]), lut)[2]
    assert not R.silu_mul(np.array([1 << 32]), np.array([1 << 31]), lut)[2]


def test_exp2_table_accuracy():
    """Every entry of the 2^-f table is within 2 float64 units (256 at 2^59..2^60) of the exact 2^(60 - i / 2^14)
    (50-digit decimal arithmetic): a wrong index, sign or scale misses by far more. End points are exact."""
    from decimal import Decimal, getcontext
    getcontext().prec = 50
    t = R.exp2_table()
    assert t.shape == ((1 << 14) + 1,) and t[0] == 1 << 60 and t[-1] == 1 << 59
    ln2 = Decimal(2).ln()
    for i in range(0, (1 << 14) + 1, 7):
        exact = (Decimal(2) ** 60) * (-(Decimal(i) * ln2) / (1 << 14)).exp()
        assert abs(Decimal(int(t[i])) - exact) <= 256, i
