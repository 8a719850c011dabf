"""CPU restatement of the reference's integer rules for the exact / int8 linear and attention path.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it. The product (bitexact-llm_amd/) never imports it and has no CPU path.

Everything is numpy int64 (two's complement, wrapping like torch's CPU int64) or Python int. Shifts follow
torch's CPU rules where the reference could produce counts >= 64: `<<` by >= 64 gives 0, `>>` by >= 64
gives the sign (the helpers _shl / _sar); every other shift stays in [0, 63] by the reference's own clamps.
Each function cites the reference function it restates (paths under the reference checkout).

How each function is pinned (tests/test_oracle.py):
  rshc / rsh / fdiv / rdiv / isqrt / bitlen / div_round / combine / shift_round_hl / quant
      against Fraction / math.isqrt / int.bit_length closed forms, and the self-check fixture hash
  split/stack/join_limbs             round-trip invariants and an integer matmul
  decompose + wmm_f64 + residual + epilogue
                                     the closed form round(sum_k q w_bf16 2^(sh+FR)) as an exact Fraction,
                                     the self-check fixture `bf16_linear_with_sparse_residual`, and the
                                     reconstruction invariant W 2^g + R 2^gf == w
  epilogue(checked) flag             the big-integer rule |y| >= 2^62 (reference tests/test_model_bounds.py)
  quant_rows / rdiv32 / bitlen32     closed forms and rdiv equality near ties
  imm / bmm / int8 GEMM              brute-force Python-int matmul
  exp2neg_lut / softmax_w / rms /    golden vectors written from the reference (tests/golden/) plus
  silu_mul / gu_silu_y               the precision bounds of the reference's own tests
  paged attention                    softmax_w + exact matmuls (the reference's own test formulation,
                                     tests/test_vllm_exact_attn.py:38-41)
  rope_y / q_group                   position-0 scale and exact-rotation closed forms; quant (pinned) + permutation
  llama3_inv_freq                    transformers' own llama3 rule, element for element
  exp2_table                         every entry within 2 float64 units of 2^(60 - i/2^14) (50-digit decimal)
  first_argmax                       numpy argmax (documented: the first occurrence of the maximum)
  engine_forward / engine_logits     a composition of the pinned functions above, in the order of the
                                     reference's engine; checked further on the GPU by batch invariance
"""

import math

import numpy as np

I64 = np.int64

# ---- constants (src/bitexact/exact/consts.py:23-30, src/bitexact/exact/ops.py:14-23, segs.py:21) ----
LIM = {1: 127, 2: 32639, 3: 8355711}            # src/bitexact/intops.py:11
FR = 24
FT = 30
EXP2_BITS = 14
EXP2_ONE = 60
LIM3 = LIM[3]
QB = 22
FN = 40
FT2 = 26
FZ = 26
L2E28 = 387270501
L2E30 = 1549082005
L2E28_HD = {64: L2E28, 128: 273841598}
EPS60 = 11529215046068
NEG_BIG = -(1 << 20)
FK, FV, FP = 17, 19, 22
NEG = -(1 << 62)


def _a(x):
    return np.asarray(x, dtype=I64)


def _shl(x, s):
    """torch CPU `x << s` for int64 (s >= 0): 0 when s >= 64, else the wrapped product."""
    x, s = np.broadcast_arrays(_a(x), _a(s))
    out = np.left_shift(x, np.minimum(s, 63))
    return np.where(s >= 64, I64(0), out)


def _sar(x, s):
    """torch CPU `x >> s` for int64 (s >= 0): arithmetic shift with the count clamped to 63."""
    return np.right_shift(_a(x), np.minimum(_a(s), 63))


# ---- src/bitexact/intops.py ----
def bitlen(x):
    """Bit length of int64 x >= 0 (intops.bitlen, src/bitexact/intops.py:14-21); exact by integer compare."""
    x = _a(x)
    b = np.frexp(x.astype(np.float64))[1].astype(I64)
    up = _shl(np.ones_like(b), np.maximum(b - 1, 0)) > x
    return np.where(x > 0, b - up.astype(I64), I64(0))


def rsh(x, s):
    """round(x / 2^s) ties up for s > 0, x * 2^-s for s <= 0 (src/bitexact/intops.py:24-33)."""
    x = _a(x)
    if np.isscalar(s) or np.ndim(s) == 0:
        s = int(s)
        if s > 0:
            return (x + I64(1 << (s - 1))) >> I64(s)
        return _shl(x, -s)
    s = _a(s)
    pos = np.maximum(s, 0)
    neg = np.maximum(-s, 0)
    half = np.where(pos > 0, _shl(np.ones_like(pos), np.maximum(pos - 1, 0)), I64(0))
    return _shl(_sar(x + half, pos), neg)


def fdiv(a, b):
    """floor(a / b), b > 0 (src/bitexact/intops.py:36-38)."""
    return np.floor_divide(_a(a), _a(b))


def rdiv(a, b):
    """round(a / b) ties up (src/bitexact/intops.py:41-43)."""
    a, b = _a(a), _a(b)
    return fdiv(2 * a + b, 2 * b)


def isqrt(x):
    """floor(sqrt(x)), x >= 0 (src/bitexact/intops.py:46-52): float64 estimate + integer correction."""
    x = _a(x)
    s = np.floor(np.sqrt(x.astype(np.float64))).astype(I64)
    for _ in range(2):
        s = np.where(s * s > x, s - 1, s)
        s = np.where((s + 1) * (s + 1) <= x, s + 1, s)
    return s


def first_argmax(v):
    """First maximum index per row (src/bitexact/intops.py:55-59)."""
    return np.argmax(_a(v), axis=-1)      # numpy argmax returns the first maximum


def split_limbs(x, n):
    """Signed base-256 digits, least significant first (src/bitexact/intops.py:62-70)."""
    out, r = [], _a(x)
    for _ in range(n):
        lo = ((r + 128) & 255) - 128
        out.append(lo)
        r = (r - lo) >> 8
    return out, r


def stack_limbs(q, n):
    """[n M padded to >= 24 rows and a multiple of 8, K] int8 (src/bitexact/intops.py:73-79)."""
    a = np.concatenate([lo.astype(np.int8) for lo in split_limbs(q, n)[0]])
    rows = a.shape[0]
    pad = max(24, (rows + 7) // 8 * 8) - rows
    return np.concatenate([a, np.zeros((pad, a.shape[1]), np.int8)]) if pad else a


def join_limbs(c, M, n):
    """sum_i c[iM:(i+1)M] 2^(8i) (src/bitexact/intops.py:82-87)."""
    c = _a(c)
    acc = c[:M].copy()
    for i in range(1, n):
        acc = acc + (c[i * M:(i + 1) * M] << I64(8 * i))
    return acc


# ---- src/bitexact/exact/ops.py ----
def rshc(x, s):
    """round(x / 2^s) with s clamped to [-62, 62] (src/bitexact/exact/ops.py:25-34)."""
    x = _a(x)
    if np.isscalar(s) or np.ndim(s) == 0:
        s = max(-62, min(62, int(s)))
        return ((x + I64(1 << (s - 1))) >> I64(s)) if s > 0 else (x << I64(-s))
    s = np.clip(_a(s), -62, 62)
    pos = np.maximum(s, 0)
    half = np.where(pos > 0, I64(1) << np.maximum(pos - 1, 0), I64(0))
    return ((x + half) >> pos) << np.maximum(-s, 0)


def div_round(a, p, r, chunk=28):
    """round(a 2^p / r) by 28-bit long division (src/bitexact/exact/ops.py:37-57)."""
    a, r = np.broadcast_arrays(_a(a), _a(r))
    p = np.broadcast_to(_a(p), a.shape)
    Q = np.floor_divide(a, r)
    R = a - Q * r
    left = np.maximum(p, 0)
    for _ in range(3):
        c = np.minimum(left, chunk)
        X = R << c
        q1 = np.floor_divide(X, r)
        Q = (Q << c) + q1
        R = X - q1 * r
        left = left - c
    up = Q + (2 * R >= r).astype(I64)
    k = np.clip(-p, 1, 62)
    down = (Q + (I64(1) << (k - 1))) >> k
    return np.where(p >= 0, up, down)


def combine(T, d, B):
    """(H, L): H 2^32 + L = T 2^d + B, 0 <= L < 2^32 (src/bitexact/exact/ops.py:60-66)."""
    T, d, B = np.broadcast_arrays(_a(T), _a(d), _a(B))
    s = 32 - d
    H = T >> s
    L = (T & ((I64(1) << s) - 1)) << d
    L = L + B
    return H + (L >> 32), L & I64(0xFFFFFFFF)


def shift_round_hl(H, L, p):
    """round((H 2^32 + L) 2^p) (src/bitexact/exact/ops.py:69-79)."""
    H, L, p = np.broadcast_arrays(_a(H), _a(L), _a(p))
    k = np.maximum(-p, 0)
    pp = np.clip(p, 0, 30)
    up = (H << (32 + pp)) + (L << pp)
    k1 = np.clip(k, 1, 31)
    small = (H << (32 - k1)) + ((L + (I64(1) << (k1 - 1))) >> k1)
    k2 = np.clip(k, 32, 94)
    carry = np.where(k2 == 32, (L + I64(1 << 31)) >> 32, _shl(np.ones_like(L), np.maximum(k2 - 33, 0)))
    big = (H + carry) >> np.minimum(k2 - 32, 62)
    return np.where(p >= 0, up, np.where(k < 32, small, big))


def quant(P, eps):
    """Per-row power-of-two quantization, |q| <= 2^22 (src/bitexact/exact/ops.py:82-89). Returns (q, sh)."""
    P = _a(P)
    eps = np.broadcast_to(_a(eps), P.shape) if np.ndim(eps) else np.full(P.shape, int(eps), I64)
    e = np.where(P != 0, bitlen(np.abs(P)) + eps, I64(NEG_BIG))
    sh = np.maximum(e.max(-1) - QB, NEG_BIG)
    return rshc(P, sh[..., None] - eps), sh


def rms(x):
    """(r, er): rms = r 2^er, 2^30 <= r < 2^31 (src/bitexact/exact/ops.py:92-105)."""
    x = _a(x)
    D = x.shape[-1]
    lg = D.bit_length() - 1
    assert D == 1 << lg and lg <= 12, "row length a power of two <= 4096"
    amax = np.maximum(np.abs(x).max(-1), 1)
    shx = np.maximum(bitlen(amax) - 25, -6)
    xs = rshc(x, shx[:, None])
    S = (xs * xs).sum(-1)
    T = S + rshc(np.full(S.shape, EPS60 * D, I64), 60 - 2 * (FR - shx))
    m = (62 + lg - bitlen(T)) // 2
    s = 2 * m - lg
    V = np.where(s >= 0, T << np.maximum(s, 0), T >> np.maximum(-s, 0))
    return isqrt(V), shx - FR - m


def ndiv(x, gm, ge, r, er):
    """x gamma / rms at FN (src/bitexact/exact/segs.py:49-51)."""
    return div_round(_a(x) * _a(gm), _a(ge) - FR - _a(er)[:, None] + FN, _a(r)[:, None])


def norm_quant(x, gm, ge):
    """rms + ndiv + quant(-FN) (src/bitexact/exact/segs.py:59-63). Returns (q int32, sh, flag)."""
    x = _a(x)
    r, er = rms(x)
    q, sh = quant(ndiv(x, gm, ge, r, er), -FN)
    return q.astype(np.int32), sh, bool(np.abs(x).max() >= 1 << 40)


def exp2_table():
    """2^-f at 2^60 for f = i / 2^14, i = 0 .. 2^14 (src/bitexact/exact/consts.py:110-115)."""
    import torch                                   # the reference's float64 pow (CPU): its rounding, bit for bit
    f = torch.arange((1 << EXP2_BITS) + 1, dtype=torch.float64) / (1 << EXP2_BITS)
    return torch.round(torch.pow(2.0, -f) * 2.0 ** EXP2_ONE).long().numpy()


def exp2neg_lut(t, lut, out_bits):
    """2^-t at out_bits, t >= 0 at FT2 bits (src/bitexact/exact/ops.py:108-116)."""
    t = _a(t)
    lut = _a(lut)
    n = t >> FT2
    f = t & ((1 << FT2) - 1)
    idx = f >> (FT2 - EXP2_BITS)
    rr = f & ((1 << (FT2 - EXP2_BITS)) - 1)
    a = lut[idx]
    v = a + rshc((lut[idx + 1] - a) * rr, FT2 - EXP2_BITS)
    return rshc(v, EXP2_ONE - out_bits + n)


def softmax_w(raw, ok, sh, kbits, lut, fp, l2e=None):
    """Attention weights at fp bits and row sums (src/bitexact/exact/ops.py:133-143)."""
    raw = np.where(ok, _a(raw), I64(NEG))
    z = raw.max(-1, keepdims=True) - raw
    zf = np.minimum(rshc(z, kbits + 3 - _a(sh) - FZ), I64(48 << FZ))
    t = rshc(zf * I64(L2E28 if l2e is None else l2e), FZ + 28 - FT2)
    p = np.where(ok, exp2neg_lut(t, lut, fp), I64(0))
    return p, p.sum(-1, keepdims=True)


def attn_div(num, den):
    """o = round(num 2^(FR-FV) / den) (src/bitexact/exact/segs.py:108-113, before the regroup)."""
    return div_round(_a(num), FR - FV, _a(den))


def silu_mul(g, u, lut):
    """silu(g) u for g, u at FR -> (P, eps, ok): P 2^eps the product, ok when every |s| |u| < 2^62 by bit
    lengths and |g| <= 2^32 (src/bitexact/exact/ops.py:119-130)."""
    g, u = np.broadcast_arrays(_a(g), _a(u))
    a = np.minimum(np.abs(g), I64(64 << FR))
    t = rshc(a * I64(L2E30), FR + 30 - FT2)
    E = exp2neg_lut(t, lut, 30)                                  # e^-|g| at 2^30
    den = I64(1 << 30) + E
    sig = np.where(g >= 0, rdiv(np.full_like(E, 1 << 60), den), rdiv(E << I64(30), den))
    gc = np.clip(g, -(1 << 32), 1 << 32)
    s = rshc(gc * sig, 30)
    ok = bool(((bitlen(np.abs(s)) + bitlen(np.abs(u))) <= 62).all()) and int(np.abs(g).max(initial=0)) <= 1 << 32
    return s * u, -2 * FR, ok


def gu_silu_y(y, lut):
    """Segs.gu_silu_y = silu_y + quant_silu (src/bitexact/exact/segs.py:120-128, 180-182): y int64 [M, 2 ff]
    (gate | up) at FR -> (q int32, sh, flag) with flag = not ok."""
    y = _a(y)
    ff = y.shape[1] // 2
    P, eps, ok = silu_mul(y[:, :ff], y[:, ff:], lut)
    q, sh = quant(P, eps)
    return q.astype(np.int32), sh, not ok


def add_norm_y(y, x, gm, ge):
    """Segs.add_norm_y = add_y + norm_q (src/bitexact/exact/segs.py:40-41, 175-178): x + y, then norm_quant.
    Returns (x + y, q, sh, flag)."""
    x = _a(x) + _a(y).reshape(np.shape(x))
    q, sh, flag = norm_quant(x, gm, ge)
    return x, q, sh, flag


# ---- src/bitexact/exact/consts.py ----
def bf16_parts(bits):
    """bf16 raw bits (uint16 / int16 array) -> (signed significand, exponent): w = sm 2^ex
    (src/bitexact/exact/consts.py:33-42)."""
    b = _a(np.asarray(bits).view(np.uint16)) & 0xFFFF
    e = (b >> 7) & 0xFF
    assert not bool((e == 255).any()), "inf/nan weight"
    m = b & 0x7F
    mag = np.where(e > 0, m | 0x80, m)
    ex = np.where(e > 0, e, 1) - 134
    sm = np.where((b >> 15) == 1, -mag, mag)
    return sm, ex


def _bitlen9(x):
    out = np.zeros_like(x)
    for i in range(9):
        out = np.where(x >> i != 0, i + 1, out)
    return out


def _lowbit9(x):
    out = np.full_like(x, 99)
    for i in range(8, -1, -1):
        out = np.where(((x >> i) & 1) == 1, i, out)
    return out


def bf16_to_f64(bits):
    sm, ex = bf16_parts(bits)
    return sm.astype(np.float64) * np.power(2.0, ex.astype(np.float64))


def decompose(bits):
    """bf16 [N, K] (raw bits) -> dict(limbs int8 [3, N, K], g, d, rr, rc, rv)
    (src/bitexact/exact/consts.py:67-107). Residual COO in row-major (rr, rc) order."""
    sm, ex = bf16_parts(bits)
    mag = np.abs(sm)
    nz = mag > 0
    top = np.where(nz, ex + _bitlen9(mag), -10 ** 6).max(1)
    g = top - 23
    while True:
        sh = np.minimum(ex - g[:, None], 40)
        big = nz & (sh >= 0) & ((mag << np.maximum(sh, 0)) > LIM3)
        bad = big.any(1)
        if not bool(bad.any()):
            break
        g = np.where(bad, g + 1, g)
    g = np.where(top < -10 ** 5, 0, g)
    sh = ex - g[:, None]
    up = sh >= 0
    dmag = np.where(up, mag << np.clip(sh, 0, 40), mag >> np.clip(-sh, 0, 40))
    rmag = mag - np.where(up, mag, dmag << np.clip(-sh, 0, 40))
    rmag = np.where(up, 0, rmag)
    W = np.where(sm < 0, -dmag, dmag)
    has = rmag > 0
    low = np.where(has, ex + _lowbit9(rmag), 10 ** 6)
    gf = np.minimum(low.min(1), g)
    d = g - gf
    assert int(d.max()) <= 30, "residual grid too fine"
    rr, rc = np.nonzero(has)
    rsh_ = ex[rr, rc] - gf[rr]
    rm_ = rmag[rr, rc]
    rv = np.where(rsh_ >= 0, rm_ << np.maximum(rsh_, 0), rm_ >> np.maximum(-rsh_, 0))
    rv = np.where(sm[rr, rc] < 0, -rv, rv)
    lo, rem = split_limbs(W, 3)
    assert not bool(rem.any())
    return {"limbs": np.stack([x.astype(np.int8) for x in lo]), "W": W, "g": g.astype(I64),
            "d": d.astype(I64), "rr": rr.astype(I64), "rc": rc.astype(I64), "rv": rv.astype(I64)}


def to_ell(rr, rc, rv, N):
    """Padded per-row residual lists (src/bitexact/vllm_plugin/exact_gemm.py:264-282): cnt, ec, ev."""
    cnt = np.bincount(rr, minlength=N).astype(I64) if len(rr) else np.zeros(N, I64)
    R = int(cnt.max()) if len(rr) else 0
    start = np.cumsum(cnt) - cnt
    j = np.arange(len(rr)) - start[rr] if len(rr) else np.zeros(0, I64)
    ec = np.zeros((N, max(R, 1)), I64)
    ev = np.zeros((N, max(R, 1)), I64)
    if len(rr):
        ec[rr, j] = rc
        ev[rr, j] = rv
    return cnt, ec, ev, R


# ---- src/bitexact/exact/wmm.py ----
def wmm_f64(q, W):
    """T = q W^T exactly: q's 3 limbs as float64 [3M, K] times W^T (|W| <= 2^23) -- every partial sum
    < 2^43 < 2^53, so float64 BLAS is exact in any order (src/bitexact/exact/wmm.py:117-121)."""
    q = _a(q)
    M = q.shape[0]
    A = np.concatenate(split_limbs(q, 3)[0]).astype(np.float64)
    C = (A @ _a(W).astype(np.float64).T).astype(I64)
    return C[:M] + (C[M:2 * M] << 8) + (C[2 * M:] << 16)


def residual(q, rr, rc, rv, N):
    """B [M, N] = sum over residual entries of q[:, k] v (src/bitexact/exact/wmm.py:124-129)."""
    q = _a(q)
    B = np.zeros((q.shape[0], N), I64)
    if len(rr):
        np.add.at(B.T, _a(rr), (q[:, _a(rc)] * _a(rv)).T)
    return B


def epilogue(T, B, d, g, sh, FR_=FR, checked=False):
    """round((T 2^d + B) 2^p), p = sh + g - d + FR, and the checked flag
    (src/bitexact/exact/wmm.py:132-150). With checked=True returns (y, flag_any, flag_per_element)."""
    d, g, sh = _a(d), _a(g), _a(sh)
    H, L = combine(T, d[None, :], B)
    p = sh[:, None] + (g - d)[None, :] + FR_
    y = shift_round_hl(H, L, p)
    if not checked:
        return y
    up_limit = I64(1) << (31 - np.clip(p, 0, 30))
    small_limit = I64(1) << (31 + np.clip(-p, 1, 31))
    up_lost = (H >= up_limit) | (H < -up_limit) | ((p > 30) & ((H != 0) | (L != 0)))
    small_lost = (H >= small_limit) | (H < -small_limit)
    lost = np.where(p >= 0, up_lost, (p > -32) & small_lost)
    bad = lost | (y <= -(1 << 62)) | (y >= 1 << 62)
    return y, bool(bad.any()), bad


def exact_linear(q, dec, sh, checked=True):
    """The whole exact linear (segs.lin_y over Lin on CPU, src/bitexact/exact/segs.py:25-32):
    y int64 [M, N] at FR and the checked flag."""
    T = wmm_f64(q, dec["W"])
    B = residual(q, dec["rr"], dec["rc"], dec["rv"], dec["W"].shape[0])
    if checked:
        y, flag, _ = epilogue(T, B, dec["d"], dec["g"], sh, FR, True)
        return y, flag
    return epilogue(T, B, dec["d"], dec["g"], sh, FR), False


# ---- src/bitexact/int8/ops.py ----
def qmax(nl):
    return 127 << (8 * (nl - 1))


def bitlen32(x):
    """Same integers as bitlen (src/bitexact/int8/ops.py:38-44); restated through bitlen."""
    return bitlen(x)


def rdiv32(a, b):
    """Same integers as rdiv in its range (src/bitexact/int8/ops.py:47-55)."""
    return rdiv(a, b)


def quant_rows(z, nl):
    """(q, as_, sh): q = round(rsh(z, sh) qmax / as_) (src/bitexact/int8/ops.py:24-35)."""
    z = _a(z)
    amax = np.maximum(np.abs(z).max(-1), 1)
    sh = bitlen(amax) - 30
    as_ = rsh(amax, sh)
    zs = rsh(z, sh[:, None])
    return rdiv(zs * qmax(nl), as_[:, None]), as_, sh


def imm(q, W):
    """Exact q @ W^T (src/bitexact/int8/ops.py:87-90): float64, |partial sums| < 2^53."""
    return (_a(q).astype(np.float64) @ _a(W).astype(np.float64).T).astype(I64)


def int_mm(a, w):
    """int8 [R, K] x int8 [N, K]^T -> exact int (int32 contract of gemm_skinny.int_mm,
    src/bitexact/int8/gemm_skinny.py:80-97)."""
    return imm(a, w)


# ---- src/bitexact/bmm.py ----
def bmm(a, b):
    """Exact [Z, M, K] x [Z, K, N] -> int64, by 3x3 limbs in float64 (each partial < 2^53 for K < 2^21)
    (src/bitexact/bmm.py:78-102 computes the same integers)."""
    a, b = _a(a), _a(b)
    la, ra = split_limbs(a, 3)
    lb, rb = split_limbs(b, 3)
    assert not ra.any() and not rb.any(), "operands within 3 limbs"
    out = np.zeros((a.shape[0], a.shape[1], b.shape[2]), I64)
    for i in range(3):
        for j in range(3):
            out += (la[i].astype(np.float64) @ lb[j].astype(np.float64)).astype(I64) << I64(8 * (i + j))
    return out


def brute_matmul(a, b):
    """Python-int matmul [M, K] x [K, N] (tiny shapes only)."""
    a = [[int(v) for v in r] for r in np.asarray(a).tolist()]
    bt = [[int(v) for v in c] for c in np.asarray(b).T.tolist()]
    return [[sum(x * y for x, y in zip(r, c)) for c in bt] for r in a]


# ---- paged limb-plane cache (src/bitexact/vllm_plugin/tri_paged.py:22-26, 311-348) ----
def to_limbs(c):
    """int32 cache [nb, HKV, bs, 2 HD] (K | V) -> int8 limb planes [nb, HKV, bs, 8 HD]."""
    c = _a(c)
    HD = c.shape[-1] // 2
    out = np.zeros(c.shape[:3] + (8 * HD,), np.int8)
    for part, o in ((c[..., :HD], 0), (c[..., HD:], 3)):
        lo, _ = split_limbs(part, 3)
        for i in range(3):
            out[..., (o + i) * HD:(o + i + 1) * HD] = lo[i].astype(np.int8)
    return out


def paged_attend(q, sh, qpos, c32, bt, rmap, lut, l2e):
    """Exact paged attention as the reference's test states it (tests/test_vllm_exact_attn.py:38-41 over
    src/bitexact/vllm_plugin/tri_exact_attn.py:1-15): q [R, HKV, M, HD], sh [R, HKV, M], qpos [R, M],
    c32 int32 cache [nb, HKV, bs, 2 HD], bt [*, nblk], rmap [R] -> num [R, HKV, M, HD], den [R, HKV, M, 1]."""
    q, sh, qpos, c32, bt, rmap = (_a(x) for x in (q, sh, qpos, c32, bt, rmap))
    R, HKV, M, HD = q.shape
    bs = c32.shape[2]
    num = np.zeros((R, HKV, M, HD), I64)
    den = np.zeros((R, HKV, M, 1), I64)
    for r in range(R):
        S = int(qpos[r].max()) + 1
        if S <= 0:
            continue
        s = np.arange(S)
        kv = c32[bt[rmap[r], s // bs], :, s % bs]                      # [S, HKV, 2 HD]
        for h in range(HKV):
            K, V = kv[:, h, :HD], kv[:, h, HD:]
            raw = bmm(q[r, h][None], K.T[None])[0]                    # [M, S]
            ok = s[None, :] <= qpos[r][:, None]
            p, dn = softmax_w(raw, ok, sh[r, h][:, None], FK, lut, FP, l2e)
            num[r, h] = bmm(p[None], V[None])[0]
            den[r, h] = dn
    return num, den


def attention_prefill(qg, shg, K, V, qpos, lut, l2e):
    """The unfused exact/model.py attention (src/bitexact/exact/model.py:114-120): qg int32 [Z, gT, HD],
    shg [Z, gT, 1], K / V [Z, S, HD] int32, qpos [Z, gT, 1] -> num [Z, gT, HD], den [Z, gT, 1]."""
    raw = bmm(qg, np.swapaxes(_a(K), 1, 2))
    ok = np.arange(raw.shape[-1])[None, None, :] <= _a(qpos)
    p, den = softmax_w(raw, ok, shg, FK, lut, FP, l2e)
    return bmm(p, V), den


# ---- RoPE tables (src/bitexact/llama.py:52-68): llama3 inverse frequencies in closed form ----
def llama3_inv_freq(hd=64, theta=500000.0, factor=32.0, low=1.0, high=4.0, orig=8192):
    """transformers' llama3 rope rule (the function src/bitexact/llama.py:57-62 calls; transformers 5.x
    modeling_rope_utils._compute_llama3_parameters), restated: float32 throughout, the power correctly rounded
    (float64 pow of the float32 exponent, rounded to float32, which is what torch's CPU float32 pow returns);
    returned widened to float64 as the reference's `.double()`."""
    f = np.float32
    e = np.arange(0, hd, 2).astype(f) / f(hd)
    inv = f(1.0) / np.power(np.float64(f(theta)), e.astype(np.float64)).astype(f)
    wl = f(2 * math.pi) / inv
    out = np.where(wl > f(orig / low), inv / f(factor), inv)
    smooth = (f(orig) / wl - f(low)) / (f(high) - f(low))
    mid = (f(1) - smooth) * out / f(factor) + smooth * out
    is_mid = ~(wl < f(orig / high)) & ~(wl > f(orig / low))
    return np.where(is_mid, mid, out).astype(np.float32).astype(np.float64)


def rope_tables(n_pos, bits, inv_freq):
    """Integer cos / sin at `bits` (src/bitexact/llama.py:65-68), with torch's float64 cos / sin on the CPU as the
    reference calls them."""
    import torch
    ang = torch.arange(n_pos, dtype=torch.float64)[:, None] * torch.from_numpy(np.asarray(inv_freq, np.float64))[None, :]
    return (torch.round(torch.cos(ang) * 2.0 ** bits).long().numpy(),
            torch.round(torch.sin(ang) * 2.0 ** bits).long().numpy())

# ---- RoPE + q quantization + regroup (src/bitexact/exact/segs.py:66-99) ----
FT_ROPE = 30                                    # cos / sin fractional bits (src/bitexact/exact/consts.py:24)


def _rope_full(x, c, s):
    """(x1 c - x2 s, x2 c + x1 s) over the two halves of the last axis (src/bitexact/exact/segs.py:66-69)."""
    hd = x.shape[-1]
    x1, x2 = x[..., :hd // 2], x[..., hd // 2:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def rope_y(y, pos, cos, sin, B, T, dm):
    """segs.rope_y (src/bitexact/exact/segs.py:78-86): y int64 [B T, (H + 2 HKV) HD] at FR, positions [B, T],
    integer tables [n_pos, HD / 2] -> (Pq [B, T, H, HD] at FR + FT, k [B, T, HKV, HD] at FK, v at FV)."""
    h, hkv, hd = dm
    y = _a(y).reshape(B, T, -1)
    pos = _a(pos)
    c, s = _a(cos)[pos][:, :, None], _a(sin)[pos][:, :, None]
    Pq = _rope_full(y[..., :h * hd].reshape(B, T, h, hd), c, s)
    k = rshc(_rope_full(y[..., h * hd:(h + hkv) * hd].reshape(B, T, hkv, hd), c, s), FR + FT_ROPE - FK)
    v = rshc(y[..., (h + hkv) * hd:].reshape(B, T, hkv, hd), FR - FV)
    return Pq, k, v


def q_group(Pq, k, v, y):
    """segs.q_group (src/bitexact/exact/segs.py:89-99): per (token, head) quant of q at -(FR + FT), grouped by
    KV head -> (qg int32 [B HKV, g T, HD], shg [B HKV, g T, 1], err)."""
    B, T, h, hd = Pq.shape
    hkv = k.shape[2]
    qi, shq = quant(Pq, -(FR + FT_ROPE))
    g = h // hkv
    qg = qi.reshape(B, T, hkv, g, hd).transpose(0, 2, 3, 1, 4).reshape(B * hkv, g * T, hd).astype(np.int32)
    shg = shq.reshape(B, T, hkv, g).transpose(0, 2, 3, 1).reshape(B * hkv, g * T, 1)
    err = bool((np.abs(_a(y)) >= 1 << 31).any() or (np.abs(k) > LIM3).any() or (np.abs(v) > LIM3).any()
               or (shq.max() > FK + 3 - FZ))
    return qg, shg, err


# ---- int8-mode row scales and the linear post-segment (src/bitexact/int8/ops.py:73-77,
# src/bitexact/int8/segs.py:62-67) ----
FR8 = 16                                        # int8 engine residual stream (src/bitexact/int8/consts.py:26)


def norm24(mant, e):
    """(mant, e) -> the same value with mant in [2^23, 2^24] (src/bitexact/int8/ops.py:73-76)."""
    b = bitlen(_a(mant)) - 24
    return rsh(_a(mant), b), _a(e) + b


def int8_post(acc, m, fmsh, mant, e, FR_=FR8):
    """segs.post (src/bitexact/int8/segs.py:62-67): t = rsh(acc m_c, fmsh); y = rsh(t mant_r, 24 - FR - e_r).
    Returns (y, flag) with flag = max |t| >= 2^38."""
    t = rsh(_a(acc) * _a(m)[None, :], int(fmsh))
    flag = bool(np.abs(t).max() >= 1 << 38) if t.size else False
    return rsh(t * _a(mant)[:, None], (24 - FR_ - _a(e))[:, None]), flag


# ---- int8-mode attention weights (src/bitexact/int8/segs.py:29-37, 92-100; src/bitexact/int8/ops.py:93-97)
# and the paged attention over the limb-plane cache (src/bitexact/vllm_plugin/tri_paged.py:1-26, 363-401) ----
FQ8, FP8 = 14, 20
FA8, FE8, EXP_MIN8 = 12, 30, -32
SC128 = 11863283
ZCLAMP8 = -(1 << 38)


def int8_exp_table():
    """e^x at FE bits, x = EXP_MIN .. 0 at step 2^-FA (src/bitexact/int8/consts.py:50-53)."""
    xs = np.arange(EXP_MIN8 << FA8, 1, dtype=np.float64) / (1 << FA8)
    return np.round(np.exp(xs) * float(1 << FE8)).astype(I64)


def int8_softmax(raw, ok, expt, hd):
    """int8 segs.softmax with the visibility mask given (src/bitexact/int8/segs.py:92-100)."""
    raw = np.where(ok, _a(raw), I64(NEG))
    d = raw - raw.max(-1, keepdims=True)
    base = 2 * FQ8 + 3 - FA8
    z = rsh(d, base) if hd == 64 else rsh(np.maximum(d, I64(ZCLAMP8)) * I64(SC128), base + 24)
    idx = np.maximum(z, -(1 << 40)) - I64(EXP_MIN8 << FA8)
    val = _a(expt)[np.maximum(idx, 0)]
    e = np.where(idx < 0, I64(0), val)                           # int8 ops.exp_of
    p = np.where(ok, rsh(e, FE8 - FP8), I64(0))
    return p, p.sum(-1, keepdims=True)


def paged_attend_int8(q, qpos, c32, bt, expt):
    """tri_paged.attend as the unfused int8 rules (int8 segs.softmax between two exact matmuls): q int64
    [R, HKV, M, HD], qpos [R, M], c32 int32 cache [nb, HKV, bs, 2 HD], bt [R, nblk]."""
    q, qpos, c32, bt = (_a(x) for x in (q, qpos, c32, bt))
    R, HKV, M, HD = q.shape
    bs = c32.shape[2]
    num = np.zeros((R, HKV, M, HD), I64)
    den = np.zeros((R, HKV, M, 1), I64)
    for r in range(R):
        S = int(qpos[r].max()) + 1
        if S <= 0:
            continue
        s = np.arange(S)
        kv = c32[bt[r, s // bs], :, s % bs]
        for h in range(HKV):
            K, V = kv[:, h, :HD], kv[:, h, HD:]
            raw = bmm(q[r, h][None], K.T[None])[0]
            ok = s[None, :] <= qpos[r][:, None]
            p, dn = int8_softmax(raw, ok, expt, HD)
            num[r, h] = bmm(p[None], V[None])[0]
            den[r, h] = dn
    return num, den



# ---- int8-mode RMSNorm front, SiLU and the remaining int8 segments (src/bitexact/int8/ops.py:76-108,
# src/bitexact/int8/segs.py:47-118) ----
FG8, FT8, FV8 = 12, 16, 14
SILU_LIM8 = 32
EPS40 = 10995116                                # round(1e-5 2^40) (src/bitexact/int8/ops.py:18)


def int8_rms(x, FR_=FR8):
    """int8 ops.rms (src/bitexact/int8/ops.py:76-84): (r, shx) with rms = r 2^(shx - FR)."""
    x = _a(x)
    d = x.shape[-1]
    amax = np.maximum(np.abs(x).max(-1), 1)
    shx = bitlen(amax) - 24
    xs = rsh(x, shx[:, None])
    ms = (xs * xs).sum(-1) // d
    eps = rsh(np.full_like(shx, EPS40), 40 - 2 * (FR_ - shx))
    return isqrt(ms + eps), shx


def int8_pre_norm(x, gamma, nl, FR_=FR8, FG_=FG8):
    """int8 segs.pre_norm (src/bitexact/int8/segs.py:47-52): RMSNorm + quant_rows of x gamma, and the row scale
    norm24(rdiv(as_ << 30, r), sh - FG - shx - 30) -> (q, mant, e)."""
    x = _a(x)
    r, shx = int8_rms(x, FR_)
    q, as_, sh = quant_rows(x * _a(gamma), nl)
    mant, e = norm24(rdiv(as_ << I64(30), r), sh - FG_ - shx - 30)
    return q, mant, e


def int8_pre_plain(x, nl, FR_=FR8):
    """int8 segs.pre_plain (src/bitexact/int8/segs.py:56-59) -> (q, mant, e)."""
    q, as_, sh = quant_rows(x, nl)
    mant, e = norm24(as_, sh - FR_)
    return q, mant, e


def int8_silu_table():
    """SiLU(x) at FR bits, x in [-SILU_LIM, SILU_LIM] at step 2^-FA (src/bitexact/int8/consts.py:79-80), with torch's
    float64 exp on the CPU as the reference's offline build calls it."""
    import torch
    xs = torch.arange(-SILU_LIM8 << FA8, (SILU_LIM8 << FA8) + 1, dtype=torch.float64) / (1 << FA8)
    return torch.round(xs / (1.0 + torch.exp(-xs)) * (1 << FR8)).long().numpy()


def int8_exp_of(z, lut):
    """int8 ops.exp_of (src/bitexact/int8/ops.py:93-97): e^z at FE bits, 0 below EXP_MIN."""
    idx = _a(z) - I64(EXP_MIN8 << FA8)
    val = _a(lut)[np.maximum(idx, 0)]
    return np.where(idx < 0, I64(0), val)


def int8_silu(g, lut, FR_=FR8):
    """int8 ops.silu (src/bitexact/int8/ops.py:100-108): table at step 2^-FA with linear interpolation, identity
    above the table and 0 below it."""
    g, lut = _a(g), _a(lut)
    lo, hi = -SILU_LIM8 << FA8, SILU_LIM8 << FA8
    gi = g >> I64(FR_ - FA8)
    r = g - (gi << I64(FR_ - FA8))
    i = np.clip(gi, lo, hi - 1) - lo
    a = lut[i]
    v = a + rsh((lut[i + 1] - a) * r, FR_ - FA8)
    return np.where(gi >= hi, g, np.where(gi < lo, I64(0), v))


def _amax8(z):
    return I64(np.abs(_a(z)).max()) if np.size(z) else I64(0)


def int8_silu_mul(gu, lut, nl, FR_=FR8):
    """int8 segs.silu_mul (src/bitexact/int8/segs.py:112-118) -> (q, mant, e, flag); the flag compares the wrapped
    int64 product of the two maxima with 2^62, as the reference's int64 tensors do."""
    gu = _a(gu)
    ff = gu.shape[1] // 2
    g, u = gu[:, :ff], gu[:, ff:]
    sg = int8_silu(g, lut, FR_)
    with np.errstate(over="ignore"):
        flag = bool(_amax8(sg) * _amax8(u) >= I64(1 << 62))
    q, mant, e = int8_pre_plain(rsh(sg * u, FR_), nl, FR_)
    return q, mant, e, flag


def _rope8(x, c, s, FR_=FR8):
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    sh = FT8 + FR_ - FQ8
    return np.concatenate([rsh(x1 * c - x2 * s, sh), rsh(x2 * c + x1 * s, sh)], -1)


def int8_qkv(y, c, s, dm, FR_=FR8):
    """int8 segs.qkv (src/bitexact/int8/segs.py:77-87): y [B, T, (H + 2 HKV) HD] at FR, c / s [B, T, 1, HD / 2]
    -> (qg [B HKV, g T, HD], k, v [B, T, HKV, HD], flag)."""
    H, HKV, HD = dm
    y, c, s = _a(y), _a(c), _a(s)
    B, T = y.shape[0], y.shape[1]
    D = H * HD
    q = _rope8(y[..., :D].reshape(B, T, H, HD), c, s, FR_)
    k = _rope8(y[..., D:D + HKV * HD].reshape(B, T, HKV, HD), c, s, FR_)
    v = rsh(y[..., D + HKV * HD:].reshape(B, T, HKV, HD), FR_ - FV8)
    g = H // HKV
    qg = q.reshape(B, T, HKV, g, HD).transpose(0, 2, 3, 1, 4).reshape(B * HKV, g * T, HD)
    flag = bool(_amax8(q) > LIM3 or _amax8(k) > LIM3 or _amax8(v) > LIM3)
    return qg, k, v, flag


def int8_attn_out(num, den, T, nl, dm, FR_=FR8):
    """int8 segs.attn_out (src/bitexact/int8/segs.py:102-109): rdiv(num << (FR - FV), den), regrouped, pre_plain."""
    H, HKV, HD = dm
    num = _a(num)
    B = num.shape[0]
    g = H // HKV
    o = rdiv(num << I64(FR_ - FV8), _a(den))
    o = o.reshape(B, HKV, g, T, HD).transpose(0, 3, 1, 2, 4).reshape(B * T, H * HD)
    return int8_pre_plain(o, nl, FR_)


# ---- the exact decode engine (src/bitexact/vllm_plugin/exact_run.py:60-128, src/bitexact/exact/model.py:95-148) ----
def engine_constants(emb_bits, lin_bits, gammas, cos, sin, L):
    """Oracle-side model from raw bf16 bits: emb_bits [V, D], lin_bits {(i, name) or "lm": bits [N, K]},
    gammas {"0.ga": (m, e), ..., "gf": (m, e)}. Every linear is decomposed here (decompose above) and the
    embedding rounded to 2^-FR (src/bitexact/exact/consts.py:131-135)."""
    sm, ex = bf16_parts(emb_bits)
    s = ex + FR
    e = np.where(s >= 0, _shl(sm, np.maximum(s, 0)),
                 _sar(sm + _shl(np.ones_like(s), np.clip(-s - 1, 0, 62)), np.clip(-s, 0, 63)))
    return {"emb": e.astype(np.int32), "dec": {k: decompose(b) for k, b in lin_bits.items()}, "gam": dict(gammas),
            "cos": _a(cos), "sin": _a(sin), "lut": exp2_table(), "L": L}


def engine_forward(m, c32, ids, pos, slot, bt, rmap, dm):
    """ExactEngine.forward (src/bitexact/vllm_plugin/exact_run.py:60-128): one step over token rows. c32: per layer
    int32 caches [nb, HKV, bs, 2 HD] (K | V), updated in place. Returns (x [N, D] int64 at FR, err)."""
    H, HKV, HD = dm
    G = H // HKV
    ids, pos, bt, rmap = _a(ids), _a(pos), _a(bt), _a(rmap)
    slot = np.where(_a(slot) < 0, 0, _a(slot))
    N = ids.shape[0]
    qpos = np.repeat(pos[:, None], G, 1)
    lut, l2e = m["lut"], L2E28_HD[HD]
    err = False
    x = m["emb"][ids].astype(I64)
    q, sh, f = norm_quant(x, *m["gam"]["0.ga"])
    err |= f
    for i in range(m["L"]):
        dec = lambda n: m["dec"][(i, n)]
        y, _ = exact_linear(q, dec("wqkv"), sh, checked=False)
        Pq, k, v = rope_y(y, pos[:, None], m["cos"], m["sin"], N, 1, dm)
        qg, shg, e = q_group(Pq, k, v, y)
        err |= e
        c = c32[i]
        bs = c.shape[2]
        for n in range(N):
            c[slot[n] // bs, :, slot[n] % bs, :HD] = k[n, 0]
            c[slot[n] // bs, :, slot[n] % bs, HD:] = v[n, 0]
        num, den = paged_attend(qg.reshape(N, HKV, G, HD), shg.reshape(N, HKV, G), qpos, c, bt, rmap, lut, l2e)
        o = attn_div(num, den).reshape(N, H * HD)             # Segs.attn_out at T = 1: the regroup is a reshape
        qo, sho = quant(o, -FR)
        y, f = exact_linear(qo.astype(np.int32), dec("wo"), sho, checked=True)
        err |= f
        x, q, sh, f = add_norm_y(y, x, *m["gam"][f"{i}.gm"])
        err |= f
        y, _ = exact_linear(q, dec("wgu"), sh, checked=False)
        q, sh, f = gu_silu_y(y, lut)
        err |= f
        y, f = exact_linear(q, dec("wd"), sh, checked=True)
        err |= f
        if i + 1 < m["L"]:
            x, q, sh, f = add_norm_y(y, x, *m["gam"][f"{i + 1}.ga"])
            err |= f
        else:
            x = x + y
            err |= bool((np.abs(x) >= 1 << 40).any())
    return x, err


def engine_logits(m, h):
    """ExactEngine.logits (src/bitexact/vllm_plugin/exact_run.py:157-175): final norm + tied lm_head."""
    q, sh, f = norm_quant(h, *m["gam"]["gf"])
    y, f2 = exact_linear(q, m["dec"]["lm"], sh, checked=True)
    return y, f or f2
