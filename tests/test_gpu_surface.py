"""The reference's Python helper surface on the GPU (csrc/bx_elem.hip through bitexact.intops, bitexact.exact.ops,
the module-level bitexact.exact.segs stages, bitexact.int8.ops and bitexact.int8.segs) against the oracle and the
reference-written golden vectors, bit for bit; the reference's own GPU test call pattern
(tests/test_gpu_kernels.py:22-61: int8 Segs eager = compiled, rdiv32 / bitlen32 = rdiv / bitlen, exact Segs
pre_norm eager = compiled); and the int8 linear front to back (pre_norm -> int_mm -> post) against the oracle."""

import os

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))


def T(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def eq(t, ref):
    return np.array_equal(t.cpu().numpy(), np.asarray(ref))


def _edge_ints(g, n=4000):
    x = g.integers(-(1 << 62), 1 << 62, n) >> g.integers(0, 62, n)
    return np.concatenate([x, [0, 1, -1, 2, -2, 127, 128, -128, -129, (1 << 62) - 1, -(1 << 62)]])


def test_intops(dev):
    from bitexact import intops
    g = np.random.default_rng(1)
    x = _edge_ints(g)
    xp = np.abs(x)
    assert eq(intops.bitlen(T(xp, dev)), R.bitlen(xp))
    s = g.integers(-70, 70, x.shape)
    for sv in (s, 0, 5, -3, 62, 63):
        assert eq(intops.rsh(T(x >> 2, dev), T(sv, dev) if np.ndim(sv) else sv), R.rsh(x >> 2, sv)), sv
    b = g.integers(1, 1 << 40, x.shape)
    assert eq(intops.fdiv(T(x, dev), T(b, dev)), R.fdiv(x, b))
    assert eq(intops.rdiv(T(x >> 2, dev), T(b, dev)), R.rdiv(x >> 2, b))
    assert eq(intops.rdiv(T(x >> 2, dev), 7), R.rdiv(x >> 2, 7))
    assert eq(intops.isqrt(T(xp, dev)), R.isqrt(xp))
    q = g.integers(-(1 << 23), 1 << 23, (7, 96))
    for n in (1, 2, 3):
        lo, rem = intops.split_limbs(T(q, dev), n)
        rlo, rrem = R.split_limbs(q, n)
        assert all(eq(a, b_) for a, b_ in zip(lo, rlo)) and eq(rem, rrem)
        assert eq(intops.stack_limbs(T(q, dev), n), R.stack_limbs(q, n))
        c = g.integers(-(1 << 30), 1 << 30, (n * 7, 40))
        assert eq(intops.join_limbs(T(c, dev).to(torch.int32), 7, n), R.join_limbs(c, 7, n))
    lo, rem = intops.split_limbs(T(q, dev).to(torch.int32), 3)    # int32 input, the reference's x.long()
    rlo, rrem = R.split_limbs(q, 3)
    assert eq(rem, rrem) and all(eq(a, b_) for a, b_ in zip(lo, rlo))


def test_exact_primitives(dev):
    from bitexact.exact import ops
    from bitexact.exact.consts import exp2_table
    g = np.random.default_rng(2)
    x = g.integers(-(1 << 61), 1 << 61, 3000) >> g.integers(0, 60, 3000)
    s = g.integers(-70, 70, 3000)
    assert eq(ops.rshc(T(x >> 4, dev), T(s, dev)), R.rshc(x >> 4, s))
    assert eq(ops.rshc(T(x, dev), 17), R.rshc(x, 17))
    assert eq(ops.div_round(T(GOLD["dr_num"], dev), R.FR - R.FV, T(GOLD["dr_den"], dev)), GOLD["dr_o"])
    a = g.integers(-(1 << 61), 1 << 61, 3000)
    r = g.integers(1 << 11, 1 << 34, 3000)
    p = g.integers(-70, 84, 3000)
    assert eq(ops.div_round(T(a, dev), T(p, dev), T(r, dev)), R.div_round(a, p, r))
    Tt = g.integers(-(1 << 58), 1 << 58, 3000)
    d = g.integers(0, 31, 3000)
    B = g.integers(-(1 << 59), 1 << 59, 3000)
    H, L = ops.combine(T(Tt, dev), T(d, dev), T(B, dev))
    rH, rL = R.combine(Tt, d, B)
    assert eq(H, rH) and eq(L, rL)
    pp = g.integers(-90, 31, 3000)
    assert eq(ops.shift_round_hl(H, L, T(pp, dev)), R.shift_round_hl(rH, rL, pp))
    P = g.integers(-(1 << 50), 1 << 50, (6, 300)) >> g.integers(0, 50, (6, 1))
    P[2] = 0
    for eps in (-40, T(g.integers(-50, -30, (6, 1)), dev)):
        q, sh = ops.quant(T(P, dev), eps)
        rq, rsh_ = R.quant(P, eps if isinstance(eps, int) else eps.cpu().numpy())
        assert eq(q, rq) and eq(sh, rsh_)
    P3 = g.integers(-(1 << 50), 1 << 50, (2, 3, 64))
    q, sh = ops.quant(T(P3, dev), -48)
    rq, rsh_ = R.quant(P3, -48)
    assert eq(q, rq) and eq(sh, rsh_) and tuple(sh.shape) == (2, 3)
    lut = exp2_table(dev)
    for D in (512, 2048, 4096):
        rr, er = ops.rms(T(GOLD[f"rms{D}_x"], dev))
        assert eq(rr, GOLD[f"rms{D}_r"]) and eq(er, GOLD[f"rms{D}_er"]), D
    for bits in (22, 30, 40):
        assert eq(ops.exp2neg_lut(T(GOLD["exp2_t"], dev), lut, bits), GOLD[f"exp2_o{bits}"])
    P, eps, ok = ops.silu_mul(T(GOLD["silu_g"], dev), T(GOLD["silu_u"], dev), lut)
    assert eq(P, GOLD["silu_P"]) and eps == -48 and bool(ok) == bool(GOLD["silu_ok"])
    bad = GOLD["silu_g"].copy()
    bad[0, 0] = (1 << 32) + 1
    assert bool(ops.silu_mul(T(bad, dev), T(GOLD["silu_u"], dev), lut)[2]) == bool(GOLD["silu_bad_ok"])
    for hd in (64, 128):
        raw, sh, qpos = GOLD[f"sm{hd}_raw"], GOLD[f"sm{hd}_sh"], GOLD[f"sm{hd}_qpos"]
        okm = T(np.arange(raw.shape[1])[None, :] <= qpos, dev)
        pw, den = ops.softmax_w(T(raw, dev), okm, T(sh, dev), R.FK, lut, R.FP, ops.L2E28_HD[hd])
        assert eq(pw, GOLD[f"sm{hd}_p"]) and eq(den, GOLD[f"sm{hd}_den"]), hd


def test_exact_segs_stages(dev):
    """The module-level stages against the oracle, and each chain against the fused kernel the engine runs."""
    from bitexact.exact import ops, segs
    from bitexact.exact.consts import exp2_table, llama3_inv_freq, rope_tables
    g = np.random.default_rng(3)
    err0 = torch.zeros((), dtype=torch.bool, device=dev)
    for D in (512, 2048):
        x = GOLD[f"rms{D}_x"]
        gm, ge = GOLD[f"nq{D}_gm"], GOLD[f"nq{D}_ge"]
        r, er, err = segs.rms(T(x, dev), err0)
        q, sh = segs.quant(segs.ndiv(T(x, dev), T(gm, dev), T(ge, dev), r, er), -ops.FN)
        assert eq(q, GOLD[f"nq{D}_q"]) and eq(sh, GOLD[f"nq{D}_sh"]) and bool(err) == bool(GOLD[f"nq{D}_err"])
        assert q.dtype == torch.int32
    # RoPE + q_group against the oracle and the fused kernel
    B, Tn, dm = 2, 9, (8, 2, 64)
    h, hkv, hd = dm
    cos, sin = rope_tables(64, 30, llama3_inv_freq(hd))
    cos, sin = T(cos, dev), T(sin, dev)
    y = g.integers(-(1 << 30), 1 << 30, (B * Tn, (h + 2 * hkv) * hd))
    pos = T(g.integers(0, 64, (B, Tn)), dev)
    Pq, k, v, yv = segs.rope_y(T(y, dev), pos, cos, sin, B, Tn, dm)
    rPq, rk, rv = R.rope_y(y, pos.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(), B, Tn, dm)
    assert eq(Pq, rPq) and eq(k, rk) and eq(v, rv)
    qg, shg, err = segs.q_group(Pq, k, v, yv, err0)
    rqg, rshg, rerr = R.q_group(rPq, rk, rv, y)
    assert eq(qg, rqg) and eq(shg, rshg) and bool(err) == rerr
    fqg, fshg, fk, fv, ferr = ops.qkv_y(T(y, dev), pos, cos, sin, B, Tn, dm)
    assert torch.equal(qg, fqg) and torch.equal(shg, fshg) and bool(ferr) == bool(err)
    y2 = y.copy()
    y2[0, 0] = 1 << 32
    assert bool(segs.q_group(*segs.rope_y(T(y2, dev), pos, cos, sin, B, Tn, dm), err0)[2])
    # attn_div + quant = the fused attention output stage
    num = g.integers(-(1 << 55), 1 << 55, (B * hkv, (h // hkv) * Tn, hd))
    den = g.integers(1 << 22, 1 << 34, (B * hkv, (h // hkv) * Tn, 1))
    o = segs.attn_div(T(num, dev), T(den, dev), Tn, hkv)
    assert eq(o, R.attn_div(num, den).reshape(B, hkv, h // hkv, Tn, hd).transpose(0, 3, 1, 2, 4).reshape(B * Tn, -1))
    qo, sho = segs.quant(o, -R.FR)
    fq, fsh = ops.attn_out(T(num, dev), T(den, dev), Tn, hkv)
    assert torch.equal(qo, fq) and torch.equal(sho, fsh)
    # silu_y + quant_silu against the golden stage and the fused kernel
    lut = exp2_table(dev)
    gu = T(np.concatenate([GOLD["silu_g"], GOLD["silu_u"]], 1), dev)
    q, sh, err = segs.quant_silu(*segs.silu_y(gu, lut), err0)
    assert eq(q, GOLD["gus_q"]) and eq(sh, GOLD["gus_sh"]) and bool(err) == bool(GOLD["gus_err"])
    fq, fsh, ferr = ops.gu_silu_y(gu, lut, err0)
    assert torch.equal(q, fq) and torch.equal(sh, fsh)
    # the stage table, eager and compiled (aot_eager: no generated kernels)
    x = T(GOLD["rms2048_x"], dev)
    for comp in (False, True):
        S = segs.Segs(comp)
        assert set(segs.STAGES) <= set(vars(S.s))
        r, er, _ = S.s.rms(x, err0)
        q, sh = S.s.quant(S.s.ndiv(x, T(GOLD["nq2048_gm"], dev), T(GOLD["nq2048_ge"], dev), r, er), -ops.FN)
        assert eq(q, GOLD["nq2048_q"]) and eq(sh, GOLD["nq2048_sh"]), comp


def test_int8_ops(dev):
    from bitexact.int8 import ops
    from bitexact.int8.consts import exp_table, silu_table
    g = np.random.default_rng(4)
    x = GOLD["i8rms_x"]
    r, shx = ops.rms(T(x, dev))
    assert eq(r, GOLD["i8rms_r"]) and eq(shx, GOLD["i8rms_shx"])
    m, e = ops.norm24(T(GOLD["n24_m"], dev), T(GOLD["n24_e"], dev))
    assert eq(m, GOLD["n24_mo"]) and eq(e, GOLD["n24_eo"])
    assert eq(ops.exp_of(T(GOLD["i8eo_z"], dev), exp_table(dev)), GOLD["i8eo_v"])
    assert eq(ops.silu(T(GOLD["i8silu_g"], dev), silu_table(dev)), GOLD["i8silu_v"])
    z = GOLD["qr_z"]
    q, as_, sh = ops.quant_rows(T(z, dev), 2)
    assert eq(q, GOLD["qr_q"]) and eq(as_, GOLD["qr_as"]) and eq(sh, GOLD["qr_sh"])
    # rdiv32 / bitlen32 give rdiv's / bitlen's integers (the reference's tests/test_int8_ops.py:41-63 cases)
    b = g.integers(1 << 29, (1 << 30) + 1, 4000)
    j = g.integers(-32512, 32513, 4000)
    a = j * b - b // 2 + g.integers(-3, 4, 4000)
    assert eq(ops.rdiv32(T(a, dev), T(b, dev)), R.rdiv(a, b))
    xs = np.concatenate([g.integers(0, 1 << 62, 5000) >> g.integers(0, 62, 5000), (1 << np.arange(1, 62)) - 1,
                         1 << np.arange(0, 62)])
    assert eq(ops.bitlen32(T(xs, dev)), R.bitlen(xs))
    # imm: exact q @ W^T through the 3-limb int8 GEMM
    qq = g.integers(-(127 << 16), (127 << 16) + 1, (9, 256))
    W = g.integers(-127, 128, (40, 256))
    assert eq(ops.imm(T(qq, dev), T(W.T.astype(np.float64), dev)), R.imm(qq, W))
    w8 = T(W, dev).to(torch.int8)
    mm = T(g.integers(1, 1 << 20, 40), dev)
    assert ops.post_bound(w8, mm, 30, 2) == (32512 * int((np.abs(W).sum(1) * mm.cpu().numpy()).max()) + (1 << 29)) >> 30


def test_int8_segs_against_golden(dev):
    from bitexact.int8 import segs
    from bitexact.int8.consts import exp_table, silu_table
    x, gamma = T(GOLD["i8rms_x"], dev), T(GOLD["i8pn_gamma"], dev)
    for nl in (1, 2, 3):
        for got, key in zip(segs.pre_norm(x, gamma, nl), ("q", "mant", "e")):
            assert eq(got, GOLD[f"i8pn{nl}_{key}"]), (nl, key)
        for got, key in zip(segs.pre_plain(x, nl), ("q", "mant", "e")):
            assert eq(got, GOLD[f"i8pp{nl}_{key}"]), (nl, key)
    st = silu_table(dev)
    gu = T(GOLD["i8sm_gu"], dev)
    for nl in (1, 2):
        q, mant, e, flag = segs.silu_mul(gu, st, nl)
        assert eq(q, GOLD[f"i8sm{nl}_q"]) and eq(mant, GOLD[f"i8sm{nl}_mant"]) and eq(e, GOLD[f"i8sm{nl}_e"])
        assert bool(flag) == bool(GOLD[f"i8sm{nl}_flag"])
    assert bool(segs.silu_mul(T(GOLD["i8sm_big_gu"], dev), st, 2)[3]) == bool(GOLD["i8sm_big_flag"])
    dm = (8, 2, 16)
    qg, k, v, flag = segs.qkv(T(GOLD["i8qkv_y"], dev), T(GOLD["i8qkv_c"], dev), T(GOLD["i8qkv_s"], dev), dm)
    assert eq(qg, GOLD["i8qkv_qg"]) and eq(k, GOLD["i8qkv_k"]) and eq(v, GOLD["i8qkv_v"])
    assert bool(flag) == bool(GOLD["i8qkv_flag"])
    y2 = GOLD["i8qkv_y"].copy()
    y2[0, 0, 0] = 1 << 40
    assert bool(segs.qkv(T(y2, dev), T(GOLD["i8qkv_c"], dev), T(GOLD["i8qkv_s"], dev), dm)[3])
    for nl in (1, 2):
        for got, key in zip(segs.attn_out(T(GOLD["i8ao_num"], dev), T(GOLD["i8ao_den"], dev), 5, nl, dm),
                            ("q", "mant", "e")):
            assert eq(got, GOLD[f"i8ao{nl}_{key}"]), (nl, key)
    expt = exp_table(dev)
    for hd in (64, 128):
        p, den = segs.softmax(T(GOLD[f"i8sm{hd}_raw"], dev), T(GOLD[f"i8sm{hd}_qpos"], dev), expt, hd)
        assert eq(p, GOLD[f"i8sm{hd}_p"]) and eq(den, GOLD[f"i8sm{hd}_den"]), hd


def test_reference_gpu_kernels_call_pattern(dev):
    """tests/test_gpu_kernels.py:22-37 and 52-61 of the reference, on this package: int8 Segs(2, True, False) and
    Segs(2, True, True) give equal pre_norm and silu_mul outputs (and equal to the oracle); exact Segs(False) and
    Segs(True) give equal pre_norm outputs."""
    from bitexact.exact.segs import Segs as ESegs
    from bitexact.int8 import segs
    g = torch.Generator(device=dev).manual_seed(1)
    eager, comp = segs.Segs(2, True, False), segs.Segs(2, True, True)
    for M in (3, 40):
        x = torch.randint(-(1 << 26), 1 << 26, (M, 2048), device=dev, generator=g)
        x = x >> torch.randint(0, 20, (M, 1), device=dev, generator=g)
        gamma = torch.randint(1, 1 << 13, (2048,), device=dev, generator=g)
        a1, a2 = eager.pre_norm(x, gamma), comp.pre_norm(x, gamma)
        for a, b in zip(a1, a2):
            assert torch.equal(a, b)
        rq, rmant, re_ = R.int8_pre_norm(x.cpu().numpy(), gamma.cpu().numpy(), 2)
        assert eq(a1[0], R.stack_limbs(rq, 2)) and eq(a1[1], rmant) and eq(a1[2], re_)
        gu = torch.randint(-(1 << 22), 1 << 22, (M, 16384), device=dev, generator=g)
        lut = torch.randint(-(1 << 20), 1 << 20, ((64 << 12) + 1,), device=dev, generator=g)
        s1, s2 = eager.silu_mul(gu, lut), comp.silu_mul(gu, lut)
        for a, b in zip(s1, s2):
            assert torch.equal(a, b)
        rq, rmant, re_, rflag = R.int8_silu_mul(gu.cpu().numpy(), lut.cpu().numpy(), 2)
        assert eq(s1[0], R.stack_limbs(rq, 2)) and eq(s1[1], rmant) and eq(s1[2], re_) and bool(s1[3]) == rflag
    e_eager, e_comp = ESegs(False), ESegs(True)
    for M in (1, 37):
        x = torch.randint(-(1 << 30), 1 << 30, (M, 2048), device=dev, generator=g)
        x = x >> torch.randint(0, 24, (M, 1), device=dev, generator=g)
        gm = torch.randint(-255, 256, (2048,), device=dev, generator=g)
        ge = torch.randint(-14, -6, (2048,), device=dev, generator=g)
        for a, b in zip(e_eager.pre_norm(x, gm, ge), e_comp.pre_norm(x, gm, ge)):
            assert torch.equal(a.cpu(), b.cpu())


def test_int8_linear_front_to_back(dev):
    """int8 pre_norm -> int_mm -> post (Segs(nl, True, .): stacked limbs, the int8 MFMA GEMM, join + post) against
    the oracle's pre_norm, imm and post, at config-2 shapes."""
    from bitexact.int8 import segs
    from bitexact.int8.gemm_skinny import int_mm
    g = np.random.default_rng(6)
    for M, N, K in ((1, 8192, 2048), (8, 2048, 8192), (64, 8192, 2048)):
        x = g.integers(-(1 << 28), 1 << 28, (M, K)) >> g.integers(0, 12, (M, 1))
        gamma = g.integers(1, 1 << 13, K)
        W = g.integers(-127, 128, (N, K))
        m = g.integers(1, 1 << 20, N)
        fmsh = 30
        S = segs.Segs(2, True, False)
        a, mant, e = S.pre_norm(T(x, dev), T(gamma, dev))
        c = int_mm(a, T(W, dev).to(torch.int8))
        y, flag = S.post(c, T(m, dev), fmsh, mant, e)
        rq, rmant, re_ = R.int8_pre_norm(x, gamma, 2)
        ry, rflag = R.int8_post(R.imm(rq, W), m, fmsh, rmant, re_)
        assert eq(y, ry) and bool(flag) == rflag, (M, N, K)
