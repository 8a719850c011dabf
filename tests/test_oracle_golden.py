"""The oracle against vectors the reference's own CPU rules produced (tests/golden/make_golden.py):
ops.rms, segs.norm_quant, ops.exp2neg_lut, ops.softmax_w (head_dim 64 and 128), ops.div_round, int8 quant_rows,
int8 segs.softmax (head_dim 64 and 128), ops.silu_mul and the gate/up stage (segs.silu_y + quant_silu); int8 ops.rms,
norm24, exp_of, silu (and its table) and int8 segs.pre_norm, pre_plain, silu_mul, qkv, attn_out."""

import os

import numpy as np
import pytest

from oracle import bxref as R

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))


@pytest.mark.parametrize("D", [512, 2048, 4096])
def test_rms_and_norm_quant(D):
    x = GOLD[f"rms{D}_x"]
    r, er = R.rms(x)
    assert np.array_equal(r, GOLD[f"rms{D}_r"]) and np.array_equal(er, GOLD[f"rms{D}_er"])
    q, sh, err = R.norm_quant(x, GOLD[f"nq{D}_gm"], GOLD[f"nq{D}_ge"])
    assert np.array_equal(q, GOLD[f"nq{D}_q"]) and np.array_equal(sh, GOLD[f"nq{D}_sh"])
    assert err == bool(GOLD[f"nq{D}_err"])


def test_exp2neg_lut():
    lut = R.exp2_table()
    for bits in (22, 30, 40):
        assert np.array_equal(R.exp2neg_lut(GOLD["exp2_t"], lut, bits), GOLD[f"exp2_o{bits}"])


@pytest.mark.parametrize("hd", [64, 128])
def test_softmax_w(hd):
    raw, sh, qpos = GOLD[f"sm{hd}_raw"], GOLD[f"sm{hd}_sh"], GOLD[f"sm{hd}_qpos"]
    ok = np.arange(raw.shape[1])[None, :] <= qpos
    p, den = R.softmax_w(raw, ok, sh, R.FK, R.exp2_table(), R.FP, R.L2E28_HD[hd])
    assert np.array_equal(p, GOLD[f"sm{hd}_p"]) and np.array_equal(den, GOLD[f"sm{hd}_den"])


def test_div_round_attn():
    assert np.array_equal(R.div_round(GOLD["dr_num"], R.FR - R.FV, GOLD["dr_den"]), GOLD["dr_o"])


def test_quant_rows():
    q, as_, sh = R.quant_rows(GOLD["qr_z"], 2)
    assert np.array_equal(q, GOLD["qr_q"]) and np.array_equal(as_, GOLD["qr_as"]) and np.array_equal(sh, GOLD["qr_sh"])


def test_int8_exp_table_and_softmax():
    expt = R.int8_exp_table()
    assert expt.shape == ((1 << 17) + 1,) and expt[-1] == 1 << R.FE8
    import hashlib
    assert hashlib.sha256(expt.astype("<i8").tobytes()).digest() == GOLD["i8_exp_sha256"].tobytes()
    for hd in (64, 128):
        raw, qpos = GOLD[f"i8sm{hd}_raw"], GOLD[f"i8sm{hd}_qpos"]
        ok = np.arange(raw.shape[-1]) <= qpos
        p, den = R.int8_softmax(raw, ok, expt, hd)
        assert np.array_equal(p, GOLD[f"i8sm{hd}_p"]) and np.array_equal(den, GOLD[f"i8sm{hd}_den"])


def test_silu_mul_and_gate_up_stage():
    lut = R.exp2_table()
    P, eps, ok = R.silu_mul(GOLD["silu_g"], GOLD["silu_u"], lut)
    assert np.array_equal(P, GOLD["silu_P"]) and eps == -2 * R.FR and ok == bool(GOLD["silu_ok"])
    bad = GOLD["silu_g"].copy()
    bad[0, 0] = (1 << 32) + 1
    assert R.silu_mul(bad, GOLD["silu_u"], lut)[2] == bool(GOLD["silu_bad_ok"])
    q, sh, err = R.gu_silu_y(np.concatenate([GOLD["silu_g"], GOLD["silu_u"]], 1), lut)
    assert np.array_equal(q, GOLD["gus_q"]) and np.array_equal(sh, GOLD["gus_sh"]) and err == bool(GOLD["gus_err"])


# ---- int8 RMSNorm front and the other int8 segments (src/bitexact/int8/ops.py:70-108, segs.py:47-118) ----
def test_int8_rms_pre_norm_pre_plain():
    x = GOLD["i8rms_x"]
    r, shx = R.int8_rms(x)
    assert np.array_equal(r, GOLD["i8rms_r"]) and np.array_equal(shx, GOLD["i8rms_shx"])
    for nl in (1, 2, 3):
        for got, key in zip(R.int8_pre_norm(x, GOLD["i8pn_gamma"], nl), ("q", "mant", "e")):
            assert np.array_equal(got, GOLD[f"i8pn{nl}_{key}"]), (nl, key)
        for got, key in zip(R.int8_pre_plain(x, nl), ("q", "mant", "e")):
            assert np.array_equal(got, GOLD[f"i8pp{nl}_{key}"]), (nl, key)


def test_int8_norm24_exp_of():
    m, e = R.norm24(GOLD["n24_m"], GOLD["n24_e"])
    assert np.array_equal(m, GOLD["n24_mo"]) and np.array_equal(e, GOLD["n24_eo"])
    assert np.array_equal(R.int8_exp_of(GOLD["i8eo_z"], R.int8_exp_table()), GOLD["i8eo_v"])


def test_int8_silu_table_and_silu():
    import hashlib
    t = R.int8_silu_table()
    assert hashlib.sha256(t.astype("<i8").tobytes()).digest() == GOLD["i8silu_sha256"].tobytes()
    assert np.array_equal(R.int8_silu(GOLD["i8silu_g"], t), GOLD["i8silu_v"])


def test_int8_silu_mul():
    t = R.int8_silu_table()
    for nl in (1, 2):
        q, mant, e, flag = R.int8_silu_mul(GOLD["i8sm_gu"], t, nl)
        assert np.array_equal(q, GOLD[f"i8sm{nl}_q"]) and np.array_equal(mant, GOLD[f"i8sm{nl}_mant"])
        assert np.array_equal(e, GOLD[f"i8sm{nl}_e"]) and flag == bool(GOLD[f"i8sm{nl}_flag"])
    assert R.int8_silu_mul(GOLD["i8sm_big_gu"], t, 2)[3] == bool(GOLD["i8sm_big_flag"])


def test_int8_qkv_attn_out():
    dm = (8, 2, 16)
    qg, k, v, flag = R.int8_qkv(GOLD["i8qkv_y"], GOLD["i8qkv_c"], GOLD["i8qkv_s"], dm)
    assert np.array_equal(qg, GOLD["i8qkv_qg"]) and np.array_equal(k, GOLD["i8qkv_k"])
    assert np.array_equal(v, GOLD["i8qkv_v"]) and flag == bool(GOLD["i8qkv_flag"])
    y2 = GOLD["i8qkv_y"].copy()
    y2[0, 0, 0] = 1 << 40
    assert R.int8_qkv(y2, GOLD["i8qkv_c"], GOLD["i8qkv_s"], dm)[3] == bool(GOLD["i8qkv_big_flag"])
    for nl in (1, 2):
        for got, key in zip(R.int8_attn_out(GOLD["i8ao_num"], GOLD["i8ao_den"], 5, nl, dm), ("q", "mant", "e")):
            assert np.array_equal(got, GOLD[f"i8ao{nl}_{key}"]), (nl, key)
