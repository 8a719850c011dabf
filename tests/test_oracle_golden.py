"""The oracle against vectors the reference's own CPU rules produced (tests/golden/make_golden.py):
ops.rms, segs.norm_quant, ops.exp2neg_lut, ops.softmax_w (head_dim 64 and 128), ops.div_round, int8 quant_rows,
int8 segs.softmax (head_dim 64 and 128), ops.silu_mul and the gate/up stage (segs.silu_y + quant_silu)."""

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
