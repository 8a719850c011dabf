"""HIP row stages against the reference's own vectors (tests/golden/reference_vectors.npz) and the oracle:
RMSNorm + quantization (segs.norm_quant), masked softmax weights (segs.softmax), attention output rule."""

import os

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))


@pytest.mark.parametrize("D", [512, 2048, 4096])
def test_norm_quant_golden(dev, D):
    from bitexact.exact import ops
    x = torch.from_numpy(GOLD[f"rms{D}_x"]).to(dev)
    q, sh, err = ops.norm_quant(x, torch.from_numpy(GOLD[f"nq{D}_gm"]).to(dev), torch.from_numpy(GOLD[f"nq{D}_ge"]).to(dev))
    assert np.array_equal(q.cpu().numpy(), GOLD[f"nq{D}_q"]) and np.array_equal(sh.cpu().numpy(), GOLD[f"nq{D}_sh"])
    assert bool(err) == bool(GOLD[f"nq{D}_err"])


def test_norm_quant_random(dev):
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(2)
    for M in (1, 37):
        x = torch.randint(-(1 << 30), 1 << 30, (M, 2048), generator=g)
        x = x >> torch.randint(0, 24, (M, 1), generator=g)
        gm = torch.randint(-255, 256, (2048,), generator=g)
        ge = torch.randint(-14, -6, (2048,), generator=g)
        q, sh, err = ops.norm_quant(x.to(dev), gm.to(dev), ge.to(dev))
        rq, rsh, rerr = R.norm_quant(x.numpy(), gm.numpy(), ge.numpy())
        assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(sh.cpu().numpy(), rsh) and bool(err) == rerr
    x = torch.zeros(2, 512, dtype=torch.long)
    x[1, 3] = 1 << 41                                          # bound violation sets the flag
    _, _, err = ops.norm_quant(x.to(dev), torch.ones(512, dtype=torch.long, device=dev),
                               torch.full((512,), -7, dtype=torch.long, device=dev))
    assert bool(err)


@pytest.mark.parametrize("hd", [64, 128])
def test_softmax_golden(dev, hd):
    from bitexact.exact import ops
    raw = torch.from_numpy(GOLD[f"sm{hd}_raw"]).to(dev)
    qpos = torch.from_numpy(GOLD[f"sm{hd}_qpos"]).to(dev)
    sh = torch.from_numpy(GOLD[f"sm{hd}_sh"]).to(dev)
    lut = torch.from_numpy(R.exp2_table()).to(dev)
    p, den = ops.softmax(raw, qpos, sh, lut, R.L2E28_HD[hd])
    assert np.array_equal(p.cpu().numpy().astype(np.int64), GOLD[f"sm{hd}_p"])
    assert np.array_equal(den.cpu().numpy(), GOLD[f"sm{hd}_den"])


def test_attn_out(dev):
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(5)
    B, HKV, grp, T, HD = 2, 8, 4, 9, 64
    Z = B * HKV
    num = torch.randint(-(1 << 60), 1 << 60, (Z, grp * T, HD), generator=g)
    den = torch.randint(1 << 22, 1 << 34, (Z, grp * T, 1), generator=g)
    q, sh = ops.attn_out(num.to(dev), den.to(dev), T, HKV)
    o = R.attn_div(num.numpy(), den.numpy())
    o = o.reshape(B, HKV, grp, T, HD).transpose(0, 3, 1, 2, 4).reshape(B * T, HKV * grp * HD)
    rq, rsh = R.quant(o, -R.FR)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(sh.cpu().numpy(), rsh)
