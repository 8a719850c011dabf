"""HIP stages between the exact decoder's GEMMs against the CPU oracle and the reference's golden vectors, bit
for bit: the residual add + RMSNorm + quantization (Segs.add_norm_y), the embedding gather + pre_norm, and the
SiLU gating + quantization (Segs.gu_silu_y)."""

import os

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))


def _gamma(g, D):
    return torch.randint(-255, 256, (D,), generator=g), torch.randint(-14, -6, (D,), generator=g)


@pytest.mark.parametrize("M,D", [(1, 2048), (5, 512), (32, 2048), (3, 4096)])
def test_add_norm(dev, M, D):
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(M * D)
    x = torch.randint(-(1 << 33), 1 << 33, (M, D), generator=g)
    y = torch.randint(-(1 << 32), 1 << 32, (M, D), generator=g)
    x[0] >>= 14
    gm, ge = _gamma(g, D)
    xs, q, sh, flag = R.add_norm_y(y.numpy(), x.numpy(), gm.numpy(), ge.numpy())
    xd = x.to(dev)
    xo, qd, shd, err = ops.add_norm_y(y.to(dev), xd, gm.to(dev), ge.to(dev))
    assert xo.data_ptr() == xd.data_ptr()                 # in place
    assert np.array_equal(xo.cpu().numpy(), xs)
    assert np.array_equal(qd.cpu().numpy(), q) and np.array_equal(shd.cpu().numpy(), sh)
    assert bool(err) == flag
    # the add alone, and the bound flag on it
    xd = x.to(dev)
    xo, qn, shn, err = ops.add_norm_y(y.to(dev), xd, None, None)
    assert qn is None and np.array_equal(xo.cpu().numpy(), xs) and not bool(err)
    big = torch.zeros(M, D, dtype=torch.long)
    big[-1, -1] = 1 << 40
    assert bool(ops.add_norm_y(big.to(dev), torch.zeros(M, D, dtype=torch.long, device=dev), None, None)[3])


@pytest.mark.parametrize("M,D", [(1, 512), (7, 2048), (32, 2048), (129, 2048), (20, 4096)])
def test_add_norm_rows_planes(dev, M, D):
    """add + norm with limb planes, then norm_quant of the new x: q, sh, planes, the new x and the flag, two calls
    in a row, the second with a row over the bound."""
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(M + D)
    gm, ge = _gamma(g, D)
    for call in range(2):
        x = torch.randint(-(1 << 33), 1 << 33, (M, D), generator=g)
        y = torch.randint(-(1 << 32), 1 << 32, (M, D), generator=g)
        x[0] >>= 20 + call
        if call == 1:
            x[-1, 5] = 1 << 41
        xs, q, sh, flag = R.add_norm_y(y.numpy(), x.numpy(), gm.numpy(), ge.numpy())
        xd = x.to(dev)
        xo, (qd, pl), shd, err = ops.add_norm_y(y.to(dev), xd, gm.to(dev), ge.to(dev), planes=True)
        assert np.array_equal(xo.cpu().numpy(), xs), call
        assert np.array_equal(qd.cpu().numpy(), q) and np.array_equal(shd.cpu().numpy(), sh), call
        assert np.array_equal(pl.cpu().numpy(), np.stack([lo.astype(np.int8) for lo in R.split_limbs(q, 3)[0]])), call
        assert bool(err) == flag == (call == 1)
        q2, sh2, _ = ops.norm_quant(xd, gm.to(dev), ge.to(dev))
        rq, rsh, _ = R.norm_quant(xs, gm.numpy(), ge.numpy())
        assert np.array_equal(q2.cpu().numpy(), rq) and np.array_equal(sh2.cpu().numpy(), rsh), call


def test_add_norm_golden(dev):
    """norm_quant of the reference's golden rows, reached as 0 + x."""
    from bitexact.exact import ops
    for D in (512, 2048, 4096):
        x = torch.from_numpy(GOLD[f"rms{D}_x"])
        gm, ge = torch.from_numpy(GOLD[f"nq{D}_gm"]), torch.from_numpy(GOLD[f"nq{D}_ge"])
        _, q, sh, err = ops.add_norm_y(x.to(dev), torch.zeros_like(x).to(dev), gm.to(dev), ge.to(dev))
        assert np.array_equal(q.cpu().numpy(), GOLD[f"nq{D}_q"]) and np.array_equal(sh.cpu().numpy(), GOLD[f"nq{D}_sh"])
        assert bool(err) == bool(GOLD[f"nq{D}_err"])


@pytest.mark.parametrize("V,D,M", [(1000, 2048, 9), (50, 512, 64)])
def test_embed_norm(dev, V, D, M):
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(V + M)
    emb = torch.randint(-(1 << 24), 1 << 24, (V, D), generator=g, dtype=torch.int32)
    ids = torch.randint(0, V, (M,), generator=g)
    ids[0] = V - 1
    gm, ge = _gamma(g, D)
    x_ref = emb.numpy()[ids.numpy()].astype(np.int64)
    q, sh, flag = R.norm_quant(x_ref, gm.numpy(), ge.numpy())
    x, qd, shd, err = ops.embed_norm(emb.to(dev), ids.to(dev), gm.to(dev), ge.to(dev))
    assert np.array_equal(x.cpu().numpy(), x_ref)
    assert np.array_equal(qd.cpu().numpy(), q) and np.array_equal(shd.cpu().numpy(), sh) and bool(err) == flag


def test_gu_silu_golden(dev):
    from bitexact.exact import ops
    lut = torch.from_numpy(R.exp2_table()).to(dev)
    gu = torch.from_numpy(np.concatenate([GOLD["silu_g"], GOLD["silu_u"]], 1)).to(dev)
    q, sh, err = ops.gu_silu_y(gu, lut)
    assert np.array_equal(q.cpu().numpy(), GOLD["gus_q"]) and np.array_equal(sh.cpu().numpy(), GOLD["gus_sh"])
    assert bool(err) == bool(GOLD["gus_err"])


@pytest.mark.parametrize("M,ff", [(1, 8192), (32, 8192), (7, 96)])
def test_gu_silu(dev, M, ff):
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(M + ff)
    gu = torch.randint(-(1 << 31), 1 << 31, (M, 2 * ff), generator=g)
    gu[0, :ff] >>= 10
    gu[-1, :ff] = 0                                     # a zero row: sh = NEG_BIG
    lut = R.exp2_table()
    q, sh, flag = R.gu_silu_y(gu.numpy(), lut)
    qd, shd, err = ops.gu_silu_y(gu.to(dev), torch.from_numpy(lut).to(dev))
    assert np.array_equal(qd.cpu().numpy(), q) and np.array_equal(shd.cpu().numpy(), sh) and bool(err) == flag
    bad = gu.clone()
    bad[0, 1] = (1 << 32) + 1                           # |g| > 2^32
    assert bool(ops.gu_silu_y(bad.to(dev), torch.from_numpy(lut).to(dev))[2]) and R.gu_silu_y(bad.numpy(), lut)[2]
    bad = gu.clone()
    bad[0, 0], bad[0, ff] = 1 << 32, 1 << 31           # bitlen(s) + bitlen(u) > 62
    assert bool(ops.gu_silu_y(bad.to(dev), torch.from_numpy(lut).to(dev))[2]) and R.gu_silu_y(bad.numpy(), lut)[2]


@pytest.mark.parametrize("M,ff", [(1, 8192), (32, 8192), (7, 96), (5, 3000), (130, 2048)])
def test_gu_silu_split(dev, M, ff):
    """The column-chunked SiLU stage (few rows) against the oracle and the row-per-block kernel: q, sh and the flag,
    with ragged chunks (ff = 3000), a zero row and an overflowing element."""
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(3 * M + ff)
    gu = torch.randint(-(1 << 31), 1 << 31, (M, 2 * ff), generator=g)
    gu[0, :ff] >>= 12
    gu[-1, :ff] = 0
    lut = R.exp2_table()
    q, sh, flag = R.gu_silu_y(gu.numpy(), lut)
    L = torch.from_numpy(lut).to(dev)
    qa, sha, ea = ops.gu_silu_y(gu.to(dev), L, split=True)
    qb, shb, eb = ops.gu_silu_y(gu.to(dev), L, split=False)
    assert np.array_equal(qa.cpu().numpy(), q) and np.array_equal(sha.cpu().numpy(), sh) and bool(ea) == flag
    assert torch.equal(qa, qb) and torch.equal(sha, shb) and bool(ea) == bool(eb)
    bad = gu.clone()
    bad[M // 2, ff - 1] = (1 << 32) + 1
    assert bool(ops.gu_silu_y(bad.to(dev), L, split=True)[2]) and R.gu_silu_y(bad.numpy(), lut)[2]


@pytest.mark.parametrize("ticks", ["0", "1"])
def test_gu_silu_split_exchange_fallback(dev, monkeypatch, ticks):
    """The column chunks of a row exchange their maxima with a bounded wait; with the wait cut to 0 / 1 tick
    (forced from the host), blocks that have not seen every chunk form the row maximum from gu themselves: same
    q, sh and flag, on three calls in a row (the workspace's slots and counters are left zeroed)."""
    from bitexact.exact import ops
    M, ff = 32, 8192
    g = torch.Generator().manual_seed(11)
    gu = torch.randint(-(1 << 31), 1 << 31, (M, 2 * ff), generator=g)
    gu[1, :ff] >>= 12
    lut = R.exp2_table()
    q, sh, flag = R.gu_silu_y(gu.numpy(), lut)
    L = torch.from_numpy(lut).to(dev)
    monkeypatch.setenv("BX_SILU_TICKS", ticks)
    for _ in range(3):
        qa, sha, ea = ops.gu_silu_y(gu.to(dev), L, split=True)
        assert np.array_equal(qa.cpu().numpy(), q) and np.array_equal(sha.cpu().numpy(), sh) and bool(ea) == flag
    monkeypatch.delenv("BX_SILU_TICKS")
    qa, sha, _ = ops.gu_silu_y(gu.to(dev), L, split=True)
    assert np.array_equal(qa.cpu().numpy(), q) and np.array_equal(sha.cpu().numpy(), sh)


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("M,N", [(1, 128256), (5, 1000), (3, 7), (32, 128256), (4, 40000)])
def test_first_argmax(dev, M, N, split):
    """First index of the row maximum, ties included; a row of int64 minima gives 0."""
    from bitexact.intops import first_argmax
    g = torch.Generator().manual_seed(N)
    v = torch.randint(-(1 << 40), 1 << 40, (M, N), generator=g)
    v[0, N // 3] = v[0, N - 1] = v[0, N // 2] = 1 << 50          # ties: the first one wins
    if M > 1:
        v[1] = -(1 << 63)
    if M > 2:
        v[2] = 5
    if M > 3 and N > 9000:                                        # ties across chunk edges (8016 / 8192 wide)
        v[3, 9000] = v[3, 8000] = v[3, N - 1] = 1 << 51
    want = [R.first_argmax(r) for r in v.numpy()]
    assert first_argmax(v.to(dev), split=split).cpu().tolist() == want
    assert want[0] == N // 3 and (M < 2 or want[1] == 0) and (M < 3 or want[2] == 0)
