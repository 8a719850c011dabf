"""HIP element-wise segments against the CPU oracle, bit for bit: exact-mode RoPE + q quantization + regroup
(segs.rope_y + segs.q_group), int8-mode row quantization with stacked limbs (ops.quant_rows + stack_limbs,
segs.pre_plain's row scale) and the int8 linear post-segment (segs.post)."""

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu


def _tables(n_pos, hd):
    return R.rope_tables(n_pos, R.FT_ROPE, R.llama3_inv_freq(hd))


@pytest.mark.parametrize("HD,H,HKV,B,T", [(64, 8, 2, 2, 5), (128, 4, 2, 3, 7), (64, 32, 8, 2, 256)])
def test_rope_qgroup(dev, HD, H, HKV, B, T):
    from bitexact.exact import ops
    g = torch.Generator().manual_seed(HD + T)
    cos, sin = _tables(300, HD)
    W = (H + 2 * HKV) * HD
    y = torch.randint(-(1 << 30), 1 << 30, (B * T, W), generator=g)
    y[:, :HD] >>= 20                                   # small and zero rows: exponents near NEG_BIG
    y[0, :HD] = 0
    pos = torch.randint(0, 300, (B, T), generator=g)
    Pq, k, v = R.rope_y(y.numpy(), pos.numpy(), cos, sin, B, T, (H, HKV, HD))
    qg, shg, err = R.q_group(Pq, k, v, y.numpy())
    out = ops.qkv_y(y.to(dev), pos.to(dev), torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev), B, T,
                    (H, HKV, HD))
    assert np.array_equal(out[0].cpu().numpy(), qg) and np.array_equal(out[1].cpu().numpy(), shg)
    assert np.array_equal(out[2].cpu().numpy(), k) and np.array_equal(out[3].cpu().numpy(), v)
    assert bool(out[4]) == err


def test_rope_qgroup_flags(dev):
    from bitexact.exact import ops
    HD, H, HKV, B, T = 64, 4, 2, 1, 3
    cos, sin = _tables(16, HD)
    c, s = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    y = torch.zeros(B * T, (H + 2 * HKV) * HD, dtype=torch.long)
    pos = torch.tensor([[0, 1, 2]])
    assert not bool(ops.qkv_y(y.to(dev), pos.to(dev), c, s, B, T, (H, HKV, HD))[4])
    y2 = y.clone()
    y2[1, 5] = 1 << 31                                  # |y| >= 2^31
    assert bool(ops.qkv_y(y2.to(dev), pos.to(dev), c, s, B, T, (H, HKV, HD))[4])
    y3 = y.clone()
    y3[2, (H + HKV) * HD + 3] = (R.LIM3 + 1) << (R.FR - R.FV)   # |v| > LIM3
    assert bool(ops.qkv_y(y3.to(dev), pos.to(dev), c, s, B, T, (H, HKV, HD))[4])
    # a position past the tables: the reference's index fails; flagged here
    assert bool(ops.qkv_y(y.to(dev), torch.tensor([[0, 1, 16]]).to(dev), c, s, B, T, (H, HKV, HD))[4])


@pytest.mark.parametrize("nl", [1, 2, 3])
def test_int8_quant_rows(dev, nl):
    from bitexact.int8 import segs
    g = torch.Generator().manual_seed(nl)
    for M, K in [(1, 2048), (7, 512), (64, 8192), (3, 16)]:
        z = torch.randint(-(1 << 40), 1 << 40, (M, K), generator=g)
        z = z >> torch.randint(0, 40, (M, 1), generator=g)
        z[0, :] = 0                                      # amax clamps to 1
        a, as_, sh = segs.quant_rows_limbs(z.to(dev), nl)
        rq, ras, rsh_ = R.quant_rows(z.numpy(), nl)
        assert np.array_equal(a.cpu().numpy(), R.stack_limbs(rq, nl)[:nl * M].astype(np.int8))
        assert np.array_equal(as_.cpu().numpy(), ras) and np.array_equal(sh.cpu().numpy(), rsh_)
        a2, mant, e = segs.pre_plain_limbs(z.to(dev), nl)
        rm, re = R.norm24(ras, rsh_ - R.FR8)
        assert torch.equal(a, a2)
        assert np.array_equal(mant.cpu().numpy(), rm) and np.array_equal(e.cpu().numpy(), re)


def test_int8_post(dev):
    from bitexact.int8 import segs
    g = torch.Generator().manual_seed(9)
    M, N = 9, 3000
    acc = torch.randint(-(1 << 38), 1 << 38, (M, N), generator=g)
    m = torch.randint(-(1 << 20), 1 << 20, (N,), generator=g)
    mant = torch.randint(1 << 23, (1 << 24) + 1, (M,), generator=g)
    e = torch.randint(-40, -10, (M,), generator=g)
    for fmsh in (30, 45):
        y, flag = segs.post(acc.to(dev), m.to(dev), fmsh, mant.to(dev), e.to(dev))
        ry, rflag = R.int8_post(acc.numpy(), m.numpy(), fmsh, mant.numpy(), e.numpy())
        assert np.array_equal(y.cpu().numpy(), ry) and bool(flag) == rflag


@pytest.mark.parametrize("HD,H,HKV,B,T,bs", [(64, 8, 2, 2, 5, 16), (128, 4, 2, 3, 7, 4), (64, 32, 8, 32, 1, 16)])
def test_rope_qgroup_store(dev, HD, H, HKV, B, T, bs):
    """The fused rope + cache store (exact_fuse.qkv with STORE) writes the same cache bytes as the separate
    rope + tri_paged.store, skips slot < 0 and leaves every other cache byte as it was."""
    from bitexact.exact import ops
    from bitexact.vllm_plugin import tri_paged
    g = torch.Generator().manual_seed(HD * T + B)
    cos, sin = _tables(300, HD)
    c, s = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    y = torch.randint(-(1 << 30), 1 << 30, (B * T, (H + 2 * HKV) * HD), generator=g).to(dev)
    pos = torch.randint(0, 300, (B, T), generator=g).to(dev)
    nb = (B * T + bs - 1) // bs + 2
    slot = torch.randperm(nb * bs, generator=g)[:B * T]
    slot[1] = -1
    slot = slot.to(dev)
    c0 = torch.randint(-128, 128, (nb, HKV, bs, 8 * HD), generator=g, dtype=torch.int8).to(dev)
    qg, shg, k, v, err = ops.qkv_y(y, pos, c, s, B, T, (H, HKV, HD))
    ref = c0.clone()
    tri_paged.store(ref, slot, k.view(B * T, HKV, HD), v.view(B * T, HKV, HD))
    got = c0.clone()
    qg2, shg2, k2, v2, err2 = ops.qkv_y(y, pos, c, s, B, T, (H, HKV, HD), store=(got, slot))
    assert k2 is None and v2 is None
    assert torch.equal(qg, qg2) and torch.equal(shg, shg2) and bool(err) == bool(err2)
    assert torch.equal(got, ref)
