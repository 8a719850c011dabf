"""HIP attention-side kernels against the CPU oracle, bit for bit: paged exact attention (reference
tests/test_vllm_exact_attn.py: head_dim 64 / 128, three magnitudes, five (R, M, P) cases, four splits),
the paged KV store, the fused prefill attention (exact/model.py's bmm -> softmax -> bmm), and the limb bmm
(reference tests/test_gpu_kernels.py:9-19)."""

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu


def _lut(dev):
    return torch.from_numpy(R.exp2_table()).to(dev)


def test_kv_store_matches_oracle(dev):
    from bitexact.vllm_plugin.tri_paged import store, to_limbs
    g = torch.Generator().manual_seed(0)
    c = torch.randint(-R.LIM3, R.LIM3 + 1, (5, 3, 16, 2 * 64), generator=g).to(torch.int32)
    assert np.array_equal(to_limbs(c.to(dev)).cpu().numpy(), R.to_limbs(c.numpy()))
    # store with skipped slots and int64 input
    cache = torch.zeros(4, 2, 16, 8 * 64, dtype=torch.int8, device=dev)
    k = torch.randint(-R.LIM3, R.LIM3 + 1, (6, 2, 64), generator=g)
    v = torch.randint(-R.LIM3, R.LIM3 + 1, (6, 2, 64), generator=g)
    slot = torch.tensor([0, 17, -1, 33, 63, 5])
    store(cache, slot.to(dev), k.to(dev), v.to(dev))
    ref = np.zeros((4, 2, 16, 8 * 64), np.int8)
    kv = np.concatenate([k.numpy(), v.numpy()], -1)
    lim = R.to_limbs(kv[:, :, None, :].transpose(0, 1, 2, 3).reshape(6, 2, 1, 128))
    for n, s in enumerate(slot.tolist()):
        if s >= 0:
            ref[s // 16, :, s % 16] = lim[n, :, 0]
    assert np.array_equal(cache.cpu().numpy(), ref)


@pytest.mark.parametrize("HD", [64, 128])
def test_exact_paged_attention(dev, HD):
    from bitexact.vllm_plugin import tri_exact_attn, tri_paged
    g = torch.Generator().manual_seed(HD)
    lut = _lut(dev)
    nb, bs, HKV = 96, 16, 8
    l2e = R.L2E28_HD[HD]
    for lim in (R.LIM3, 1 << 13, 1 << 10):
        c = torch.randint(-lim, lim + 1, (nb, HKV, bs, 2 * HD), generator=g).to(torch.int32)
        cl = tri_paged.to_limbs(c.to(dev))
        for Rr, M, P in [(3, 4, 600), (5, 4, 3000), (6, 1, 900), (2, 3, 50), (7, 4, 5)]:
            bt = torch.randint(1, nb, (Rr, 200), generator=g).to(torch.int32)
            qpos = torch.randint(0, P, (Rr, M), generator=g)
            q = torch.randint(-(1 << 22), (1 << 22) + 1, (Rr, HKV, M, HD), generator=g).to(torch.int32)
            sh = torch.randint(-40, -10, (Rr, HKV, M), generator=g)
            rmap = torch.arange(Rr)
            ref_num, ref_den = R.paged_attend(q.numpy(), sh.numpy(), qpos.numpy(), c.numpy(), bt.numpy(),
                                              rmap.numpy(), R.exp2_table(), l2e)
            for ns in (None, 1, 5, 64):
                num, den = tri_exact_attn.attend(q.to(dev), sh.to(dev), qpos.to(dev), cl, bt.to(dev), rmap.to(dev),
                                                 lut, l2e, nsplit=ns)
                assert np.array_equal(num.cpu().numpy(), ref_num), (Rr, M, ns, lim)
                assert np.array_equal(den.cpu().numpy(), ref_den), (Rr, M, ns, lim)


def test_paged_attention_rmap_and_empty_rows(dev):
    """Rows mapped to shared block-table rows, a query with no visible key (qpos -1), repeated calls
    (the split workspace is restored after each call)."""
    from bitexact.vllm_plugin import tri_exact_attn, tri_paged
    g = torch.Generator().manual_seed(7)
    HD, nb, bs, HKV = 64, 20, 16, 2
    c = torch.randint(-R.LIM3, R.LIM3 + 1, (nb, HKV, bs, 2 * HD), generator=g).to(torch.int32)
    cl = tri_paged.to_limbs(c.to(dev))
    bt = torch.randint(0, nb, (2, 8), generator=g).to(torch.int32)
    rmap = torch.tensor([1, 0, 1])
    qpos = torch.tensor([[100, -1, 3, 127], [5, 6, 7, 8], [0, 0, 0, 0]])
    q = torch.randint(-(1 << 22), (1 << 22) + 1, (3, HKV, 4, HD), generator=g).to(torch.int32)
    sh = torch.randint(-40, -10, (3, HKV, 4), generator=g)
    ref = R.paged_attend(q.numpy(), sh.numpy(), qpos.numpy(), c.numpy(), bt.numpy(), rmap.numpy(), R.exp2_table(),
                         R.L2E28)
    for ns in (3, 3, 1, 8):
        num, den = tri_exact_attn.attend(q.to(dev), sh.to(dev), qpos.to(dev), cl, bt.to(dev), rmap.to(dev), _lut(dev),
                                         R.L2E28, nsplit=ns)
        assert np.array_equal(num.cpu().numpy(), ref[0]) and np.array_equal(den.cpu().numpy(), ref[1]), ns


@pytest.mark.parametrize("HD,bs,nblk,M", [(64, 16, 128, 4), (128, 4, 300, 3), (64, 1, 700, 1), (128, 16, 9, 2)])
def test_paged_attention_one_block_per_tile(dev, HD, bs, nblk, M):
    """The unsplit launch for rows of at most 2048 keys (block-table row copied to LDS, scores kept in LDS, K and V
    streamed once through a register ring): cache blocks of 16, 4 and 1 keys, the full 2048-key reach, queries
    past nvalid, a query with no visible key; against the oracle."""
    from bitexact.vllm_plugin import tri_exact_attn, tri_paged
    g = torch.Generator().manual_seed(HD + bs + nblk)
    HKV, Rr = 2, 3
    nb = Rr * nblk + 1
    c = torch.randint(-R.LIM3, R.LIM3 + 1, (nb, HKV, bs, 2 * HD), generator=g).to(torch.int32)
    cl = tri_paged.to_limbs(c.to(dev))
    bt = (1 + torch.randperm(Rr * nblk, generator=g)).to(torch.int32).reshape(Rr, nblk)
    S = nblk * bs
    qpos = torch.randint(0, S, (Rr, M), generator=g)
    qpos[0, 0] = S - 1
    if M > 1:
        qpos[1, 1] = -1
    q = torch.randint(-(1 << 22), (1 << 22) + 1, (Rr, HKV, M, HD), generator=g).to(torch.int32)
    sh = torch.randint(-40, -10, (Rr, HKV, M), generator=g)
    rmap = torch.tensor([2, 0, 1])
    l2e = R.L2E28_HD[HD]
    ref = R.paged_attend(q.numpy(), sh.numpy(), qpos.numpy(), c.numpy(), bt.numpy(), rmap.numpy(), R.exp2_table(),
                         l2e)
    num, den = tri_exact_attn.attend(q.to(dev), sh.to(dev), qpos.to(dev), cl, bt.to(dev), rmap.to(dev), _lut(dev),
                                     l2e, nsplit=1)
    assert np.array_equal(num.cpu().numpy(), ref[0]) and np.array_equal(den.cpu().numpy(), ref[1])


@pytest.mark.parametrize("ticks,ns", [(None, 8), ("0", 8), (None, 4), ("0", 4)])
def test_paged_attention_split_exchange(dev, monkeypatch, ticks, ns):
    """Config 4's decode shape (4 rows x 8 KV heads, 2048 keys, group 4) over 8 or 4 key splits in one launch, where the
    splits of a tile exchange their maxima through the workspace: equal to the unsplit launch and to the oracle on
    a sample of tiles, three calls in a row. ticks "0": no wait for the other splits, each block computes the
    maxima it has not seen from the keys (the path a block takes when its partners are not resident)."""
    from bitexact.vllm_plugin import tri_exact_attn, tri_paged
    if ticks is not None:
        monkeypatch.setenv("BX_ATTN_EXCH_TICKS", ticks)
    g = torch.Generator().manual_seed(11)
    B, HKV, M, HD, S, bs = 4, 8, 4, 64, 2048, 16
    nblk = S // bs
    c = torch.randint(-R.LIM3, R.LIM3 + 1, (B * nblk, HKV, bs, 2 * HD), generator=g).to(torch.int32)
    cl = tri_paged.to_limbs(c.to(dev))
    bt = torch.randperm(B * nblk, generator=g).to(torch.int32).reshape(B, nblk)
    qpos = torch.tensor([[S - 1] * M, [S - 1, 1000, 5, 0], [1500] * M, [2047, 2046, 64, 63]])
    q = torch.randint(-(1 << 22), (1 << 22) + 1, (B, HKV, M, HD), generator=g).to(torch.int32)
    sh = torch.randint(-40, -25, (B, HKV, M), generator=g)
    args = (q.to(dev), sh.to(dev), qpos.to(dev), cl, bt.to(dev), torch.arange(B).to(dev), _lut(dev), R.L2E28)
    assert tri_exact_attn.default_nsplit(B, HKV, nblk, bs) == 8
    n1, d1 = tri_exact_attn.attend(*args, nsplit=1)
    for _ in range(3):
        n8, d8 = tri_exact_attn.attend(*args, nsplit=ns)
        assert torch.equal(n8, n1) and torch.equal(d8, d1)
    rows = [0, 1]
    ref_num, ref_den = R.paged_attend(q[rows].numpy(), sh[rows].numpy(), qpos[rows].numpy(), c.numpy(),
                                      bt[rows].numpy(), np.arange(2), R.exp2_table(), R.L2E28)
    assert np.array_equal(n8[:2].cpu().numpy(), ref_num) and np.array_equal(d8[:2].cpu().numpy(), ref_den)


@pytest.mark.parametrize("HD", [64, 128])
@pytest.mark.parametrize("planes,shr", [(True, (-40, -10)), (False, (-40, -10)), (True, (-9, 7))])
def test_prefill_attention(dev, HD, planes, shr):
    """Both prefill forms (limb planes streamed into LDS; register-staged) against the oracle's unfused
    bmm -> softmax -> bmm, on a strided cache view with two sequence offsets. Query exponents from -9 up give
    negative score shifts for some rows (the limb-plane kernel's general weight path)."""
    from bitexact.exact.attention import prefill
    g = torch.Generator().manual_seed(3 + HD)
    B, HKV, grp, T, L = 2, 2, 4, 70, 96
    Z = B * HKV
    qg = torch.randint(-(1 << 22), (1 << 22) + 1, (Z, grp * T, HD), generator=g).to(torch.int32)
    shg = torch.randint(shr[0], shr[1], (Z, grp * T, 1), generator=g)
    cache_k = torch.randint(-R.LIM3, R.LIM3 + 1, (B, HKV, L, HD), generator=g).to(torch.int32)
    cache_v = torch.randint(-R.LIM3, R.LIM3 + 1, (B, HKV, L, HD), generator=g).to(torch.int32)
    pos = torch.arange(T)[None].expand(B, T) + torch.tensor([[0], [20]])           # two sequences, offsets
    S = int(pos.max()) + 1
    qpos = pos[:, None, None, :].expand(B, HKV, grp, T).reshape(Z, grp * T, 1)
    Kc = cache_k[:, :, :S].reshape(Z, S, HD)
    Vc = cache_v[:, :, :S].reshape(Z, S, HD)
    ref_num, ref_den = R.attention_prefill(qg.numpy(), shg.numpy(), Kc.numpy(), Vc.numpy(), qpos.numpy(),
                                           R.exp2_table(), R.L2E28_HD[HD])
    kd = cache_k.to(dev)[:, :, :S].reshape(Z, S, HD)      # strided view of the cache (row stride L * HD)
    vd = cache_v.to(dev)[:, :, :S].reshape(Z, S, HD)
    num, den = prefill(qg.to(dev), shg.to(dev), kd, vd, qpos.to(dev), _lut(dev), R.L2E28_HD[HD], planes=planes)
    assert np.array_equal(num.cpu().numpy(), ref_num) and np.array_equal(den.cpu().numpy(), ref_den)


@pytest.mark.parametrize("HD,T,Z", [(64, 2048, 4), (128, 640, 2)])
def test_prefill_attention_full_size(dev, HD, T, Z):
    """Config 4's prefill shape (group 4, causal T = 2048) and a head_dim-128 case: the limb-plane form equals the
    register-staged form on every row (two kernels with different tilings and operand orders), every row that
    sees a key has den >= 2^22 (its own maximum's weight is 2^FP), and a sample of rows (first and last of each
    head's block, the partial last tile) equals the oracle."""
    from bitexact.exact.attention import prefill
    g = torch.Generator().manual_seed(HD + T)
    grp = 4
    qg = torch.randint(-(1 << 22), (1 << 22) + 1, (Z, grp * T, HD), generator=g).to(torch.int32)
    shg = torch.randint(-40, -25, (Z, grp * T, 1), generator=g)
    K = torch.randint(-R.LIM3, R.LIM3 + 1, (Z, T, HD), generator=g).to(torch.int32)
    V = torch.randint(-R.LIM3, R.LIM3 + 1, (Z, T, HD), generator=g).to(torch.int32)
    qpos = torch.arange(T).repeat(grp).reshape(1, grp * T, 1).expand(Z, grp * T, 1).contiguous()
    args = (qg.to(dev), shg.to(dev), K.to(dev), V.to(dev), qpos.to(dev), _lut(dev), R.L2E28_HD[HD])
    n1, d1 = prefill(*args, planes=True)
    n2, d2 = prefill(*args, planes=False)
    assert torch.equal(n1, n2) and torch.equal(d1, d2)
    assert bool((d1 >= 1 << 22).all())
    rows = np.unique(np.concatenate([np.arange(0, 40), np.arange(T - 40, T + 40), np.arange(grp * T - 70, grp * T)]))
    z = Z - 1
    ref_num, ref_den = R.attention_prefill(qg[z:z + 1, rows].numpy(), shg[z:z + 1, rows].numpy(), K[z:z + 1].numpy(),
                                           V[z:z + 1].numpy(), qpos[z:z + 1, rows].numpy(), R.exp2_table(),
                                           R.L2E28_HD[HD])
    assert np.array_equal(n1[z, rows].cpu().numpy(), ref_num[0]) and np.array_equal(d1[z, rows].cpu().numpy(),
                                                                                     ref_den[0])


def test_bmm_exact(dev):
    from bitexact.bmm import bmm
    g = torch.Generator().manual_seed(0)
    # (two 64-row tiles per block from M = 128; one k step when K <= 64)
    for Z, M, K, N in [(3, 5, 64, 70), (16, 4, 700, 64), (2, 130, 64, 129), (2, 70, 33, 600), (2, 200, 33, 300),
                       (2, 256, 700, 64)]:
        a = torch.randint(-R.LIM3, R.LIM3 + 1, (Z, M, K), generator=g)
        b = torch.randint(-R.LIM3, R.LIM3 + 1, (Z, K, N), generator=g).to(torch.int32)
        ref = R.bmm(a.numpy(), b.numpy())
        assert np.array_equal(bmm(a.to(dev), b.to(dev)).cpu().numpy(), ref)
        bt = b.to(dev).transpose(1, 2).contiguous().transpose(1, 2)
        assert np.array_equal(bmm(a.to(dev), bt).cpu().numpy(), ref)
    # fewer limbs: values within 1 limb times 3-limb values
    a = torch.randint(-128, 128, (2, 9, 33), generator=g)
    b = torch.randint(-R.LIM3, R.LIM3 + 1, (2, 33, 11), generator=g)
    assert np.array_equal(bmm(a.to(dev), b.to(dev), na=1).cpu().numpy(), R.bmm(a.numpy(), b.numpy()))
    for na, nb in ((1, 2), (2, 3), (3, 1), (2, 2)):
        la, lb = (-128, 127) if na == 1 else (-R.LIM[na], R.LIM[na]), (-128, 127) if nb == 1 else (-R.LIM[nb], R.LIM[nb])
        a = torch.randint(la[0], la[1] + 1, (3, 70 if na != 2 else 150, 150), generator=g)
        b = torch.randint(lb[0], lb[1] + 1, (3, 150, 66), generator=g)
        assert np.array_equal(bmm(a.to(dev), b.to(dev), na=na, nb=nb).cpu().numpy(), R.bmm(a.numpy(), b.numpy()))
    # A transposed in memory (m contiguous), both int32
    a = torch.randint(-R.LIM3, R.LIM3 + 1, (2, 67, 100), generator=g).to(torch.int32)
    b = torch.randint(-R.LIM3, R.LIM3 + 1, (2, 100, 65), generator=g).to(torch.int32)
    at = a.to(dev).transpose(1, 2).contiguous().transpose(1, 2)
    assert np.array_equal(bmm(at, b.to(dev)).cpu().numpy(), R.bmm(a.numpy(), b.numpy()))
    for M, K in ((190, 100), (129, 40)):   # the same over two row tiles per block
        a = torch.randint(-R.LIM3, R.LIM3 + 1, (2, M, K), generator=g).to(torch.int32)
        b = torch.randint(-R.LIM3, R.LIM3 + 1, (2, K, 65), generator=g).to(torch.int32)
        at = a.to(dev).transpose(1, 2).contiguous().transpose(1, 2)
        assert np.array_equal(bmm(at, b.to(dev)).cpu().numpy(), R.bmm(a.numpy(), b.numpy()))


def test_bmm_int32_bound(dev):
    """The int32 limb-weight sums at the reference's bound (K < 43690): every limb -128, the largest K, and a
    mixed-sign case, against Python-int products."""
    from bitexact.bmm import bmm
    K = 43689
    x = -128 - 128 * 256 - 128 * 65536                  # three limbs of -128
    a = torch.full((1, 3, K), x, dtype=torch.long)
    b = torch.full((1, K, 5), x, dtype=torch.int32)
    got = bmm(a.to(dev), b.to(dev)).cpu().numpy()
    assert (got == x * x * K).all()
    b2 = b.clone()
    b2[0, ::2] = R.LIM3                                  # three limbs of 127
    got = bmm(a.to(dev), b2.to(dev)).cpu().numpy()
    assert (got == x * x * (K // 2) + x * R.LIM3 * ((K + 1) // 2)).all()


def test_unfused_equals_fused_attention(dev):
    """GPU bmm -> GPU softmax -> GPU bmm (the reference model's unfused order) against the fused prefill."""
    from bitexact.bmm import bmm
    from bitexact.exact import ops
    from bitexact.exact.attention import prefill
    g = torch.Generator().manual_seed(11)
    Z, gT, S, HD = 4, 96, 96, 64
    qg = torch.randint(-(1 << 22), (1 << 22) + 1, (Z, gT, HD), generator=g).to(torch.int32).to(dev)
    shg = torch.randint(-40, -10, (Z, gT, 1), generator=g).to(dev)
    K = torch.randint(-R.LIM3, R.LIM3 + 1, (Z, S, HD), generator=g).to(torch.int32).to(dev)
    V = torch.randint(-R.LIM3, R.LIM3 + 1, (Z, S, HD), generator=g).to(torch.int32).to(dev)
    qpos = (torch.arange(gT) % 24 * 4).reshape(1, gT, 1).expand(Z, gT, 1).contiguous().to(dev)
    raw = bmm(qg, K.transpose(-1, -2))
    p, den = ops.softmax(raw, qpos, shg, _lut(dev), R.L2E28)
    num = bmm(p, V)
    num2, den2 = prefill(qg, shg, K, V, qpos, _lut(dev), R.L2E28)
    assert torch.equal(num, num2) and torch.equal(den, den2)


@pytest.mark.parametrize("HD", [64, 128])
def test_int8_paged_attention(dev, HD):
    """tri_paged.attend (int8 mode) against the unfused int8 rules; M = 9 spans several 4-query tiles."""
    from bitexact.int8.consts import exp_table
    from bitexact.vllm_plugin import tri_paged
    g = torch.Generator().manual_seed(100 + HD)
    ptab = tri_paged.weight_table(exp_table(dev))
    expt = R.int8_exp_table()
    nb, bs, HKV = 64, 16, 4
    for lim, qlim in ((R.LIM3, 1 << 6), (1 << 13, 1 << 12), (1 << 10, 1 << 16)):
        c = torch.randint(-lim, lim + 1, (nb, HKV, bs, 2 * HD), generator=g).to(torch.int32)
        cl = tri_paged.to_limbs(c.to(dev))
        for Rr, M, P in [(3, 4, 600), (2, 9, 300), (6, 1, 900), (7, 4, 5)]:
            bt = torch.randint(0, nb, (Rr, 64), generator=g).to(torch.int32)
            qpos = torch.randint(0, P, (Rr, M), generator=g)
            qpos[0, 0] = -1
            q = torch.randint(-qlim, qlim + 1, (Rr, HKV, M, HD), generator=g)
            ref_num, ref_den = R.paged_attend_int8(q.numpy(), qpos.numpy(), c.numpy(), bt.numpy(), expt)
            for ns in (None, 1, 5, 64):
                num, den = tri_paged.attend(q.to(dev), qpos.to(dev), cl, bt.to(dev), ptab, nsplit=ns)
                assert np.array_equal(num.cpu().numpy(), ref_num), (Rr, M, ns, lim)
                assert np.array_equal(den.cpu().numpy(), ref_den), (Rr, M, ns, lim)


@pytest.mark.parametrize("HD,H,HKV", [(64, 32, 8), (128, 8, 2), (64, 6, 2)])
def test_rope_attend_equals_store_then_attend(dev, HD, H, HKV):
    """The decode step's fused launch (tri_exact_attn.rope_attend: RoPE, q quantization and the K / V store as the
    attention's prologue) against the two-launch path it replaces (ops.qkv_y with the cache store, then attend
    unsplit): the same num / den, the same cache bytes and the same flag; rope_attend_out (the attention output
    stage fused as well) against ops.attn_out of that num / den, one token per sequence at different
    context lengths, with a padding token (slot -1 keeps the cache unchanged) and the key at the token's own
    position read back from the slot the prologue just wrote."""
    from bitexact.exact import ops
    from bitexact.exact.consts import FT, llama3_inv_freq, rope_tables
    from bitexact.vllm_plugin import tri_exact_attn
    g = torch.Generator().manual_seed(HD + H)
    N, bs, nblk = 6, 16, 20
    cos, sin = rope_tables(400, FT, llama3_inv_freq(HD))
    cos, sin = cos.to(dev), sin.to(dev)
    W = (H + 2 * HKV) * HD
    y = torch.randint(-(1 << 30), 1 << 30, (N, W), generator=g)
    y[1, :HD] >>= 24                                   # a small q head: exponent near NEG_BIG
    pos = torch.tensor([0, 17, 100, 255, 319, 5])
    nb = 1 + N * nblk
    bt = (1 + torch.randperm(N * nblk, generator=g)).to(torch.int32).view(N, nblk)
    rmap = torch.arange(N)
    slot = bt[rmap, pos // bs].long() * bs + pos % bs
    slot[5] = -1                                       # padding: nothing stored
    c0 = torch.randint(-128, 128, (nb, HKV, bs, 8 * HD), dtype=torch.int8, generator=g).to(dev)
    lut = _lut(dev)
    l2e = R.L2E28_HD[HD]
    ca, cb = c0.clone(), c0.clone()
    fa = torch.zeros(1, dtype=torch.int32, device=dev)
    qg, shg, _, _, _ = ops.qkv_y(y.to(dev), pos.view(N, 1).to(dev), cos, sin, N, 1, (H, HKV, HD), flag=fa,
                                 store=(ca, slot.to(dev)))
    G = H // HKV
    qpos = pos.view(-1, 1).expand(-1, G).contiguous().to(dev)
    na, da = tri_exact_attn.attend(qg.view(N, HKV, G, HD), shg.view(N, HKV, G), qpos, ca, bt.to(dev), rmap.to(dev),
                                   lut, l2e, nsplit=1)
    fb = torch.zeros(1, dtype=torch.int32, device=dev)
    nb_, db = tri_exact_attn.rope_attend(y.to(dev), pos.to(dev), cos, sin, (H, HKV, HD), cb, slot.to(dev),
                                         bt.to(dev), rmap.to(dev), lut, l2e, fb)
    torch.cuda.synchronize()
    assert torch.equal(ca, cb), "cache bytes differ"
    assert torch.equal(na, nb_) and torch.equal(da, db)
    assert int(fa.item()) == int(fb.item())
    # with the attention output stage fused too: the rows ops.attn_out makes of the same num / den (twice in a
    # row: the exchange slots are left zero for the next call)
    qo, sho = ops.attn_out(na.view(N * HKV, G, HD), da.view(N * HKV, G, 1), 1, HKV)
    for _ in range(2):
        cc = c0.clone()
        fc = torch.zeros(1, dtype=torch.int32, device=dev)
        qf, shf = tri_exact_attn.rope_attend_out(y.to(dev), pos.to(dev), cos, sin, (H, HKV, HD), cc, slot.to(dev),
                                                 bt.to(dev), rmap.to(dev), lut, l2e, fc)
        torch.cuda.synchronize()
        assert torch.equal(cc, ca), "cache bytes differ (fused output stage)"
        assert torch.equal(qf, qo) and torch.equal(shf, sho)
        assert int(fc.item()) == int(fa.item())
    # the form that also writes q's limb planes (the wo linear's q_planes): the same rows, and the planes are their
    # signed base-256 digits
    cp, fp = c0.clone(), torch.zeros(1, dtype=torch.int32, device=dev)
    qp, shp, plp = tri_exact_attn.rope_attend_out(y.to(dev), pos.to(dev), cos, sin, (H, HKV, HD), cp, slot.to(dev),
                                                  bt.to(dev), rmap.to(dev), lut, l2e, fp, planes=True)
    torch.cuda.synchronize()
    assert torch.equal(cp, ca) and torch.equal(qp, qo) and torch.equal(shp, sho) and int(fp.item()) == int(fa.item())
    r = qp.long()
    for i in range(3):
        lo = ((r + 128) & 255) - 128
        assert torch.equal(plp[i].long(), lo)
        r = (r - lo) >> 8
    # a position past the rope tables flags in both forms
    pos2 = pos.clone()
    pos2[2] = 400
    fa2, fb2 = torch.zeros(1, dtype=torch.int32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev)
    ops.qkv_y(y.to(dev), pos2.view(N, 1).to(dev), cos, sin, N, 1, (H, HKV, HD), flag=fa2, store=(c0.clone(),
                                                                                                     slot.to(dev)))
    tri_exact_attn.rope_attend(y.to(dev), pos2.to(dev), cos, sin, (H, HKV, HD), c0.clone(), slot.to(dev), bt.to(dev),
                               rmap.to(dev), lut, l2e, fb2)
    assert int(fa2.item()) == 1 and int(fb2.item()) == 1
