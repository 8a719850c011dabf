"""HIP exact / int8 linear kernels against the CPU oracle, bit for bit (reference tests/test_exact_ops.py:137-152,
tests/test_gemm_skinny.py, tests/test_vllm_exact_gemm.py: shapes, row counts, extremes, magnitude ranges)."""

import ctypes
import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu


def _bf16(N, K, seed, force=True):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    if force:
        w[0, :5] = torch.tensor([1e-9, -3e-8, 0.0, 2.0, -0.5]).to(torch.bfloat16)
        w[min(3, N - 1), K - 3:] = torch.tensor([3e-7, -1e-6, 1e-10]).to(torch.bfloat16)
    return w


def _dec(w):
    return R.decompose(w.view(torch.int16).numpy())


def _ell(dec, N, dev):
    cnt, ec, ev, Rr = R.to_ell(dec["rr"], dec["rc"], dec["rv"], N)
    return (torch.from_numpy(cnt).to(torch.int32).to(dev), torch.from_numpy(ec).to(torch.int32).to(dev),
            torch.from_numpy(ev).to(dev), Rr)


def test_decompose_matches_oracle(dev):
    from bitexact.exact.consts import decompose
    for N, K, seed in [(48, 256, 2), (3072, 2048, 5), (7, 64, 9)]:
        w = _bf16(N, K, seed)
        ref = _dec(w)
        got = decompose(w.to(dev))
        assert np.array_equal(got["limbs"].cpu().numpy(), ref["limbs"])
        assert np.array_equal(got["g"].cpu().numpy(), ref["g"]) and np.array_equal(got["d"].cpu().numpy(), ref["d"])
        assert np.array_equal(got["rr"].cpu().numpy(), ref["rr"])
        assert np.array_equal(got["rc"].cpu().numpy(), ref["rc"])
        assert np.array_equal(got["rv"].cpu().numpy(), ref["rv"])
    # an all-zero row and a row of tiny values (residual grid at its limit)
    w = torch.zeros(4, 128, dtype=torch.bfloat16)
    w[1, 0], w[1, 5] = 1.0, 2.0 ** -20
    w[2] = (torch.randn(128) * 1e-30).to(torch.bfloat16)
    ref = _dec(w)
    got = decompose(w.to(dev))
    for k in ("g", "d", "rr", "rc", "rv"):
        assert np.array_equal(got[k].cpu().numpy(), ref[k]), k


@pytest.mark.parametrize("M,N,K", [(1, 256, 2048), (7, 3072, 2048), (37, 512, 8192), (300, 1024, 2048), (2048, 512, 2048),
                                   (21, 200, 320), (22, 130, 64), (32, 16384, 256), (32, 2048, 8192)])
def test_wmm_exact_extremes(dev, M, N, K):
    from bitexact.exact.wmm import wmm_hip
    g = np.random.default_rng(M * 1000 + N)
    q = g.integers(-(1 << 22), (1 << 22) + 1, (M, K))
    q[0, :] = 1 << 22
    if M > 1:
        q[1, :] = -(1 << 22)
    W = g.integers(-R.LIM3, R.LIM3 + 1, (N, K))
    W[0, :] = R.LIM3
    W[-1, :] = -R.LIM3
    L = np.stack([x.astype(np.int8) for x in R.split_limbs(W, 3)[0]])
    ref = R.wmm_f64(q, W)
    T = wmm_hip(torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(L).to(dev))
    assert T.shape == (1, M, N)
    assert np.array_equal(T[0].cpu().numpy(), ref)


@pytest.mark.parametrize("M", [1, 3, 8, 9, 16, 17, 21, 22, 33, 64, 65, 100, 129, 200])
def test_exact_linear_matches_oracle(dev, M):
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    N, K = 160, 512
    w = _bf16(N, K, 11)
    dec = _dec(w)
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    assert Rr > 0
    g = np.random.default_rng(M)
    for lim, shr in ((1 << 22, (-30, -20)), (1 << 12, (-45, -8)), (3, (-70, 10))):
        q = g.integers(-lim, lim + 1, (M, K))
        sh = g.integers(shr[0], shr[1], M)
        ref, rflag, _ = R.epilogue(R.wmm_f64(q, dec["W"]), R.residual(q, dec["rr"], dec["rc"], dec["rv"], N),
                                   dec["d"], dec["g"], sh, R.FR, True)
        flag = torch.zeros(1, dtype=torch.int32, device=dev)
        y = exact_linear(torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(sh).to(dev), limbs, d, gg,
                         cnt, ec, ev, Rr, flag, True)
        assert np.array_equal(y.cpu().numpy(), ref), (M, lim)
        assert bool(flag.item()) == rflag, (M, lim)


@pytest.mark.parametrize("M,N,K,kern", [(22, 16384, 512, "stream"), (32, 16400, 512, "stream"),
                                        (42, 16384, 512, "stream"), (17, 16384, 512, "stream"),
                                        (33, 16384, 256, "stream"), (32, 8192, 512, "wide"), (32, 2048, 512, "gemv"),
                                        (27, 3000, 512, "gemv"), (32, 2048, 8192, "stream"),
                                        (40, 4096, 8192, "stream"), (32, 3072, 2048, "gemv")])
def test_exact_linear_wide_rows(dev, M, N, K, kern):
    """49..128 limb rows (17 <= M <= 42): the stream kernel where its 64-column tiles cover the chip (N = 16400
    leaves a partial column tile; 51, 66, 96, 99, 126 limb rows) or K splits into >= 1024-k parts (N = 2048 / 4096,
    K = 8192: the zeroed workspace and the tile's last block), the wide kernel at N = 8192 with K = 512, the gemv's
    row parts otherwise (N = 3000 leaves a partial column tile)."""
    from bitexact.vllm_plugin.exact_gemm import exact_linear, plan
    assert plan(M, N, K)[0] == kern, plan(M, N, K)
    w = _bf16(N, K, 5)
    dec = _dec(w)
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    g = np.random.default_rng(M + N)
    for lim, shr in ((1 << 22, (-30, -20)), (3, (-70, 10))):
        q = g.integers(-lim, lim + 1, (M, K))
        sh = g.integers(shr[0], shr[1], M)
        ref, rflag, _ = R.epilogue(R.wmm_f64(q, dec["W"]), R.residual(q, dec["rr"], dec["rc"], dec["rv"], N),
                                   dec["d"], dec["g"], sh, R.FR, True)
        flag = torch.zeros(1, dtype=torch.int32, device=dev)
        y = exact_linear(torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(sh).to(dev), limbs, d, gg,
                         cnt, ec, ev, Rr, flag, True)
        assert np.array_equal(y.cpu().numpy(), ref), (M, N, lim)
        assert bool(flag.item()) == rflag, (M, N, lim)


def test_exact_linear_flag_cases(dev):
    """The checked epilogue's loss / range flag, per element (reference tests/test_model_bounds.py)."""
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    N, K = 64, 64
    W = np.zeros((N, K), np.int64)
    W[:, 0] = 1
    L = torch.from_numpy(np.stack([x.astype(np.int8) for x in R.split_limbs(W, 3)[0]])).to(dev)
    zeros = torch.zeros(N, dtype=torch.long, device=dev)
    for value, shift in [(1 << 21, 22), (-(1 << 21), 22), (1 << 20, 30), (5, 31), (-5, 31), (1 << 21, -90),
                         (12345, -33), (1, 0)]:
        q = np.zeros((1, K), np.int64)
        q[0, 0] = value
        ref, rflag, _ = R.epilogue(R.wmm_f64(q, W), np.zeros((1, N), np.int64), np.zeros(N, np.int64),
                                   np.zeros(N, np.int64), np.array([shift - R.FR]), R.FR, True)
        flag = torch.zeros(1, dtype=torch.int32, device=dev)
        y = exact_linear(torch.from_numpy(q).to(torch.int32).to(dev), torch.tensor([shift - R.FR], device=dev), L,
                         zeros, zeros, None, None, None, 0, flag, True)
        assert np.array_equal(y.cpu().numpy(), ref), (value, shift)
        assert bool(flag.item()) == rflag, (value, shift)


def test_config1_exact_linear(dev):
    """Config 1: M=8, K=N=2048, bf16 N(0, 0.02) weights with forced residuals, FN=40 activations."""
    from bitexact.exact.consts import decompose
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    M, N, K = 8, 2048, 2048
    w = _bf16(N, K, 1)
    dec = _dec(w)
    gd = decompose(w.to(dev))
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    P = torch.floor(x * 2.0 ** 40 + 0.5).long().numpy()
    q, sh = R.quant(P, -40)
    ref, rflag = R.exact_linear(q, dec, sh)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    y = exact_linear(torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(sh).to(dev), gd["limbs"], gd["d"],
                     gd["g"], gd["ell_cnt"], gd["ell_col"], gd["ell_val"], gd["R"], flag, True)
    assert np.array_equal(y.cpu().numpy(), ref) and bool(flag.item()) == rflag


@pytest.mark.parametrize("N,K", [(3072, 2048), (2048, 2048), (2048, 8192), (8192, 2048), (512, 256)])
def test_int_mm_rows(dev, N, K):
    from bitexact.int8.gemm_skinny import int_mm
    g = torch.Generator().manual_seed(N + K)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    for Rr in (2, 16, 24, 56, 64, 72, 128, 200, 264):
        for kind in ("rand", "max", "min"):
            a = torch.randint(-128, 128, (Rr, K), dtype=torch.int8, generator=g)
            w2 = w
            if kind == "max":
                a.fill_(-128)
                w2 = torch.full_like(w, -128)
            elif kind == "min":
                a.fill_(127)
                w2 = torch.full_like(w, -128)
            ref = R.imm(a.numpy(), w2.numpy())
            c = int_mm(a.to(dev), w2.to(dev))
            assert c.dtype == torch.int32 and np.array_equal(c.cpu().numpy().astype(np.int64), ref), (N, K, Rr, kind)


@pytest.mark.parametrize("M", [1, 8, 64, 100])
@pytest.mark.parametrize("nl", [1, 2, 3])
def test_int_mm_join(dev, M, nl):
    from bitexact.int8.gemm_skinny import int_mm_join
    N, K = 1024, 2048
    g = np.random.default_rng(M * 10 + nl)
    z = g.integers(-(1 << 44), 1 << 44, (M, K))
    q, _, _ = R.quant_rows(z, nl)
    a = R.stack_limbs(q, nl)
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    ref = R.imm(q, w)
    y = int_mm_join(torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev), M, nl)
    assert np.array_equal(y.cpu().numpy(), ref)


@pytest.mark.parametrize("M", [1, 4, 8, 33, 64])
@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192), (16384, 2048)])
def test_config2_int8_decode(dev, M, N, K):
    """Config 2 shapes at full size: int8 uniform weights, N(0,1) activations in 2 limbs."""
    from bitexact.int8.gemm_skinny import int_mm_join
    g = torch.Generator().manual_seed(7)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    z = torch.floor(x * 2.0 ** 16 + 0.5).long().numpy()
    q, _, _ = R.quant_rows(z, 2)
    a = R.stack_limbs(q, 2)
    y = int_mm_join(torch.from_numpy(a).to(dev), w.to(dev), M, 2)
    assert np.array_equal(y.cpu().numpy(), R.imm(q, w.numpy()))


def test_standalone_epilogue_and_lin_y(dev):
    """wmm.epilogue / segs.lin_y on the device: dense residual and ELL forms, split partials, the checked flag."""
    from bitexact.exact import wmm
    N, K, M = 160, 512, 37
    w = _bf16(N, K, 23)
    dec = _dec(w)
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    _, ec, ev, Rr = _ell(dec, N, dev)
    g = np.random.default_rng(4)
    for lim, shr in ((1 << 22, (-30, -20)), (3, (-70, 10))):
        q = g.integers(-lim, lim + 1, (M, K))
        sh = g.integers(shr[0], shr[1], M)
        T_ref = R.wmm_f64(q, dec["W"])
        B_ref = R.residual(q, dec["rr"], dec["rc"], dec["rv"], N)
        ref, rflag, _ = R.epilogue(T_ref, B_ref, dec["d"], dec["g"], sh, R.FR, True)
        qd, shd = torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(sh).to(dev)
        T = wmm.wmm_hip(qd, limbs)
        y, flag = wmm.lin_y(T, (qd, ec, ev), d, gg, shd, checked=True)
        assert np.array_equal(y.cpu().numpy(), ref) and bool(flag) == rflag
        y2, flag2 = wmm.epilogue(T[0], torch.from_numpy(B_ref).to(dev), d, gg, shd, R.FR, True)
        assert np.array_equal(y2.cpu().numpy(), ref) and bool(flag2) == rflag
        X = torch.from_numpy(g.integers(-(1 << 40), 1 << 40, (M, N))).to(dev)
        T3 = torch.stack([T[0] - X, X])                  # two split partials summing to T
        y3 = wmm.lin_y(T3, (qd, ec, ev), d, gg, shd)
        assert np.array_equal(y3.cpu().numpy(), ref)


@pytest.mark.parametrize("N,K", [(2048, 2048), (2044, 4096), (2048, 8192), (2050, 16384), (16384, 2048)])
def test_int8_staged_rows(dev, N, K):
    """int8 decode with <= 8 stacked rows (the staged kernel: 8-column blocks over K / 1024 waves, or 64-column
    blocks at K = 2048), join and raw int32 modes, against the float64 oracle."""
    from bitexact.int8.gemm_skinny import int_mm, int_mm_join
    g = np.random.default_rng(N + K)
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    w[0, :] = -127
    for M in (1, 2, 3, 4, 5, 8):   # 5, 8: 10 and 16 stacked rows (the gemv)
        z = g.integers(-(1 << 44), 1 << 44, (M, K))
        q, _, _ = R.quant_rows(z, 2)
        a = R.stack_limbs(q, 2)
        y = int_mm_join(torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev), M, 2)
        assert np.array_equal(y.cpu().numpy(), R.imm(q, w)), (M, "join")
    for Rr in (1, 5, 8, 13, 16):
        a = g.integers(-128, 128, (Rr, K)).astype(np.int8)
        a[0, :] = -128
        c = int_mm(torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev))
        assert np.array_equal(c.cpu().numpy().astype(np.int64), R.imm(a, w)), (Rr, "raw")


@pytest.mark.parametrize("M,N,K", [(8, 160, 512), (100, 160, 512), (200, 160, 512), (300, 1024, 2048),
                                   (32, 16384, 512), (32, 2048, 8192)])
def test_exact_linear_dense_residual_rows(dev, M, N, K):
    """Rows whose residual lists are long: one element of 2^20 sets the row grid at 2^-3, so every ordinary
    N(0, 0.02) element of the row lands in the residual (hundreds of ELL entries; the epilogue keeps the first
    4 of a column in registers and reads the rest from memory). M = 8: gemv path; 100, 200: 64 x 64 tiles;
    300 x 1024 x 2048: 64 x 64 tiles with K split in 4 (the last block of a tile applies the epilogue); M = 32: the
    stream kernel, without and with K split."""
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    w = _bf16(N, K, 21)
    for n in (1, 7, 64, N - 1):
        w[n, (n * 7) % K] = 2.0 ** 20
    dec = _dec(w)
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    assert Rr > 64
    g = np.random.default_rng(M + 5)
    q = g.integers(-(1 << 22), (1 << 22) + 1, (M, K))
    sh = g.integers(-30, -20, M)
    ref, rflag, _ = R.epilogue(R.wmm_f64(q, dec["W"]), R.residual(q, dec["rr"], dec["rc"], dec["rv"], N),
                               dec["d"], dec["g"], sh, R.FR, True)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    y = exact_linear(torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(sh).to(dev), limbs, d, gg,
                     cnt, ec, ev, Rr, flag, True)
    assert np.array_equal(y.cpu().numpy(), ref), M
    assert bool(flag.item()) == rflag, M


@pytest.mark.parametrize("M", [33, 64])
@pytest.mark.parametrize("K", [1008, 2112])
def test_int8_tdec_k_tails(dev, M, K):
    """int8 decode with 65..128 stacked rows at N = 16384 (64 x 64 tiles with 128-byte k tiles): K not a multiple
    of the k tile (the last tile is partial and masked)."""
    from bitexact.int8.gemm_skinny import int_mm_join
    N = 16384
    g = np.random.default_rng(M * 7 + K)
    z = g.integers(-(1 << 44), 1 << 44, (M, K))
    q, _, _ = R.quant_rows(z, 2)
    a = R.stack_limbs(q, 2)
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    y = int_mm_join(torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev), M, 2)
    assert np.array_equal(y.cpu().numpy(), R.imm(q, w))


@pytest.mark.parametrize("M,N", [(32, 16384), (200, 2048), (8, 2048)])
def test_exact_linear_norm_planes(dev, M, N):
    """The add + norm kernel's limb planes fed to the exact linear (no split launch) give the same x, q, sh, y and
    flag as the separate stages, and y matches the oracle: the wide kernel (M = 32, 96 limb rows), the tile kernel
    (M = 200) and the row-vector path that ignores the planes (M = 8)."""
    from bitexact.exact import ops
    from bitexact.vllm_plugin.exact_gemm import exact_linear, needs_planes
    K = 512
    g = torch.Generator().manual_seed(M + N)
    x = torch.randint(-(1 << 33), 1 << 33, (M, K), generator=g)
    y = torch.randint(-(1 << 32), 1 << 32, (M, K), generator=g)
    gm, ge = torch.randint(-255, 256, (K,), generator=g), torch.randint(-14, -6, (K,), generator=g)
    x1, q1, sh1, e1 = ops.add_norm_y(y.to(dev), x.to(dev), gm.to(dev), ge.to(dev))
    x2, (q2, pl), sh2, e2 = ops.add_norm_y(y.to(dev), x.to(dev), gm.to(dev), ge.to(dev), planes=True)
    assert torch.equal(x1, x2) and torch.equal(q1, q2) and torch.equal(sh1, sh2) and bool(e1) == bool(e2)
    assert pl.shape == (3, M, K)
    assert needs_planes(M, N, K) == (M != 8)
    dec = _dec(_bf16(N, K, 3))
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    f1 = torch.zeros(1, dtype=torch.int32, device=dev)
    f2 = torch.zeros(1, dtype=torch.int32, device=dev)
    ya = exact_linear(q1, sh1, limbs, d, gg, cnt, ec, ev, Rr, f1, True)
    yb = exact_linear(q2, sh2, limbs, d, gg, cnt, ec, ev, Rr, f2, True, q_planes=pl)
    assert torch.equal(ya, yb) and f1.item() == f2.item()
    qn, shn = q1.cpu().numpy().astype(np.int64), sh1.cpu().numpy()
    ref, rflag, _ = R.epilogue(R.wmm_f64(qn, dec["W"]), R.residual(qn, dec["rr"], dec["rc"], dec["rv"], N),
                               dec["d"], dec["g"], shn, R.FR, True)
    assert np.array_equal(yb.cpu().numpy(), ref) and bool(f2.item()) == rflag


def test_norm_quant_planes(dev):
    """The norm without an add (the final norm before lm_head) writing q's limb planes: same q and sh as
    norm_quant, x left as it was, planes = the signed base-256 split of q; the exact linear on them = without. The
    embedding norm's planes likewise."""
    from bitexact.exact import ops
    from bitexact.vllm_plugin.exact_gemm import exact_linear, needs_planes
    M, K, N = 32, 512, 16384
    g = torch.Generator().manual_seed(8)
    x = torch.randint(-(1 << 35), 1 << 35, (M, K), generator=g).to(dev)
    gm, ge = torch.randint(-255, 256, (K,), generator=g).to(dev), torch.randint(-14, -6, (K,), generator=g).to(dev)
    x0 = x.clone()
    q1, sh1, e1 = ops.norm_quant(x, gm, ge)
    (q2, pl), sh2, e2 = ops.norm_quant(x, gm, ge, planes=True)
    assert torch.equal(x, x0) and torch.equal(q1, q2) and torch.equal(sh1, sh2) and bool(e1) == bool(e2)
    r = q1.long()
    for i in range(3):
        lo = ((r + 128) & 255) - 128
        assert torch.equal(pl[i].long(), lo)
        r = (r - lo) >> 8
    assert needs_planes(M, N, K)
    dec = _dec(_bf16(N, K, 12))
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    f1 = torch.zeros(1, dtype=torch.int32, device=dev)
    f2 = torch.zeros(1, dtype=torch.int32, device=dev)
    ya = exact_linear(q1, sh1, limbs, d, gg, cnt, ec, ev, Rr, f1, True)
    yb = exact_linear(q2, sh2, limbs, d, gg, cnt, ec, ev, Rr, f2, True, q_planes=pl)
    assert torch.equal(ya, yb) and f1.item() == f2.item()
    # the embedding norm's planes (the first layer's input)
    emb = torch.randint(-(1 << 30), 1 << 30, (300, K), generator=g, dtype=torch.int64).to(torch.int32).to(dev)
    ids = torch.randint(0, 300, (M,), generator=g).to(dev)
    xa, qa, sha, ea = ops.embed_norm(emb, ids, gm, ge)
    xb, (qb, plb), shb, eb = ops.embed_norm(emb, ids, gm, ge, planes=True)
    assert torch.equal(xa, xb) and torch.equal(qa, qb) and torch.equal(sha, shb) and bool(ea) == bool(eb)
    r = qa.long()
    for i in range(3):
        lo = ((r + 128) & 255) - 128
        assert torch.equal(plb[i].long(), lo)
        r = (r - lo) >> 8


@pytest.mark.parametrize("M,N,K", [(32, 3072, 2048), (22, 3080, 2048), (32, 4096, 2048), (32, 2048, 8192),
                                   (32, 2048, 2048)])
def test_exact_linear_narrow_planes(dev, M, N, K):
    """Narrow N with q's limb planes given: 32-column stream blocks with the K split over the zeroed workspace
    (without planes the gemv, or at K = 8192 64-column blocks in 8 splits, serve the shape); same y and flag as
    that path, and y matches the oracle (partial last column tile at N = 3080, forced residual entries, 66 and 96
    limb rows; the engine's down projection at N = 2048, K = 8192 and its wo at N = 2048, K = 2048, half the chip
    in 2 splits). N = 1024 keeps the gemv either way."""
    from bitexact.exact import ops
    from bitexact.vllm_plugin.exact_gemm import exact_linear, needs_planes, plan
    assert plan(32, 1024, 2048, planes=True)[0] == "gemv" and not needs_planes(32, 1024, 2048)
    assert plan(M, N, K)[0] == ("gemv" if K == 2048 else "stream")   # K = 8192: 64-column blocks, 8 splits
    kern, _, split, blocks = plan(M, N, K, planes=True)
    assert kern == "stream" and split > 1 and blocks == -(-N // 32), plan(M, N, K, planes=True)
    assert needs_planes(M, N, K)
    g = torch.Generator().manual_seed(M * N)
    if K <= 4096:                                     # the norm's row limit
        x = torch.randint(-(1 << 33), 1 << 33, (M, K), generator=g)
        y = torch.randint(-(1 << 32), 1 << 32, (M, K), generator=g)
        gm, ge = torch.randint(-255, 256, (K,), generator=g), torch.randint(-14, -6, (K,), generator=g)
        _, (q, pl), sh, _ = ops.add_norm_y(y.to(dev), x.to(dev), gm.to(dev), ge.to(dev), planes=True)
    else:                                             # quantized rows as the SiLU stage leaves them, planes by hand
        q = torch.randint(-(1 << 23) + 1, 1 << 23, (M, K), generator=g, dtype=torch.int32).to(dev)
        sh = torch.randint(-40, -20, (M,), generator=g).to(dev)
        pl = torch.empty(3, M, K, dtype=torch.int8, device=dev)
        r = q.long()
        for i in range(3):
            lo = ((r + 128) & 255) - 128
            pl[i] = lo.to(torch.int8)
            r = (r - lo) >> 8
    dec = _dec(_bf16(N, K, 11))
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    f1 = torch.zeros(1, dtype=torch.int32, device=dev)
    f2 = torch.zeros(1, dtype=torch.int32, device=dev)
    ya = exact_linear(q, sh, limbs, d, gg, cnt, ec, ev, Rr, f1, True)
    for _ in range(2):                                # the second call finds the workspace zeroed again
        f2.zero_()
        yb = exact_linear(q, sh, limbs, d, gg, cnt, ec, ev, Rr, f2, True, q_planes=pl)
        assert torch.equal(ya, yb) and f1.item() == f2.item()
    qn, shn = q.cpu().numpy().astype(np.int64), sh.cpu().numpy()
    ref, rflag, _ = R.epilogue(R.wmm_f64(qn, dec["W"]), R.residual(qn, dec["rr"], dec["rc"], dec["rv"], N),
                               dec["d"], dec["g"], shn, R.FR, True)
    assert np.array_equal(yb.cpu().numpy(), ref) and bool(f2.item()) == rflag


@pytest.mark.parametrize("M", [22, 32])
def test_exact_linear_silu_planes(dev, M):
    """The SiLU stage's limb planes fed to the exact linear at K = 8192 (MFMA tiles with K split) give the same q,
    sh, y and flag as the separate stages, and y matches the oracle."""
    from bitexact.exact import ops
    from bitexact.vllm_plugin.exact_gemm import exact_linear, needs_planes
    N, K = 2048, 8192
    g = torch.Generator().manual_seed(M)
    gu = torch.randint(-(1 << 31), 1 << 31, (M, 2 * K), generator=g)
    lut = torch.from_numpy(R.exp2_table()).to(dev)
    q1, sh1, e1 = ops.gu_silu_y(gu.to(dev), lut)
    (q2, pl), sh2, e2 = ops.gu_silu_y(gu.to(dev), lut, planes=True)
    assert torch.equal(q1, q2) and torch.equal(sh1, sh2) and bool(e1) == bool(e2) and pl.shape == (3, M, K)
    assert needs_planes(M, N, K)
    dec = _dec(_bf16(N, K, 5))
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    f1 = torch.zeros(1, dtype=torch.int32, device=dev)
    f2 = torch.zeros(1, dtype=torch.int32, device=dev)
    ya = exact_linear(q1, sh1, limbs, d, gg, cnt, ec, ev, Rr, f1, True)
    yb = exact_linear(q2, sh2, limbs, d, gg, cnt, ec, ev, Rr, f2, True, q_planes=pl)
    assert torch.equal(ya, yb) and f1.item() == f2.item()
    qn, shn = q1.cpu().numpy().astype(np.int64), sh1.cpu().numpy()
    ref, rflag, _ = R.epilogue(R.wmm_f64(qn, dec["W"]), R.residual(qn, dec["rr"], dec["rc"], dec["rv"], N),
                               dec["d"], dec["g"], shn, R.FR, True)
    assert np.array_equal(yb.cpu().numpy(), ref) and bool(f2.item()) == rflag


@pytest.mark.parametrize("M", [4, 200])
def test_corrupt_ell_index_sets_flag(dev, M):
    """A residual column outside [0, K) or a count above R (a damaged weight) never reads outside q: the linear
    raises the flag, checked or not, on the row-vector path (M = 4) and the tile path (M = 200). Valid lists leave
    the flag clear."""
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    N, K = 160, 512
    dec = _dec(_bf16(N, K, 11))
    limbs = torch.from_numpy(dec["limbs"]).to(dev)
    d, gg = torch.from_numpy(dec["d"]).to(dev), torch.from_numpy(dec["g"]).to(dev)
    cnt, ec, ev, Rr = _ell(dec, N, dev)
    q = torch.ones(M, K, dtype=torch.int32, device=dev)
    sh = torch.full((M,), -30, dtype=torch.long, device=dev)
    for checked in (True, False):
        flag = torch.zeros(1, dtype=torch.int32, device=dev)
        exact_linear(q, sh, limbs, d, gg, cnt, ec, ev, Rr, flag, checked)
        assert flag.item() == 0
    n0 = int(torch.nonzero(cnt).flatten()[0])
    for kind in ("col", "cnt"):
        ec2, cnt2 = ec.clone(), cnt.clone()
        if kind == "col":
            ec2[n0, 0] = K + 5
        else:
            cnt2[n0] = Rr + 1
        for checked in (True, False):
            flag = torch.zeros(1, dtype=torch.int32, device=dev)
            exact_linear(q, sh, limbs, d, gg, cnt2, ec2, ev, Rr, flag, checked)
            assert flag.item() == 1, (kind, checked)


@pytest.mark.parametrize("N,K", [(16384, 2048), (16400, 1024), (32768, 512), (8192, 2048), (8200, 1024)])
def test_int8_stream_wide(dev, N, K):
    """int8 decode where the 64-column tiles (or, at N = 8192, the 32-column tiles) cover the chip without a K split
    (the stream kernel): a partial last column tile (N = 16400, 8200), join in registers (M % 16 == 0) and through LDS (other M), raw int32 rows up to 128,
    extreme operands, against the float64 oracle."""
    from bitexact.int8.gemm_skinny import int_mm, int_mm_join
    from bitexact import _hip
    g = np.random.default_rng(N + K)
    w = g.integers(-128, 128, (N, K)).astype(np.int8)
    w[N - 1, :] = -128
    wd = torch.from_numpy(w).to(dev)
    for M, nl in ((1, 2), (16, 2), (32, 3), (21, 3), (48, 2), (64, 2), (40, 1)):
        out = (ctypes.c_int32 * 6)()
        assert _hip.lib().bx_int8_gemm_plan(M, N, K, nl, out) == 0, (M, nl)
        if N > 8200 or M * nl > 64:   # N = 8192: 32-column tiles from 65 stacked rows, the gemv below
            assert out[0] == 5, (M, nl, list(out))
        z = g.integers(-(1 << 44), 1 << 44, (M, K))
        q, _, _ = R.quant_rows(z, nl)
        a = R.stack_limbs(q, nl)
        y = int_mm_join(torch.from_numpy(a).to(dev), wd, M, nl)
        assert np.array_equal(y.cpu().numpy(), R.imm(q, w)), (M, nl)
    for Rr in (1, 7, 16, 33, 64, 100, 128):
        a = g.integers(-128, 128, (Rr, K)).astype(np.int8)
        a[0, :] = -128
        c = int_mm(torch.from_numpy(a).to(dev), wd)
        assert np.array_equal(c.cpu().numpy().astype(np.int64), R.imm(a, w)), (Rr, "raw")
