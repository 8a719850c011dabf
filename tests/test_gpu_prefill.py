"""Config 3 (exact prefill, M = 2048 over every Llama-3.2-1B linear) bit for bit against the oracle, on the tile
kernels that serve it: the 128 x 128 exact tile (q/o, gate/up, down, lm_head, the fused qkv / gate|up shapes, and
the engine's 4096-row prefill chunks), the 64 x 128 tile (M = 1024, N = 2048) and the 64 x 64 tile (k/v).
Shapes and adversarial cases follow the reference's tests/test_exact_ops.py:137-152 and
tests/test_vllm_exact_gemm.py:11-31 (extreme limbs, forced residual entries, three magnitude / shift ranges)."""

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu

RANGES = ((1 << 22, (-30, -20)), (1 << 12, (-45, -8)), (3, (-70, 10)))


def _weights(N, K, seed, dense_rows=()):
    """bf16 N(0, 0.02) with forced residual entries; rows in dense_rows get one 2^20 element, which puts the row
    grid at 2^-3 so every other element of the row lands in the residual (hundreds of ELL entries)."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    w[0, :5] = torch.tensor([1e-9, -3e-8, 0.0, 2.0, -0.5]).to(torch.bfloat16)
    w[N - 1, K - 3:] = torch.tensor([3e-7, -1e-6, 1e-10]).to(torch.bfloat16)
    for n in dense_rows:
        w[n, (n * 7) % K] = 2.0 ** 20
    return w


def _q(M, K, lim, shr, seed):
    g = np.random.default_rng(seed)
    q = g.integers(-lim, lim + 1, (M, K))
    q[0, :] = lim
    q[min(1, M - 1), :] = -lim
    return q, g.integers(shr[0], shr[1], M)


def _dev_weights(w, dev):
    from bitexact.exact.consts import decompose
    return decompose(w.to(dev))


def _run(dec, q, sh, dev):
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    y = exact_linear(torch.from_numpy(q).to(torch.int32).to(dev), torch.from_numpy(sh).to(dev), dec["limbs"],
                     dec["d"], dec["g"], dec["ell_cnt"], dec["ell_col"], dec["ell_val"], dec["R"], flag, True)
    return y, flag


def _check(w, M, dev, tile, seed, dense_rows=(), ranges=RANGES):
    from bitexact.vllm_plugin.exact_gemm import plan
    N, K = w.shape
    assert plan(M, N, K)[:2] == ("tile", tile), plan(M, N, K)
    ref_dec = R.decompose(w.view(torch.int16).numpy())
    dec = _dev_weights(w, dev)
    if dense_rows:
        assert dec["R"] > 64
    for i, (lim, shr) in enumerate(ranges):
        q, sh = _q(M, K, lim, shr, seed + i)
        ref, rflag, _ = R.epilogue(R.wmm_f64(q, ref_dec["W"]),
                                   R.residual(q, ref_dec["rr"], ref_dec["rc"], ref_dec["rv"], N),
                                   ref_dec["d"], ref_dec["g"], sh, R.FR, True)
        y, flag = _run(dec, q, sh, dev)
        got = y.cpu().numpy()
        if not np.array_equal(got, ref):
            bad = np.argwhere(got != ref)
            raise AssertionError(f"{M}x{N}x{K} range {i}: {len(bad)} mismatches, first at {bad[0].tolist()}")
        assert bool(flag.item()) == rflag, (M, N, K, i)


@pytest.mark.parametrize("name,N,K,dense", [("q_o", 2048, 2048, (1, 7, 130, 2046)), ("gate_up", 8192, 2048, ()),
                                            ("down", 2048, 8192, ()), ("qkv_fused", 3072, 2048, ()),
                                            ("k_v", 512, 2048, ())])
def test_config3_prefill_shapes(dev, name, N, K, dense):
    """Config 3 at M = 2048: q/o, gate/up and down on the 128 x 128 exact tile (q/o with dense-residual rows,
    whose residual lists run past the 4 entries kept in registers), k/v on the 64 x 64 tile."""
    tile = "64x64" if N == 512 else "128x128"
    _check(_weights(N, K, N + K, dense), 2048, dev, tile, 100 + N, dense_rows=dense)


def test_prefill_partial_tiles(dev):
    """128 x 128 tiles with a partial row tile and a partial column tile (M = 2000, N = 2088)."""
    _check(_weights(2088, 2048, 3, (2086,)), 2000, dev, "128x128", 7, dense_rows=(2086,))


def test_prefill_mid_tile(dev):
    """The 64 x 128 tile (M = 1024, N = 2048), no K split."""
    _check(_weights(2048, 2048, 4), 1024, dev, "64x128", 11)


def test_prefill_small_tile_split(dev):
    """The 64 x 64 exact tile with K split over blocks (M = 250, N = 1024, K = 8192: the last block of a tile
    applies the epilogue from the int64 partial sums). The 128 x 128 tile never splits K: it is chosen only when
    its tiles fill the chip."""
    from bitexact.vllm_plugin.exact_gemm import plan
    assert plan(250, 1024, 8192)[2] > 1
    _check(_weights(1024, 8192, 5, (3, 1000)), 250, dev, "64x64", 13, dense_rows=(3, 1000))


def test_engine_prefill_chunk(dev):
    """The engine's prefill chunk: 4096 rows through the fused gate|up shape (N = 16384) on the 128 x 128 tile."""
    _check(_weights(16384, 2048, 6), 4096, dev, "128x128", 17, ranges=RANGES[:1])


def test_lm_head_column_sample(dev):
    """lm_head (N = 128256, K = 2048) at M = 2048, the full kernel on the device, checked against the oracle on
    the first and last column of every 128-column tile plus 64 random columns, for every row."""
    from bitexact.vllm_plugin.exact_gemm import plan
    N, K, M = 128256, 2048, 2048
    assert plan(M, N, K)[:2] == ("tile", "128x128")
    gw = torch.Generator(device=dev).manual_seed(42)
    w = (torch.randn(N, K, generator=gw, device=dev) * 0.02).to(torch.bfloat16)
    w[0, :3] = torch.tensor([1e-9, 2.0, -3e-8], device=dev).to(torch.bfloat16)
    w[N - 1, 5] = 2.0 ** 20
    dec = _dev_weights(w, dev)
    cols = np.unique(np.concatenate([np.arange(0, N, 128), np.arange(127, N, 128),
                                     np.random.default_rng(1).integers(0, N, 64)]))
    ws = w[torch.from_numpy(cols).to(dev)].cpu()
    ref_dec = R.decompose(ws.view(torch.int16).numpy())
    for i, (lim, shr) in enumerate(RANGES[:2]):
        q, sh = _q(M, K, lim, shr, 50 + i)
        ref, rflag, bad = R.epilogue(R.wmm_f64(q, ref_dec["W"]),
                                     R.residual(q, ref_dec["rr"], ref_dec["rc"], ref_dec["rv"], len(cols)),
                                     ref_dec["d"], ref_dec["g"], sh, R.FR, True)
        y, flag = _run(dec, q, sh, dev)
        got = y[:, torch.from_numpy(cols).to(dev)].cpu().numpy()
        assert np.array_equal(got, ref), (i, int((got != ref).sum()))
        if rflag:
            assert bool(flag.item())
    del dec, w
    torch.cuda.empty_cache()


def test_prefill_k_tail_fallback(dev):
    """K % 64 != 0 at a 128 x 128-tile shape: the pipelined tile needs whole 64-deep k tiles, so the plain 128 x 128
    tile (2-stage ring, masked last k tile) serves it; same integers."""
    _check(_weights(2048, 2000, 8, (5,)), 2048, dev, "128x128", 19, dense_rows=(5,), ranges=RANGES[:2])


def test_prefill_xtile_order_off(dev):
    """The pipelined tile with a tile grid that is not a multiple of 8 (15 x 18 tiles), where the XCD-grouped order is
    off, at K = 8192."""
    _check(_weights(2304, 8192, 9), 1920, dev, "128x128", 23, ranges=RANGES[:1])
