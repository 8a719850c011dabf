"""bx_exact_linear_noalloc (static device scratch, no caller buffers) against bx_exact_linear, both called through
the C ABI: two calls in a row, the second with a smaller input, on the split-K tile path (workspace + limb-plane
scratch) and on the row-vector path (workspace only). The outputs and flags must be identical."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _weights(N, K, seed, dev):
    from bitexact.exact.consts import decompose
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    w[0, :3] = torch.tensor([1e-9, 2.0, -3e-8]).to(torch.bfloat16)
    return decompose(w.to(dev))


def _args(dec, q, sh, y, flag, checked):
    from bitexact import _hip
    M, K = q.shape
    N = dec["limbs"].shape[1]
    R = dec["R"]
    L = dec["limbs"]
    return (_hip.ptr(q), q.stride(0), _hip.ptr(sh), _hip.ptr(L), L.stride(0), L.stride(1), _hip.ptr(dec["d"]),
            _hip.ptr(dec["g"]), _hip.ptr(dec["ell_cnt"]) if R else None, _hip.ptr(dec["ell_col"]) if R else None,
            _hip.ptr(dec["ell_val"]) if R else None, R, _hip.ptr(y), M, N, K, 24, int(checked), _hip.ptr(flag))


def _pair(dev, dec, M, seed, lim=1 << 22, shr=(-30, -20)):
    from bitexact import _hip
    K = dec["limbs"].shape[2]
    N = dec["limbs"].shape[1]
    g = np.random.default_rng(seed)
    q = torch.from_numpy(g.integers(-lim, lim + 1, (M, K))).to(torch.int32).to(dev)
    sh = torch.from_numpy(g.integers(shr[0], shr[1], M)).to(dev)
    stream = _hip.stream_of(q)
    y1 = torch.full((M, N), 7, dtype=torch.long, device=dev)
    f1 = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(max(_hip.lib().bx_exact_linear_workspace(M, N, K), 16), dtype=torch.uint8, device=dev)
    tmp = torch.empty(max(_hip.lib().bx_exact_linear_scratch(M, N, K), 16), dtype=torch.uint8, device=dev)
    _hip.call("bx_exact_linear", *_args(dec, q, sh, y1, f1, True), _hip.ptr(ws), ws.numel(), _hip.ptr(tmp),
              tmp.numel(), stream)
    y2 = torch.full((M, N), -7, dtype=torch.long, device=dev)
    f2 = torch.zeros(1, dtype=torch.int32, device=dev)
    _hip.call("bx_exact_linear_noalloc", *_args(dec, q, sh, y2, f2, True), stream)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), (M, N, K)
    assert f1.item() == f2.item()
    return f1.item()


@pytest.mark.parametrize("N,K,Ms", [(1024, 2048, (300, 100)), (2048, 8192, (128, 32)), (2048, 2048, (8, 3)),
                                    (512, 2048, (2048, 1000))])
def test_noalloc_matches_exact_linear(dev, N, K, Ms):
    from bitexact.vllm_plugin.exact_gemm import plan
    dec = _weights(N, K, N + K, dev)
    for i, M in enumerate(Ms):
        print(f"noalloc N={N} K={K} M={M} plan={plan(M, N, K)}", flush=True)
        _pair(dev, dec, M, 10 * i + M)
    # a flagged case (values at the top of the range with a large shift) keeps the flag identical as well
    assert _pair(dev, dec, Ms[-1], 99, lim=1 << 22, shr=(30, 31)) == 1


def test_noalloc_rejects_oversize(dev):
    """A plan needing more scratch than the static array fails cleanly with BX_EINVAL before any launch."""
    from bitexact import _hip
    assert _hip.lib().bx_exact_linear_noalloc_limit() == 32 << 20
    M, N, K = 8192, 2048, 2048                      # 48 MiB of limb planes
    assert _hip.lib().bx_exact_linear_scratch(M, N, K) > 24 << 20
    dec = _weights(N, K, 3, dev)
    q = torch.zeros(M, K, dtype=torch.int32, device=dev)
    sh = torch.zeros(M, dtype=torch.long, device=dev)
    y = torch.empty(M, N, dtype=torch.long, device=dev)
    f = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(AssertionError, match="exceeds the static"):
        _hip.call("bx_exact_linear_noalloc", *_args(dec, q, sh, y, f, True), _hip.stream_of(q))
