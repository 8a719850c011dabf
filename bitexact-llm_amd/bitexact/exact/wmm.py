"""Exact products of activations with the original bf16 weights (src/bitexact/exact/wmm.py), on MFMA.

wmm_hip(q, limbs) is the wmm_triton / wmm_cublas / wmm_cpu contract: q int32 [M, K] (|q| <= 2^22), limbs int8
[3, N, K] -> the exact int64 dense product, returned as [1, M, N] (one split-K slice; the reference's caller
sums dim 0).
"""

import torch

from bitexact import _hip


def wmm_hip(q, limbs):
    _hip.require_cuda(q, limbs)
    assert q.dtype == torch.int32 and limbs.dtype == torch.int8 and limbs.shape[0] == 3
    assert q.stride(1) == 1 and limbs.stride(2) == 1
    M, K = q.shape
    N = limbs.shape[1]
    assert limbs.shape[2] == K
    T = torch.empty(1, M, N, dtype=torch.long, device=q.device)
    ws, wsb = _hip.workspace(q.device, _hip.lib().bx_exact_linear_workspace(M, N, K))
    tmp, tmpb = _hip.scratch(q.device, _hip.lib().bx_exact_linear_scratch(M, N, K))
    _hip.call("bx_exact_wmm", _hip.ptr(q), q.stride(0), _hip.ptr(limbs), limbs.stride(0), limbs.stride(1),
              _hip.ptr(T), M, N, K, _hip.ptr(ws), wsb, _hip.ptr(tmp), tmpb, _hip.stream_of(q))
    return T
