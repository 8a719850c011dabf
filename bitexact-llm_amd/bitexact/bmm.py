"""Exact batched integer matrix product for attention (src/bitexact/bmm.py:78-102).

bmm(a, b, na=3, nb=3): a [Z, M, K] x b [Z, K, N] int32 / int64 tensors (any strides), every |a| and |b| within
na / nb signed base-256 limbs -> exact int64 [Z, M, N] on the GPU.
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op


@op("bmm(Tensor a, Tensor b, int na, int nb) -> Tensor",
    lambda a, b, na, nb: empty((a.shape[0], a.shape[1], b.shape[2]), torch.long, a))
def _bmm(a, b, na, nb):
    _hip.require_cuda(a, b)
    Z, M, K = a.shape
    N = b.shape[2]
    assert b.shape[0] == Z and b.shape[1] == K
    assert K < 43690
    assert a.dtype in (torch.int32, torch.int64) and b.dtype in (torch.int32, torch.int64)
    c = torch.empty(Z, M, N, dtype=torch.long, device=a.device)
    _hip.call("bx_limb_bmm", _hip.ptr(a), a.element_size(), a.stride(0), a.stride(1), a.stride(2), _hip.ptr(b),
              b.element_size(), b.stride(0), b.stride(1), b.stride(2), _hip.ptr(c), c.stride(0), c.stride(1),
              c.stride(2), Z, M, N, K, na, nb, _hip.stream_of(a))
    return c


def bmm(a, b, na=3, nb=3):
    """Exact a @ b for [Z, M, K] x [Z, K, N] integer tensors -> int64 [Z, M, N]."""
    return _bmm(a, b, int(na), int(nb))
