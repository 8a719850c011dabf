"""Integer helpers of the sampler on HIP (src/bitexact/intops.py)."""

import torch

from bitexact import _hip


def first_argmax(v):
    """Index of the first maximum of each row of int64 v [M, N] (src/bitexact/intops.py:55-59) -> int64 [M]."""
    _hip.require_cuda(v)
    assert v.dtype == torch.int64 and v.dim() == 2 and v.stride(1) == 1
    M, N = v.shape
    out = torch.empty(M, dtype=torch.long, device=v.device)
    _hip.call("bx_first_argmax", _hip.ptr(v), v.stride(0), M, N, _hip.ptr(out), _hip.stream_of(v))
    return out
