"""Integer helpers of the sampler on HIP (src/bitexact/intops.py)."""

import torch

from bitexact import _hip
from bitexact._ops import empty, op


@op("first_argmax(Tensor v, bool split) -> Tensor", lambda v, split: empty((v.shape[0],), torch.long, v))
def _first_argmax(v, split):
    _hip.require_cuda(v)
    assert v.dtype == torch.int64 and v.dim() == 2 and v.stride(1) == 1
    M, N = v.shape
    out = torch.empty(M, dtype=torch.long, device=v.device)
    if split and M > 0 and N > 0:
        tmp, tmpb = _hip.scratch(v.device, _hip.lib().bx_first_argmax_scratch(M, N))
        _hip.call("bx_first_argmax_ws", _hip.ptr(v), v.stride(0), M, N, _hip.ptr(out), _hip.ptr(tmp), tmpb,
                  _hip.stream_of(v))
        return out
    _hip.call("bx_first_argmax", _hip.ptr(v), v.stride(0), M, N, _hip.ptr(out), _hip.stream_of(v))
    return out


def first_argmax(v, split=None):
    """Index of the first maximum of each row of int64 v [M, N] (src/bitexact/intops.py:55-59) -> int64 [M].
    split: None picks by shape (column chunks for fewer than 128 rows of at least 16384 columns); True / False
    force the chunked or the row-per-block kernel (the same indices either way)."""
    if split is None:
        split = v.shape[0] < 128 and v.shape[1] >= 16384
    return _first_argmax(v, bool(split))
