"""Exact products of activations with the original bf16 weights (src/bitexact/exact/wmm.py), on MFMA.

wmm_hip(q, limbs) is the wmm_triton / wmm_cublas / wmm_cpu contract: q int32 [M, K] (|q| <= 2^22), limbs int8
[3, N, K] -> the exact int64 dense product, returned as [1, M, N] (one split-K slice; the reference's caller
sums dim 0). epilogue(T, B, d, g, sh, FR, checked) is wmm.epilogue on the device (T [M, N] or [split, M, N]).
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


def epilogue(T, B, d, g, sh, FR, checked=False, ell=None):
    """wmm.epilogue (src/bitexact/exact/wmm.py:132-150): y int64 [M, N] = round((T 2^d + B) 2^(sh + g - d + FR));
    returns y, or (y, flag) with checked. B is the dense residual [M, N], or None with ell = (q, ec, ev) for
    segs.lin_y's gather (src/bitexact/exact/segs.py:31)."""
    _hip.require_cuda(T, d, g, sh)
    T3 = T if T.dim() == 3 else T.unsqueeze(0)
    assert T3.dtype == torch.int64 and T3.stride(2) == 1
    S, M, N = T3.shape
    d, g, sh = d.contiguous().long(), g.contiguous().long(), sh.contiguous().long()
    y = torch.empty(M, N, dtype=torch.long, device=T.device)
    flag = torch.zeros(1, dtype=torch.int32, device=T.device)
    if B is not None:
        assert B.dtype == torch.int64 and B.stride(1) == 1
        args = (_hip.ptr(B), B.stride(0), None, 0, 0, None, None, 0)
    else:
        q, ec, ev = ell
        assert q.dtype == torch.int32 and q.stride(1) == 1
        ec, ev = ec.contiguous().int(), ev.contiguous().long()
        args = (None, 0, _hip.ptr(q), q.stride(0), q.shape[1], _hip.ptr(ec), _hip.ptr(ev), ec.shape[1])
    _hip.call("bx_exact_epilogue", _hip.ptr(T3), T3.stride(1), T3.stride(0), S, *args, _hip.ptr(d), _hip.ptr(g),
              _hip.ptr(sh), int(FR), int(checked), _hip.ptr(y), y.stride(0), M, N, _hip.ptr(flag), _hip.stream_of(T))
    return (y, flag[0].bool()) if checked else y


def lin_y(C, rs, d, g, sh, checked=False, FR=24):
    """segs.lin_y (src/bitexact/exact/segs.py:25-32): rs = (B,) or (q, ec, ev)."""
    if len(rs) == 1:
        return epilogue(C, rs[0], d, g, sh, FR, checked)
    return epilogue(C, None, d, g, sh, FR, checked, ell=rs)
