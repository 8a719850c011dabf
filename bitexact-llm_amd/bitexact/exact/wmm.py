"""Exact products of activations with the original bf16 weights (src/bitexact/exact/wmm.py), on MFMA.

wmm_hip(q, limbs) is the wmm_triton / wmm_cublas / wmm_cpu contract: q int32 [M, K] (|q| <= 2^22), limbs int8
[3, N, K] -> the exact int64 dense product, returned as [1, M, N] (one split-K slice; the reference's caller
sums dim 0). epilogue(T, B, d, g, sh, FR, checked) is wmm.epilogue on the device (T [M, N] or [split, M, N]).
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op


def _wmm_fake(q, limbs):
    return empty((1, q.shape[0], limbs.shape[1]), torch.long, q)


@op("wmm(Tensor q, Tensor limbs) -> Tensor", _wmm_fake)
def wmm_hip(q, limbs):
    """q int32 [M, K], limbs int8 [3, N, K] -> the exact dense product int64 [1, M, N]."""
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


def _epilogue_fake(T, B, q, ec, ev, d, g, sh, FR, checked):
    return empty(T.shape[-2:], torch.long, T), empty((1,), torch.int32, T)


@op("epilogue(Tensor T, Tensor? B, Tensor? q, Tensor? ec, Tensor? ev, Tensor d, Tensor g, Tensor sh, int FR, "
    "bool checked) -> (Tensor, Tensor)", _epilogue_fake)
def _epilogue(T, B, q, ec, ev, d, g, sh, FR, checked):
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
        assert q.dtype == torch.int32 and q.stride(1) == 1
        ec, ev = ec.contiguous().int(), ev.contiguous().long()
        args = (None, 0, _hip.ptr(q), q.stride(0), q.shape[1], _hip.ptr(ec), _hip.ptr(ev), ec.shape[1])
    _hip.call("bx_exact_epilogue", _hip.ptr(T3), T3.stride(1), T3.stride(0), S, *args, _hip.ptr(d), _hip.ptr(g),
              _hip.ptr(sh), int(FR), int(checked), _hip.ptr(y), y.stride(0), M, N, _hip.ptr(flag), _hip.stream_of(T))
    return y, flag


def epilogue(T, B, d, g, sh, FR, checked=False, ell=None):
    """wmm.epilogue (src/bitexact/exact/wmm.py:132-150): y int64 [M, N] = round((T 2^d + B) 2^(sh + g - d + FR));
    returns y, or (y, flag) with checked. B is the dense residual [M, N], or None with ell = (q, ec, ev) for
    segs.lin_y's gather (src/bitexact/exact/segs.py:31)."""
    q, ec, ev = ell if B is None else (None, None, None)
    y, flag = _epilogue(T, B, q, ec, ev, d, g, sh, int(FR), bool(checked))
    return (y, flag[0] != 0) if checked else y


def lin_y(C, rs, d, g, sh, checked=False, FR=24):
    """segs.lin_y (src/bitexact/exact/segs.py:25-32): rs = (B,) or (q, ec, ev)."""
    if len(rs) == 1:
        return epilogue(C, rs[0], d, g, sh, FR, checked)
    return epilogue(C, None, d, g, sh, FR, checked, ell=rs)


# ---- the reference's entry names (src/bitexact/exact/wmm.py:79-129) ----
def wmm_triton(q, limbs, cfg=None, target=None):
    """wmm_triton's contract: int64 partial sums [split, M, N] whose sum is the exact product (here one slice:
    the HIP kernel joins its K splits itself). cfg / target are accepted for signature parity."""
    return wmm_hip(q, limbs)


def wmm_cublas(q, wcat, M_chunk=2048):
    """wmm_cublas's contract: wcat int8 [3 N, K] (limb j in rows j N ..) -> exact int64 [M, N]."""
    N = wcat.shape[0] // 3
    return wmm_hip(q, wcat.view(3, N, wcat.shape[1]))[0]


def wmm_cpu(q, w64):
    """The reference's float64 CPU product. This build has no CPU path: it raises."""
    raise AssertionError("bitexact (MI355X) has no CPU GEMM: use wmm_hip / wmm_triton on device tensors")


def residual(q, rr, rc, rv, N):
    """Dense residual B [M, N] = sum over entries (row n, col k, value v) of q[:, k] v (wmm.py:124-129), on the
    device with int64 index_add (integer sums: exact in any order). The fused linear and lin_y take the ELL form
    instead and never build B."""
    _hip.require_cuda(q, rr, rc, rv)
    B = torch.zeros(q.shape[0], N, dtype=torch.long, device=q.device)
    if rr.numel():
        B.index_add_(1, rr.long(), q[:, rc.long()].long() * rv.long())
    return B
