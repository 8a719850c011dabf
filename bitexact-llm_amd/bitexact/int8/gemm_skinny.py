"""int8-mode GEMM (src/bitexact/int8/gemm_skinny.py:80-97) on gfx950 MFMA.

int_mm(a, w) -> int32 [R, N] = a int8 [R, K] @ w int8 [N, K]^T, the reference's contract (exact while
K * 127 * 128 < 2^31). int_mm_join(a, w, M, nl) also joins the nl limb row blocks of a in int64
(intops.join_limbs over the product, src/bitexact/intops.py:82-87): y int64 [M, N], one launch.
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op


def _check(a, w):
    _hip.require_cuda(a, w)
    assert a.dtype == torch.int8 and w.dtype == torch.int8
    assert a.is_contiguous() and w.is_contiguous() and a.shape[1] == w.shape[1]


@op("int_mm(Tensor a, Tensor w) -> Tensor", lambda a, w: empty((a.shape[0], w.shape[0]), torch.int32, a))
def int_mm(a, w):
    _check(a, w)
    R, K = a.shape
    N = w.shape[0]
    c = torch.empty(R, N, dtype=torch.int32, device=a.device)
    ws, wsb = _hip.workspace(a.device, _hip.lib().bx_int8_gemm_workspace(R, N, K, 1))
    _hip.call("bx_int8_gemm", _hip.ptr(a), _hip.ptr(w), _hip.ptr(c), R, N, K, _hip.ptr(ws), wsb, _hip.stream_of(a))
    return c


@op("int_mm_join(Tensor a, Tensor w, int M, int nl) -> Tensor",
    lambda a, w, M, nl: empty((M, w.shape[0]), torch.long, a))
def int_mm_join(a, w, M, nl):
    """a: nl row blocks of M limb rows (rows beyond nl M, e.g. stack_limbs' padding, are ignored)."""
    _check(a, w)
    K = a.shape[1]
    N = w.shape[0]
    assert a.shape[0] >= nl * M
    y = torch.empty(M, N, dtype=torch.long, device=a.device)
    ws, wsb = _hip.workspace(a.device, _hip.lib().bx_int8_gemm_workspace(M, N, K, nl))
    _hip.call("bx_int8_gemm_join", _hip.ptr(a), _hip.ptr(w), _hip.ptr(y), M, N, K, nl, _hip.ptr(ws), wsb,
              _hip.stream_of(a))
    return y
