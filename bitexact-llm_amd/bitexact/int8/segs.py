"""int8-mode element-wise segments on HIP (src/bitexact/int8/segs.py, src/bitexact/int8/ops.py).

quant_rows(z, nl)        ops.quant_rows + intops.stack_limbs -> (a int8 [nl M, K], as_, sh)
pre_plain(x, nl)         segs.pre_plain with the limbs stacked -> (a int8 [nl M, K], mant, e)
post(acc, m, fmsh, mant, e, check=True)   segs.post on the joined products -> (y at FR, flag)

Stacked rows: limb i of row m is row i M + m (no padding rows: the HIP GEMM takes any row count).
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op

FR = 16                         # residual stream, layer outputs (src/bitexact/int8/consts.py:26)


def _quant_fake(z, nl, with_scale):
    M, K = z.shape
    n = M if with_scale else 0
    return (empty((nl * M, K), torch.int8, z), empty((M,), torch.long, z), empty((M,), torch.long, z),
            empty((n,), torch.long, z), empty((n,), torch.long, z))


@op("int8_quant_rows(Tensor z, int nl, bool with_scale) -> (Tensor, Tensor, Tensor, Tensor, Tensor)", _quant_fake)
def _quant(z, nl, with_scale):
    _hip.require_cuda(z)
    assert z.dtype == torch.int64 and z.dim() == 2 and z.stride(1) == 1 and 1 <= nl <= 3
    M, K = z.shape
    dev = z.device
    a = torch.empty(nl * M, K, dtype=torch.int8, device=dev)
    as_ = torch.empty(M, dtype=torch.long, device=dev)
    sh = torch.empty(M, dtype=torch.long, device=dev)
    mant = torch.empty(M if with_scale else 0, dtype=torch.long, device=dev)
    e = torch.empty(M if with_scale else 0, dtype=torch.long, device=dev)
    _hip.call("bx_int8_quant_rows", _hip.ptr(z), z.stride(0), M, K, nl, FR, _hip.ptr(a), _hip.ptr(as_), _hip.ptr(sh),
              _hip.ptr(mant) if with_scale else None, _hip.ptr(e) if with_scale else None, _hip.stream_of(z))
    return a, as_, sh, mant, e


def quant_rows(z, nl):
    """ops.quant_rows (src/bitexact/int8/ops.py:24-35) with the limbs stacked (src/bitexact/intops.py:73-79)."""
    a, as_, sh, _, _ = _quant(z, nl, False)
    return a, as_, sh


def pre_plain(x, nl):
    """segs.pre_plain (src/bitexact/int8/segs.py:56-59) -> (stacked limbs, mant, e)."""
    a, _, _, mant, e = _quant(x, nl, True)
    return a, mant, e


def post(acc, m, fmsh, mant, e, check=True):
    """segs.post (src/bitexact/int8/segs.py:62-67): acc int64 [M, N] joined products, m int64 [N], fmsh int,
    mant / e int64 [M] -> (y int64 [M, N] at FR, flag bool tensor or None when check is False)."""
    y, flag = _post(acc, m, int(fmsh), mant, e)
    return y, ((flag[0] != 0) if check else None)


@op("int8_post(Tensor acc, Tensor m, int fmsh, Tensor mant, Tensor e) -> (Tensor, Tensor)",
    lambda acc, m, fmsh, mant, e: (empty(acc.shape, torch.long, acc), empty((1,), torch.int32, acc)))
def _post(acc, m, fmsh, mant, e):
    _hip.require_cuda(acc, m, mant, e)
    assert acc.dtype == torch.int64 and acc.dim() == 2 and acc.stride(1) == 1
    M, N = acc.shape
    m, mant, e = m.contiguous().long(), mant.contiguous().long(), e.contiguous().long()
    y = torch.empty(M, N, dtype=torch.long, device=acc.device)
    flag = torch.zeros(1, dtype=torch.int32, device=acc.device)
    _hip.call("bx_int8_post", _hip.ptr(acc), acc.stride(0), _hip.ptr(m), int(fmsh), _hip.ptr(mant), _hip.ptr(e), FR,
              _hip.ptr(y), y.stride(0), M, N, _hip.ptr(flag), _hip.stream_of(acc))
    return y, flag
