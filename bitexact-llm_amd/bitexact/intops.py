"""Integer rules shared by both engines (src/bitexact/intops.py) on HIP.

The reference's names and contracts: every function is a fixed integer rule on int64 device tensors (two's
complement wrap, round half up, floor division), computed by the element-wise kernels of csrc/bx_elem.hip, so the
integers equal the reference's CPU tensors' bit for bit. Device tensors only (there is no CPU path); Python ints
are accepted where the reference accepts them.
"""

import torch

from bitexact import _elem, _hip
from bitexact._ops import empty, op

LIM = {1: 127, 2: 32639, 3: 8355711}          # n signed base-256 digits reach 127 * (256^n - 1) / 255


def bitlen(x):
    """Number of bits of int64 x >= 0 (0 for 0), elementwise (src/bitexact/intops.py:14-21)."""
    return _elem.elem(_elem.BITLEN, x)[0]


def rsh(x, s):
    """round(x / 2^s), ties up, for s > 0; x * 2^-s for s <= 0; s an int or an int64 tensor
    (src/bitexact/intops.py:24-33)."""
    return _elem.elem(_elem.RSH, x, s)[0]


def fdiv(a, b):
    """floor(a / b) for int64 a, b > 0 (src/bitexact/intops.py:36-38)."""
    return _elem.elem(_elem.FDIV, a, b)[0]


def rdiv(a, b):
    """round(a / b), ties up, for int64 a and b > 0, b may broadcast (src/bitexact/intops.py:41-43)."""
    return _elem.elem(_elem.RDIV, a, b)[0]


def isqrt(x):
    """floor(sqrt(x)) for int64 x >= 0, exact (src/bitexact/intops.py:46-52)."""
    return _elem.elem(_elem.ISQRT, x)[0]


def split_limbs(x, n):
    """Signed base-256 digits of x, least significant first: (n int64 tensors in [-128, 127], remainder)
    (src/bitexact/intops.py:62-70). The remainder is 0 iff |x| fits n digits."""
    planes, rem = _elem.elem(_elem.LIMBS, x, iarg=n)
    planes = planes.view(n, *x.shape)
    return [planes[i] for i in range(n)], rem


def stack_limbs(q, n):
    """q [M, K] within n limbs -> int8 [n M padded, K], limbs stacked along rows, padded with zero rows to >= 24
    rows and a multiple of 8 (src/bitexact/intops.py:73-79)."""
    M, K = q.shape
    rows = n * M
    pad_rows = max(24, (rows + 7) // 8 * 8)
    return _stack(q, n, pad_rows)


@op("stack_limbs(Tensor q, int n, int rows) -> Tensor", lambda q, n, rows: empty((rows, q.shape[1]), torch.int8, q))
def _stack(q, n, rows):
    _hip.require_cuda(q)
    M, K = q.shape
    out = torch.empty(rows, K, dtype=torch.int8, device=q.device)
    keep = []
    P, D = _elem._pack([q], (M, K), keep)
    _hip.call("bx_int_elementwise", _elem.LIMBS, 1, P, D, _hip.ptr(out), 1, None, 8, M, K, None, 0, n, rows * K, None,
              _hip.stream_of(q))
    return out


def join_limbs(c, M, n):
    """Rows [i M, (i + 1) M) of c hold the product of limb i: sum_i c_i 2^(8 i) as int64 [M, N]
    (src/bitexact/intops.py:82-87)."""
    return _elem.elem(_elem.JOIN, *[c[i * M:(i + 1) * M] for i in range(n)], iarg=n)[0]


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
