"""Integer primitives of the int8 engine (src/bitexact/int8/ops.py) on HIP.

The reference's names and contracts; every rule runs as an element-wise or row kernel of csrc/bx_elem.hip (or the
int8 MFMA GEMM for imm), so the integers equal the reference's CPU tensors'. Device tensors only.
"""

import torch

from bitexact import _elem
from bitexact.int8.consts import EXP_MIN, FA, FG, FR, SILU_LIM
from bitexact.intops import isqrt, rdiv, rsh  # noqa: F401  (the reference module re-exports these names)

EXACT = 1 << 53
EPS40 = 10995116         # round(1e-5 2^40): RMSNorm eps


def qmax(nl):
    return 127 << (8 * (nl - 1))


def quant_rows(z, nl):
    """Per-row quantization of int64 z [M, K] to |q| <= qmax(nl) -> (q, as_, sh): amax brought to 30 bits by sh,
    q = round(rsh(z, sh) qmax / as_) (src/bitexact/int8/ops.py:24-35)."""
    q, as_, sh, _ = _elem.row(_elem.R_QROWS8, z, ia=(nl,))
    return q, as_, sh


def bitlen32(x):
    """intops.bitlen's integers (src/bitexact/int8/ops.py:38-44: the reference's float32 route to them)."""
    return _elem.elem(_elem.BITLEN, x)[0]


def rdiv32(a, b):
    """rdiv's integers where the reference's float32 route is exact (src/bitexact/int8/ops.py:47-55)."""
    return _elem.elem(_elem.RDIV, a, b)[0]


def post_bound(w, m, fmsh, nl):
    """Largest |t| = |rsh(acc m_c, fmsh)| over every input of a linear layer, a Python int
    (src/bitexact/int8/ops.py:58-67): |t_c| <= rsh(qmax(nl) l1_c |m_c|, fmsh), l1_c = sum_k |W_ck|. Load time."""
    l1 = w.long().abs().sum(1)
    assert int(l1.max()) < 1 << 24 and int(m.abs().max()) < 1 << 36       # l1 |m| < 2^60 in int64
    a = qmax(nl) * int((l1 * m.abs()).max())
    return (a + (1 << (fmsh - 1))) >> fmsh if fmsh > 0 else a << -fmsh


def norm24(mant, e):
    """(mant, e) with value mant 2^e -> the same value with mant in [2^23, 2^24], rounded
    (src/bitexact/int8/ops.py:70-73)."""
    m2, e2 = _elem.elem(_elem.NORM24, mant, e)
    return m2, e2


def rms(x):
    """RMS of each row of x at FR bits as (r, shx): value r 2^(shx - FR), r >= 17 bits (src/bitexact/int8/ops.py:76-84)."""
    r, shx = _elem.row(_elem.R_RMS8, x, ia=(FR,))
    return r, shx


def imm(q, w64):
    """Exact q @ W^T: q int64 [M, K] with |q| <= qmax(3), w64 = W^T [K, N] with integer entries |W| <= 127
    (src/bitexact/int8/ops.py:87-90). On the device: q's 3 signed limbs through the int8 MFMA GEMM, joined in int64
    (the reference's float64 product, exact by its bound, has the same integers)."""
    from bitexact.int8.gemm_skinny import int_mm_join
    from bitexact.intops import stack_limbs
    M = q.shape[0]
    w = w64.t().to(torch.int8).contiguous()
    a = stack_limbs(q, 3)
    return int_mm_join(a, w, M, 3)


def exp_of(z, lut):
    """e^z at FE bits for z <= 0 at FA bits; 0 below EXP_MIN (src/bitexact/int8/ops.py:93-97)."""
    return _elem.elem(_elem.EXP_OF, z, lut=lut, iarg=EXP_MIN << FA)[0]


def silu(g, lut):
    """SiLU at FR bits from the table at step 2^-FA, linear interpolation between entries
    (src/bitexact/int8/ops.py:100-108)."""
    return _elem.elem(_elem.SILU8, g, lut=lut, iarg=FR - FA, iarg2=SILU_LIM << FA)[0]


__all__ = ["EXACT", "EPS40", "FG", "qmax", "quant_rows", "bitlen32", "rdiv32", "post_bound", "norm24", "rms", "imm",
           "exp_of", "silu"]
