"""The element-wise integer rules and row reductions of the reference's Python helpers on HIP (bx_int_elementwise,
bx_int_rowop in csrc/bx_elem.hip), as two registered operators: bitexact_hip::int_elem and bitexact_hip::int_row.

Operands broadcast as torch does: each tensor operand is expanded to the output shape and passed as a strided
view (no copy unless its leading dimensions cannot be addressed as one row index), Python ints travel as
constants. Outputs are int64 tensors of the broadcast shape. Device tensors only: there is no CPU path.
"""

import ctypes

import torch

from bitexact import _hip
from bitexact._ops import op

# element-wise rules (csrc/bx_elem.hip ElemOp)
BITLEN, RSH, RSHC, FDIV, RDIV, ISQRT, DIVROUND, COMBINE, SHRHL, EXP2NEG, SILU_MUL, EXP_OF, SILU8, NORM24, MULSUB, \
    MULADD, ABSFLAG, LIMBS, JOIN, ADD, SUB, MUL, SHIFT, NDIV, PRODGE, MUL_RSH, RDIVSH, GTFLAG = range(1, 29)
# row rules (csrc/bx_elem.hip RowOp)
R_QUANT, R_RMS, R_RMS8, R_SOFTMAX_W, R_SOFTMAX8, R_QROWS8, R_PRENORM8, R_AMAX = range(1, 9)

_TWO_OUT = (COMBINE, NORM24)
_NO_OUT = (PRODGE, ABSFLAG, GTFLAG)


def _bshape(ins):
    shapes = [t.shape for t in ins if torch.is_tensor(t)]
    return tuple(torch.broadcast_shapes(*shapes)) if shapes else ()


def _grid(shape):
    inner = shape[-1] if len(shape) else 1
    rows = 1
    for s in shape[:-1]:
        rows *= s
    return rows, inner


def _operand(x, shape, keep):
    """(pointer, [srow, scol, imm, bytes]) of operand x over the [rows, inner] grid of `shape`."""
    if not torch.is_tensor(x):
        return None, [0, 0, int(x), 8]
    _hip.require_cuda(x)
    assert not x.is_floating_point() and not x.is_complex(), "integer tensors only"
    rows, inner = _grid(shape)
    e = x.expand(shape) if len(shape) else x.reshape(())
    try:
        v = e.view(rows, inner)
    except RuntimeError:
        v = e.contiguous().view(rows, inner)
    keep.append(v)
    return ctypes.c_void_p(v.data_ptr()), [v.stride(0), v.stride(1), 0, v.element_size()]


def _pack(ins, shape, keep):
    ptrs, desc = [], []
    for x in ins:
        p, d = _operand(x, shape, keep)
        ptrs.append(p)
        desc.extend(d)
    P = (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
    D = (ctypes.c_int64 * max(1, len(desc)))(*desc)
    return P, D


def _dev(ins):
    for t in ins:
        if torch.is_tensor(t):
            return t.device
    raise AssertionError("at least one operand must be a device tensor")


def _outs_elem(code, shape, iarg, iarg2, dev):
    if code in _NO_OUT:
        return []
    if code == LIMBS:
        n = 1
        for s in shape:
            n *= s
        tot = max(iarg * n, iarg2)
        return [torch.empty(tot, dtype=torch.int64, device=dev), torch.empty(shape, dtype=torch.int64, device=dev)]
    k = 2 if code in _TWO_OUT else 1
    return [torch.empty(shape, dtype=torch.int64, device=dev) for _ in range(k)]


def _pad(outs, n, dev):
    """A fixed number of outputs (the operator returns a tuple): empty placeholders past the rule's own."""
    return tuple(outs) + tuple(torch.empty(0, dtype=torch.int64, device=dev) for _ in range(n - len(outs)))


def _elem_fake(code, ins, imms, lut, iarg, iarg2, flag):
    vals = [t if t is not None else 0 for t in ins]
    dev = _dev(vals)
    return _pad(_outs_elem(code, _bshape(vals), iarg, iarg2, dev), 2, dev)


@op("int_elem(int code, Tensor?[] ins, int[] imms, Tensor? lut, int iarg, int iarg2, Tensor(a!)? flag) -> "
    "(Tensor, Tensor)", _elem_fake)
def _int_elem(code, ins, imms, lut, iarg, iarg2, flag):
    vals = [t if t is not None else imms[j] for j, t in enumerate(ins)]
    shape = _bshape(vals)
    dev = _dev(vals)
    keep = []
    P, D = _pack(vals, shape, keep)
    outs = _outs_elem(code, shape, iarg, iarg2, dev)
    rows, inner = _grid(shape)
    lut_c = None
    if lut is not None:
        _hip.require_cuda(lut)
        lut_c = lut.contiguous().long()
        keep.append(lut_c)
    o0 = outs[0] if outs else None
    o1 = outs[1] if len(outs) > 1 else None
    _hip.call("bx_int_elementwise", code, len(vals), P, D, _hip.ptr(o0), 8, _hip.ptr(o1), 8, rows, inner,
              _hip.ptr(lut_c), 0 if lut_c is None else lut_c.numel(), iarg, iarg2, _hip.ptr(flag),
              _hip.stream_of(o0 if o0 is not None else lut_c if lut_c is not None else flag))
    return _pad(outs, 2, dev)


def elem(code, *ins, lut=None, iarg=0, iarg2=0, flag=None):
    """One element-wise rule over broadcast operands (tensors or Python ints) -> list of int64 outputs."""
    ts = [x if torch.is_tensor(x) else None for x in ins]
    imms = [0 if torch.is_tensor(x) else int(x) for x in ins]
    outs = _int_elem(code, ts, imms, lut, int(iarg), int(iarg2), flag)
    return list(outs[:0 if code in _NO_OUT else 2 if code in _TWO_OUT or code == LIMBS else 1])


def flag_for(dev, flag=None):
    """The caller's int32 [1] device flag, or a fresh zero one."""
    if flag is not None:
        assert flag.dtype == torch.int32 and flag.is_cuda
        return flag
    return torch.zeros(1, dtype=torch.int32, device=dev)


def _row_outs(code, rows, D, nl, want_q, want_limbs, dev):
    e = lambda *s: torch.empty(s, dtype=torch.int64, device=dev)
    if code == R_QUANT:
        return [e(rows, D), e(rows)]
    if code in (R_RMS, R_RMS8):
        return [e(rows), e(rows)]
    if code in (R_SOFTMAX_W, R_SOFTMAX8):
        return [e(rows, D), e(rows)]
    if code == R_AMAX:
        return [e(rows)]
    limbs = torch.empty(nl * rows if want_limbs else 0, D, dtype=torch.int8, device=dev)
    q = e(rows, D) if want_q else e(0, D)
    return [q, e(rows), e(rows), limbs]


def _row_fake(code, x, ins, imms, lut, ia, flag, want_q, want_limbs):
    rows = x.shape[0]
    return _pad(_row_outs(code, rows, x.shape[1], ia[0] if ia else 1, want_q, want_limbs, x.device), 4, x.device)


@op("int_row(int code, Tensor x, Tensor?[] ins, int[] imms, Tensor? lut, int[] ia, Tensor(a!)? flag, bool want_q, "
    "bool want_limbs) -> (Tensor, Tensor, Tensor, Tensor)", _row_fake)
def _int_row(code, x, ins, imms, lut, ia, flag, want_q, want_limbs):
    _hip.require_cuda(x)
    assert x.dtype == torch.int64 and x.dim() == 2, "int64 [rows, D]"
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, D = x.shape
    vals = [t if t is not None else imms[j] for j, t in enumerate(ins)]
    keep = []
    P, Dd = _pack(vals, (rows, D), keep)
    outs = _row_outs(code, rows, D, ia[0] if ia else 1, want_q, want_limbs, x.device)
    lut_c = None
    if lut is not None:
        lut_c = lut.contiguous().long()
        keep.append(lut_c)
    iargs = (ctypes.c_int64 * 6)(*(list(ia) + [0] * (6 - len(ia))))
    o = [(_hip.ptr(t) if t is not None and t.numel() > 0 else None) for t in outs] + [None] * (4 - len(outs))
    _hip.call("bx_int_rowop", code, len(vals), P, Dd, _hip.ptr(x), x.stride(0), rows, D, o[0], o[1], o[2], o[3],
              _hip.ptr(lut_c), 0 if lut_c is None else lut_c.numel(), iargs, _hip.ptr(flag), _hip.stream_of(x))
    return _pad(outs, 4, x.device)


def row(code, x, *ins, lut=None, ia=(), flag=None, want_q=True, want_limbs=False):
    """One row rule over x int64 [rows, D] (operands broadcast to [rows, D]) -> list of outputs."""
    ts = [t if torch.is_tensor(t) else None for t in ins]
    imms = [0 if torch.is_tensor(t) else int(t) for t in ins]
    outs = _int_row(code, x, ts, imms, lut, [int(v) for v in ia], flag, bool(want_q), bool(want_limbs))
    n = 1 if code == R_AMAX else 2 if code in (R_QUANT, R_RMS, R_RMS8, R_SOFTMAX_W, R_SOFTMAX8) else 4
    return list(outs[:n])
