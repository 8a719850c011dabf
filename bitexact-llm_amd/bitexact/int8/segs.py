"""Element-wise segments of the int8 engine between its matrix products (src/bitexact/int8/segs.py) on HIP.

Module-level stages follow the reference's contracts (q unstacked, int64):
  pre_norm(x, gamma, nl) -> (q, mant, e)        RMSNorm + per-row quantization and the row scale
  pre_plain(x, nl)       -> (q, mant, e)
  post(acc, m, fmsh, mant, e, check=True) -> (y at FR, flag)
  qkv(y, c, s, dm)       -> (qg, k, v, flag)     RoPE at FT + regroup by KV head
  softmax(raw, qpos, expt, hd) -> (p, den)       masked table softmax weights at FP
  attn_out(num, den, T, nl, dm) -> (q, mant, e)  rdiv + regroup + pre_plain
  silu_mul(gu, lut, nl)  -> (q, mant, e, flag)
Segs(nl, cuda, compiled, post_check, dm) binds them as the reference does: on the device the pre-segments return
the limbs stacked along rows (intops.stack_limbs) and the post-segments join the limb products first; compiled=True
traces each through the registered operators (torch.compile with the aot_eager backend: no generated kernels).
quant_rows_limbs / pre_plain_limbs are the one-launch stacked forms the int8 GEMM reads (limb i of row m at row
i M + m, no padding rows). Device tensors only.
"""

import torch

from bitexact import _elem, _hip
from bitexact._ops import empty, op
from bitexact.int8 import ops
from bitexact.int8.consts import FA, FE, FG, FR, FT
from bitexact.intops import LIM, join_limbs, stack_limbs

H, HKV, HD = 32, 8, 64                                      # Llama-3.2-1B attention geometry (default dm)
FQ, FV, FP = 14, 14, 20                                     # q / k, v, attention weights (fractional bits)
NEG = -(1 << 62)
# head_dim 128's score scale 2^-1/2 as an integer (src/bitexact/int8/segs.py:26-31)
SC128 = 11863283
ZCLAMP = -(1 << 38)


def score_rule(hd):
    """(mul, zsh): z = rsh(d, zsh) when mul is None, else rsh(max(d, ZCLAMP) mul, zsh) (src/bitexact/int8/segs.py:36-44)."""
    base = 2 * FQ + 3 - FA
    if hd == 64:
        return None, base
    if hd == 128:
        return SC128, base + 24
    raise ValueError(f"unsupported head_dim {hd}")


def _amax_all(z):
    """max |z| over the whole tensor as a device int64 [1] (two row reductions)."""
    z2 = z.reshape(z.shape[0], -1) if z.dim() > 1 else z.reshape(1, -1)
    per = _elem.row(_elem.R_AMAX, z2.contiguous() if z2.stride(-1) != 1 else z2)[0]
    return _elem.row(_elem.R_AMAX, per.view(1, -1))[0]


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


def quant_rows_limbs(z, nl):
    """ops.quant_rows (src/bitexact/int8/ops.py:24-35) with the limbs stacked (src/bitexact/intops.py:73-79, no
    padding rows), one launch -> (a int8 [nl M, K], as_, sh)."""
    a, as_, sh, _, _ = _quant(z, nl, False)
    return a, as_, sh


def pre_plain_limbs(x, nl):
    """segs.pre_plain (src/bitexact/int8/segs.py:56-59) with the limbs stacked, one launch -> (a, mant, e)."""
    a, _, _, mant, e = _quant(x, nl, True)
    return a, mant, e


def pre_norm(x, gamma, nl):
    """RMSNorm + per-row quantization (src/bitexact/int8/segs.py:47-52): x int64 [M, D] at FR, gamma [D] at FG ->
    (q, mant, e), the row scale amax(x gamma) / rms(x) as mant 2^e."""
    q, mant, e, _ = _elem.row(_elem.R_PRENORM8, x, gamma, ia=(nl, FR, FG))
    return q, mant, e


def pre_plain(x, nl):
    """Per-row quantization and the row scale norm24(as_, sh - FR) (src/bitexact/int8/segs.py:56-59) -> (q, mant, e)."""
    q, as_, sh = ops.quant_rows(x, nl)
    mant, e = ops.norm24(as_, _elem.elem(_elem.SUB, sh, FR)[0])
    return q, mant, e


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


def _rope(x, c, s):
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    sh = FT + FR - FQ
    return torch.cat([_elem.elem(_elem.MULSUB, x1, c, x2, s, iarg=sh)[0],
                      _elem.elem(_elem.MULADD, x2, c, x1, s, iarg=sh)[0]], -1)


def qkv(y, c, s, dm=(H, HKV, HD)):
    """y [B, T, (H + 2 HKV) HD] at FR, c / s [B, T, 1, HD / 2] -> grouped q [B HKV, g T, HD], k, v [B, T, HKV, HD],
    flag (src/bitexact/int8/segs.py:77-87)."""
    H_, HKV_, HD_ = dm
    B, T = y.shape[0], y.shape[1]
    D = H_ * HD_
    q = _rope(y[..., :D].reshape(B, T, H_, HD_), c, s)
    k = _rope(y[..., D:D + HKV_ * HD_].reshape(B, T, HKV_, HD_), c, s)
    v = _elem.elem(_elem.RSH, y[..., D + HKV_ * HD_:].reshape(B, T, HKV_, HD_), FR - FV)[0]
    g = H_ // HKV_
    qg = q.view(B, T, HKV_, g, HD_).permute(0, 2, 3, 1, 4).reshape(B * HKV_, g * T, HD_)
    fl = _elem.flag_for(y.device)
    for t in (q, k, v):
        _elem.elem(_elem.ABSFLAG, t, iarg=LIM[3], flag=fl)
    return qg, k, v, fl[0] != 0


def softmax(raw, qpos, expt, hd=HD):
    """raw [B, HKV, gT, S] q.k at 2 FQ, qpos [B, 1, gT, 1] -> weights p at FP (masked: 0), sums [.., 1]
    (src/bitexact/int8/segs.py:90-99)."""
    S = raw.shape[-1]
    lead = raw.shape[:-1]
    r2 = raw.reshape(-1, S)
    qp = qpos.expand(*lead, 1).reshape(-1, 1)
    mul, zsh = score_rule(hd)
    p, den = _elem.row(_elem.R_SOFTMAX8, r2, qp, lut=expt, ia=(0 if mul is None else mul, zsh, FE - FP, -32 << FA))
    return p.view(raw.shape), den.view(*lead, 1)


def attn_out(num, den, T, nl, dm=(H, HKV, HD)):
    """num [B, HKV, gT, HD], den [B, HKV, gT, 1] -> quantized o [B T, H HD] for o_proj (src/bitexact/int8/segs.py:102-109)."""
    H_, HKV_, HD_ = dm
    B = num.shape[0]
    g = H_ // HKV_
    o = _elem.elem(_elem.RDIVSH, num, den, iarg=FR - FV)[0]
    o = o.view(B, HKV_, g, T, HD_).permute(0, 3, 1, 2, 4).reshape(B * T, H_ * HD_)
    return pre_plain(o, nl)


def silu_mul(gu, lut, nl):
    """SiLU(gate) up with the magnitude flag and the row quantization (src/bitexact/int8/segs.py:112-118)
    -> (q, mant, e, flag)."""
    ff = gu.shape[1] // 2
    g, u = gu[:, :ff], gu[:, ff:]
    sg = ops.silu(g, lut)
    fl = _elem.flag_for(gu.device)
    _elem.elem(_elem.PRODGE, _amax_all(sg), _amax_all(u), iarg=62, flag=fl)
    q, mant, e = pre_plain(_elem.elem(_elem.MUL_RSH, sg, u, iarg=FR)[0], nl)
    return q, mant, e, fl[0] != 0


def _add(out, x):
    y, flag = out
    return _elem.elem(_elem.ADD, x, y.view(x.shape))[0], flag


class Segs:
    """The reference's int8 stage set (src/bitexact/int8/segs.py:121-139)."""

    def __init__(self, nl, cuda, compiled, post_check=True, dm=(H, HKV, HD)):
        wrap = (lambda f: torch.compile(f, dynamic=None, backend="aot_eager")) if compiled else (lambda f: f)
        lim = (lambda q: stack_limbs(q, nl)) if cuda else (lambda q: q)
        join = (lambda c, M: join_limbs(c, M, nl)) if cuda else (lambda c, M: c)

        def with_limbs(out):
            return (lim(out[0]),) + tuple(out[1:])

        self.nl, self.dm = nl, tuple(dm)
        self.pre_norm = wrap(lambda x, gamma: with_limbs(pre_norm(x, gamma, nl)))
        self.pre_plain = wrap(lambda x: with_limbs(pre_plain(x, nl)))
        self.post = wrap(lambda c, m, fmsh, mant, e: post(join(c, mant.shape[0]), m, fmsh, mant, e, post_check))
        self.post_add = wrap(lambda c, m, fmsh, mant, e, x: _add(post(join(c, mant.shape[0]), m, fmsh, mant, e,
                                                                      post_check), x))
        self.qkv = wrap(lambda y, c, s: qkv(y, c, s, dm))
        self.softmax = wrap(lambda raw, qpos, expt: softmax(raw, qpos, expt, dm[2]))
        self.attn_out = wrap(lambda num, den, T: with_limbs(attn_out(num, den, T, nl, dm)))
        self.silu_mul = wrap(lambda gu, lut: with_limbs(silu_mul(gu, lut, nl)))
