"""Element-wise segments of the exact engine between its matrix products (src/bitexact/exact/segs.py), each a
HIP launch: the reference's stage names and the Segs class with its method signatures.

A linear output is produced from C (the exact dense products, [split, M, N] or [M, N]) and the sparse residual
rs = (B,) (dense) or rs = (q, ell_c, ell_v) (padded per-row lists), as the reference's lin_y takes them; the
fused stages (RMSNorm + quantization, RoPE + q quantization + regroup, SiLU gating + quantization, attention
division + quantization) are one kernel each and give the reference's integers. Bound violations or into the
bool `err` tensor exactly where the reference's stages or them.

Segs(compiled=True) wraps each method in torch.compile (fullgraph, backend "aot_eager"): every kernel is a
registered torch.ops.bitexact_hip operator with a fake implementation, so the trace has no graph break; the
integers are the same either way.
"""

import torch

from bitexact import _elem
from bitexact.exact import ops
from bitexact.exact import wmm
from bitexact.exact.consts import FR, LIM3

H, HKV, HD = 32, 8, 64                                      # Llama-3.2-1B attention geometry (default dm)
FK, FV, FP = ops.FK, ops.FV, ops.FP


# ---- stages (src/bitexact/exact/segs.py:25-132) ----
def lin_y(C, rs, d, g, sh, checked=False):
    """The linear output at FR from the split partials C and the residual rs (segs.py:25-32)."""
    return wmm.lin_y(C, rs, d, g, sh, checked=checked, FR=FR)


def add_y(y, x):
    """x + y (segs.py:40-41) as a new tensor of x's shape."""
    out = x.reshape(-1, x.shape[-1]).clone()
    ops.add_norm_y(y.reshape(out.shape), out, None, None)
    return out.view(x.shape)


def lin_add(C, rs, d, g, sh, x):
    """(x + lin_y(...), flag) (segs.py:35-37)."""
    y, flag = lin_y(C, rs, d, g, sh, checked=True)
    return add_y(y, x), flag


def norm_quant(x, gm, ge, err):
    """RMSNorm + division by the rms + quantization at -FN (segs.py:59-63) -> (q int32, sh, err)."""
    return ops.norm_quant(x, gm, ge, err)


def softmax(raw, qpos, shg, lut, l2e):
    """Masked integer softmax weights at FP (segs.py:102-105) -> (p int32, den)."""
    return ops.softmax(raw, qpos, shg, lut, l2e)


def qkv_y(y, pos, cos, sin, B, T, dm, err):
    """rope_y + q_group (segs.py:78-99) from the qkv linear's output -> (qg, shg, k, v, err)."""
    return ops.qkv_y(y.reshape(B * T, -1), pos, cos, sin, B, T, dm, err)


def gu_silu_y(y, lut, err):
    """silu_y + quant_silu (segs.py:120-132) -> (q int32, sh, err)."""
    return ops.gu_silu_y(y, lut, err)


def attn_out(num, den, T, hkv):
    """attn_div + quant(., -FR) (segs.py:108-113, 187-188) -> (q int32 [B T, H HD], sh)."""
    return ops.attn_out(num, den, T, hkv)


def rms(x, err):
    """ops.rms plus the |x| < 2^40 bound (segs.py:44-46) -> (r, er, err)."""
    r, er = ops.rms(x)
    fl = _elem.flag_for(x.device)
    _elem.elem(_elem.ABSFLAG, x, iarg=(1 << 40) - 1, flag=fl)
    return r, er, err | (fl[0] != 0)


def ndiv(x, gm, ge, r, er):
    """x gamma / rms at FN, one rounding per element (segs.py:49-51)."""
    return _elem.elem(_elem.NDIV, x, gm, r[:, None], ge, er[:, None], iarg=ops.FN - FR)[0]


def quant(P, eps):
    """ops.quant with q as int32 (segs.py:54-56)."""
    q, sh = ops.quant(P, eps)
    return q.to(torch.int32), sh


def _rope_full(x, c, s, shift=0):
    """(x1 c - x2 s, x2 c + x1 s) over the two halves of the last axis, each rounded by `shift` bits (segs.py:66-69
    with the caller's rshc)."""
    hd = x.shape[-1]
    x1, x2 = x[..., :hd // 2], x[..., hd // 2:]
    lo = _elem.elem(_elem.MULSUB, x1, c, x2, s, iarg=shift)[0]
    hi = _elem.elem(_elem.MULADD, x2, c, x1, s, iarg=shift)[0]
    return torch.cat([lo, hi], -1)


def rope_y(y, pos, cos, sin, B, T, dm):
    """The qkv linear's output y [B T, (H + 2 HKV) HD] at FR -> (Pq at FR + FT [B, T, H, HD], k at FK, v at FV
    [B, T, HKV, HD], y [B, T, .]) (segs.py:78-86)."""
    h, hkv, hd = dm
    y = y.view(B, T, -1)
    c, s = cos[pos][:, :, None], sin[pos][:, :, None]
    Pq = _rope_full(y[..., :h * hd].reshape(B, T, h, hd), c, s)
    k = _rope_full(y[..., h * hd:(h + hkv) * hd].reshape(B, T, hkv, hd), c, s, FR + ops.FT - FK)
    v = ops.rshc(y[..., (h + hkv) * hd:].reshape(B, T, hkv, hd), FR - FV)
    return Pq, k, v, y


def lin_rope(C, rs, d, g, sh, pos, cos, sin, B, T, dm):
    """qkv linear + RoPE (segs.py:72-75)."""
    return rope_y(lin_y(C, rs, d, g, sh), pos, cos, sin, B, T, dm)


def q_group(Pq, k, v, y, err):
    """q quantized per (token, head) and grouped by KV head -> ([B HKV, g T, HD] int32, exponents [.., 1], err)
    (segs.py:89-99)."""
    B, T, h, hd = Pq.shape
    hkv = k.shape[2]
    qi, shq = ops.quant(Pq, -(FR + ops.FT))
    g = h // hkv
    qg = qi.view(B, T, hkv, g, hd).permute(0, 2, 3, 1, 4).reshape(B * hkv, g * T, hd).to(torch.int32)
    shg = shq.view(B, T, hkv, g).permute(0, 2, 3, 1).reshape(B * hkv, g * T, 1)
    fl = _elem.flag_for(Pq.device)
    _elem.elem(_elem.ABSFLAG, y, iarg=(1 << 31) - 1, flag=fl)
    _elem.elem(_elem.ABSFLAG, k, iarg=LIM3, flag=fl)
    _elem.elem(_elem.ABSFLAG, v, iarg=LIM3, flag=fl)
    _elem.elem(_elem.GTFLAG, shq, iarg=FK + 3 - ops.FZ, flag=fl)
    return qg, shg, err | (fl[0] != 0)


def attn_div(num, den, T, hkv):
    """num [B HKV, g T, HD] at FV + FP, den [B HKV, g T, 1] -> o at FR [B T, H HD], one rounding (segs.py:108-113)."""
    Z, gT, hd = num.shape
    B, g = Z // hkv, gT // T
    o = ops.div_round(num, FR - FV, den)
    return o.view(B, hkv, g, T, hd).permute(0, 3, 1, 2, 4).reshape(B * T, hkv * g * hd)


def silu_y(gu, lut):
    """silu(gate) up at 2 FR from gu = [gate | up] (segs.py:120-123) -> (P, ok)."""
    ff = gu.shape[1] // 2
    P, _, ok = ops.silu_mul(gu[:, :ff], gu[:, ff:], lut)
    return P, ok


def lin_silu(C, rs, d, g, sh, lut):
    """gate|up linear + silu_y (segs.py:116-117)."""
    return silu_y(lin_y(C, rs, d, g, sh), lut)


def quant_silu(P, ok, err):
    """quantization of the gated product at -2 FR (segs.py:126-128) -> (q int32, sh, err)."""
    q, sh = ops.quant(P, -2 * FR)
    return q.to(torch.int32), sh, err | ~ok


# the reference's stage table (segs.py:131-132); Segs.s binds them (compiled or not)
STAGES = ("lin_y", "lin_add", "rms", "ndiv", "quant", "lin_rope", "q_group", "softmax", "attn_div",
          "lin_silu", "quant_silu", "rope_y", "add_y", "silu_y", "norm_quant")


class Segs:
    """The reference's stage set (src/bitexact/exact/segs.py:135-192) with its method signatures."""

    METHODS = ("norm_q", "pre_norm", "lin_out", "add_norm", "qkv", "qkv_y", "add_norm_y", "gu_silu_y", "softmax",
               "attn_out", "gu_silu")

    def __init__(self, compiled=False, dm=(H, HKV, HD), one_region=False):
        self.dm = tuple(int(v) for v in dm)
        self.one_region = one_region            # the norm is one kernel either way
        self.l2e = ops.L2E28_HD[self.dm[2]]     # KeyError: unsupported head_dim
        self.compiled = compiled
        if compiled:
            import torch._dynamo
            torch._dynamo.config.cache_size_limit = max(torch._dynamo.config.cache_size_limit, 64)
            for name in self.METHODS:
                setattr(self, name, torch.compile(getattr(self, name), fullgraph=True, backend="aot_eager"))
        # the reference's per-stage table (segs.py:140-146); compiled stages trace through the registered operators
        wrap = (lambda f: torch.compile(f, backend="aot_eager")) if compiled else (lambda f: f)
        self.s = type("S", (), {n: staticmethod(wrap(globals()[n])) for n in STAGES})

    def norm_q(self, x, gm, ge, err):
        return norm_quant(x, gm, ge, err)

    def pre_norm(self, x, gm, ge):
        q, sh, _ = norm_quant(x, gm, ge, torch.zeros((), dtype=torch.bool, device=x.device))
        return q, sh

    def lin_out(self, C, rs, d, g, sh):
        return lin_y(C, rs, d, g, sh, True)

    def add_norm(self, C, rs, d, g, sh, x, gm, ge, err):
        y, flag = lin_y(C, rs, d, g, sh, True)
        return self.add_norm_y(y, x, gm, ge, err | flag)

    def qkv(self, C, rs, d, g, sh, pos, cos, sin, B, T, err):
        return self.qkv_y(lin_y(C, rs, d, g, sh), pos, cos, sin, B, T, err)

    def qkv_y(self, y, pos, cos, sin, B, T, err):
        return qkv_y(y, pos, cos, sin, B, T, self.dm, err)

    def add_norm_y(self, y, x, gm, ge, err):
        D = x.shape[-1]
        x2 = x.reshape(-1, D).clone()           # the reference's x + y is a new tensor
        x2, q, s, err = ops.add_norm_y(y.reshape(-1, D), x2, gm, ge, err)
        return x2.view(x.shape), q, s, err

    def gu_silu_y(self, y, lut, err):
        return gu_silu_y(y, lut, err)

    def softmax(self, raw, qpos, shg, lut):
        return softmax(raw, qpos, shg, lut, self.l2e)

    def attn_out(self, num, den, T):
        return attn_out(num, den, T, self.dm[1])

    def gu_silu(self, C, rs, d, g, sh, lut, err):
        return gu_silu_y(lin_y(C, rs, d, g, sh), lut, err)
