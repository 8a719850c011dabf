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

from bitexact.exact import ops
from bitexact.exact import wmm
from bitexact.exact.consts import FR

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


STAGES = ("lin_y", "lin_add", "add_y", "norm_quant", "softmax", "qkv_y", "gu_silu_y", "attn_out")


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
