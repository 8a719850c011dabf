"""Exact-mode linear of the plugin (src/bitexact/vllm_plugin/exact_gemm.py:228-316) on one HIP launch.

FusedLin(lin)(q, sh, flag, checked=True) -> y int64 [M, N] at FR: the 9 limb products (MFMA), the ELL sparse
residual, wmm.epilogue's rounding and, when checked, flag[0] = 1 wherever the reference's checked epilogue
flags. Decode-sized M streams the weight planes once (split-K, one launch); prefill M uses LDS-tiled MFMA.
"""

import torch

from bitexact import _hip
from bitexact.exact.consts import FR


def exact_linear(q, sh, limbs, d, g, cnt, ec, ev, R, flag=None, checked=True, fr=FR):
    """The fused exact linear on raw tensors; returns y (and sets flag)."""
    _hip.require_cuda(q, limbs)
    assert q.dtype == torch.int32 and q.stride(1) == 1 and limbs.stride(2) == 1
    M, K = q.shape
    N = limbs.shape[1]
    assert limbs.shape[2] == K and sh.shape[0] == M
    if checked:
        assert flag is not None and flag.dtype == torch.int32
    y = torch.empty(M, N, dtype=torch.long, device=q.device)
    ws, wsb = _hip.workspace(q.device, _hip.lib().bx_exact_linear_workspace(M, N, K))
    tmp, tmpb = _hip.scratch(q.device, _hip.lib().bx_exact_linear_scratch(M, N, K))
    sh = sh.contiguous()
    _hip.call("bx_exact_linear", _hip.ptr(q), q.stride(0), _hip.ptr(sh), _hip.ptr(limbs), limbs.stride(0),
              limbs.stride(1), _hip.ptr(d), _hip.ptr(g), _hip.ptr(cnt) if R else None,
              _hip.ptr(ec) if R else None, _hip.ptr(ev) if R else None, R, _hip.ptr(y), M, N, K, fr, int(checked),
              _hip.ptr(flag), _hip.ptr(ws), wsb, _hip.ptr(tmp), tmpb, _hip.stream_of(q))
    return y


class FusedLin:
    """The linear layer `lin` (bitexact.exact.model.Lin) as one fused HIP call: q int32 [M, K], sh int64 [M]
    -> y int64 [M, N] at FR; sets flag (int32 [1]) to 1 when wmm.epilogue's checked condition holds."""

    def __init__(self, lin, cfg=None):
        self.limbs, self.d, self.g, self.N = lin.limbs, lin.d, lin.g, lin.N
        self.cnt, self.ec, self.ev, self.R = lin.cnt, lin.ec, lin.ev, lin.R
        self.has_res = self.R > 0
        self.cfg = cfg               # kept for signature parity; tiles never change the integers

    def __call__(self, q, sh, flag, checked=True):
        return exact_linear(q, sh, self.limbs, self.d, self.g, self.cnt, self.ec, self.ev, self.R, flag, checked)
