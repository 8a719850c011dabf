"""Exact-mode linear of the plugin (src/bitexact/vllm_plugin/exact_gemm.py:228-316) on one HIP launch.

FusedLin(lin)(q, sh, flag, checked=True) -> y int64 [M, N] at FR: the 9 limb products (MFMA), the ELL sparse
residual, wmm.epilogue's rounding and, when checked, flag[0] = 1 wherever the reference's checked epilogue
flags. Decode-sized M streams the weight planes once (split-K, one launch); prefill M uses LDS-tiled MFMA.
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op
from bitexact.exact.consts import FR


def needs_planes(M, N, K):
    """Whether the exact linear at this shape, given q's int8 limb planes, reads them (then a caller that can
    produce them, e.g. ops.add_norm_y(planes=True), should pass them as q_planes: no split launch, and at some
    narrow shapes a faster kernel than without them)."""
    return _hip.lib().bx_exact_linear_reads_planes(M, N, K) > 0


KERNELS = {1: "gemv", 2: "wide", 3: "tile", 5: "stream"}
TILES = {0: "128x128", 1: "64x128", 2: "64x32", 3: "64x64-int8", 4: "64x64", -1: None}


def plan(M, N, K, planes=False):
    """Which kernel the exact linear runs at (M, N, K) (planes: given q's limb planes): (kernel, tile, k_splits,
    blocks_per_split)."""
    import ctypes
    out = (ctypes.c_int32 * 4)()
    _hip.call("bx_exact_linear_planes_plan" if planes else "bx_exact_linear_plan", M, N, K, out)
    return KERNELS[out[0]], TILES[out[1]], out[2], out[3]


def _exact_linear_fake(q, sh, limbs, d, g, cnt, ec, ev, R, flag, checked, fr, q_planes):
    return empty((q.shape[0], limbs.shape[1]), torch.long, q)


@op("exact_linear(Tensor q, Tensor sh, Tensor limbs, Tensor d, Tensor g, Tensor? cnt, Tensor? ec, Tensor? ev, "
    "int R, Tensor(a!)? flag, bool checked, int fr, Tensor? q_planes) -> Tensor", _exact_linear_fake)
def _exact_linear(q, sh, limbs, d, g, cnt, ec, ev, R, flag, checked, fr, q_planes):
    _hip.require_cuda(q, limbs)
    assert q.dtype == torch.int32 and q.stride(1) == 1 and limbs.stride(2) == 1
    M, K = q.shape
    N = limbs.shape[1]
    assert limbs.shape[2] == K and sh.shape[0] == M
    if checked:
        assert flag is not None and flag.dtype == torch.int32
    y = torch.empty(M, N, dtype=torch.long, device=q.device)
    sh = sh.contiguous()
    if q_planes is not None:
        ws, wsb = _hip.workspace(q.device, _hip.lib().bx_exact_linear_planes_workspace(M, N, K))
        _hip.require_cuda(q_planes)
        assert q_planes.dtype == torch.int8 and q_planes.shape == (3, M, K) and q_planes.is_contiguous()
        _hip.call("bx_exact_linear_planes", _hip.ptr(q), q.stride(0), _hip.ptr(sh), _hip.ptr(limbs), limbs.stride(0),
                  limbs.stride(1), _hip.ptr(d), _hip.ptr(g), _hip.ptr(cnt) if R else None,
                  _hip.ptr(ec) if R else None, _hip.ptr(ev) if R else None, R, _hip.ptr(y), M, N, K, fr,
                  int(checked), _hip.ptr(flag), _hip.ptr(ws), wsb, _hip.ptr(q_planes), _hip.stream_of(q))
        return y
    ws, wsb = _hip.workspace(q.device, _hip.lib().bx_exact_linear_workspace(M, N, K))
    tmp, tmpb = _hip.scratch(q.device, _hip.lib().bx_exact_linear_scratch(M, N, K))
    _hip.call("bx_exact_linear", _hip.ptr(q), q.stride(0), _hip.ptr(sh), _hip.ptr(limbs), limbs.stride(0),
              limbs.stride(1), _hip.ptr(d), _hip.ptr(g), _hip.ptr(cnt) if R else None,
              _hip.ptr(ec) if R else None, _hip.ptr(ev) if R else None, R, _hip.ptr(y), M, N, K, fr, int(checked),
              _hip.ptr(flag), _hip.ptr(ws), wsb, _hip.ptr(tmp), tmpb, _hip.stream_of(q))
    return y


def exact_linear(q, sh, limbs, d, g, cnt, ec, ev, R, flag=None, checked=True, fr=FR, q_planes=None):
    """The fused exact linear on raw tensors; returns y (and sets flag). q_planes: q's int8 limb planes [3, M, K]."""
    return _exact_linear(q, sh, limbs, d, g, cnt, ec, ev, int(R), flag, bool(checked), int(fr), q_planes)


class FusedLin:
    """The linear layer `lin` (bitexact.exact.model.Lin) as one fused HIP call: q int32 [M, K], sh int64 [M]
    -> y int64 [M, N] at FR; sets flag (int32 [1]) to 1 when wmm.epilogue's checked condition holds."""

    def __init__(self, lin, cfg=None):
        self.limbs, self.d, self.g, self.N = lin.limbs, lin.d, lin.g, lin.N
        self.cnt, self.ec, self.ev, self.R = lin.cnt, lin.ec, lin.ev, lin.R
        self.has_res = self.R > 0
        self.cfg = cfg               # kept for signature parity; tiles never change the integers

    def __call__(self, q, sh, flag, checked=True, q_planes=None):
        return exact_linear(q, sh, self.limbs, self.d, self.g, self.cnt, self.ec, self.ev, self.R, flag, checked,
                            q_planes=q_planes)

    def needs_planes(self, M):
        return needs_planes(M, self.N, self.limbs.shape[2])
