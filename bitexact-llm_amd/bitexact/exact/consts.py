"""Exact-mode weight format and tables (src/bitexact/exact/consts.py).

decompose() runs on the device (two HIP kernels, one block per output row) and returns the reference's
dict keys plus the ELL form of the residual that the fused linear reads.
"""

import torch

from bitexact import _hip

FR = 24                       # residual stream, linear outputs (src/bitexact/exact/consts.py:23)
FT = 30                       # cos / sin
EXP2_BITS = 14                # 2^-f table step
EXP2_ONE = 60                 # table values at 2^60
LIM3 = 8355711


def decompose(w):
    """bf16 [N, K] device tensor -> dict(limbs int8 [3, N, K], g, d int64 [N], ell_cnt int32 [N],
    ell_col int32 [N, R], ell_val int64 [N, R], R, rr, rc, rv (COO, row-major)).
    Same integers as consts.decompose (src/bitexact/exact/consts.py:67-107)."""
    assert w.dtype == torch.bfloat16 and w.dim() == 2
    _hip.require_cuda(w)
    w = w.contiguous()
    N, K = w.shape
    dev = w.device
    limbs = torch.empty(3, N, K, dtype=torch.int8, device=dev)
    g = torch.empty(N, dtype=torch.long, device=dev)
    d = torch.empty(N, dtype=torch.long, device=dev)
    cnt = torch.empty(N, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    st = _hip.stream_of(w)
    _hip.call("bx_decompose_rows", _hip.ptr(w), N, K, _hip.ptr(limbs), _hip.ptr(g), _hip.ptr(d), _hip.ptr(cnt),
              _hip.ptr(err), st)
    if int(err.item()):
        raise AssertionError("decompose: inf/nan weight or residual grid too fine")
    R = int(cnt.max().item()) if N else 0
    ec = torch.zeros(N, max(R, 1), dtype=torch.int32, device=dev)
    ev = torch.zeros(N, max(R, 1), dtype=torch.long, device=dev)
    if R:
        _hip.call("bx_decompose_residual", _hip.ptr(w), N, K, _hip.ptr(g), _hip.ptr(d), _hip.ptr(ec), _hip.ptr(ev),
                  R, st)
    j = torch.arange(max(R, 1), device=dev)[None, :]
    keep = j < cnt[:, None].long()
    rr = torch.arange(N, device=dev)[:, None].expand_as(keep)[keep]
    return {"limbs": limbs, "g": g, "d": d, "ell_cnt": cnt, "ell_col": ec, "ell_val": ev, "R": R,
            "rr": rr, "rc": ec[keep].long(), "rv": ev[keep]}


def exp2_table(device=None):
    """2^-f at 2^60, f = i / 2^14, i = 0..2^14 (src/bitexact/exact/consts.py:110-115; offline constant)."""
    f = torch.arange((1 << EXP2_BITS) + 1, dtype=torch.float64) / (1 << EXP2_BITS)
    t = torch.round(torch.pow(2.0, -f) * 2.0 ** EXP2_ONE).long()
    return t if device is None else t.to(device)
