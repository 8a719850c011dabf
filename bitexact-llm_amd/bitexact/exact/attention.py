"""Exact-mode attention over the contiguous integer cache, fused (src/bitexact/exact/model.py:113-119):
num, den = prefill(qg, shg, K, V, qpos, lut, l2e) computes bmm(qg, K^T) -> segs.softmax -> bmm(p, V) in one
HIP kernel without materializing the score matrix.

qg int32 [Z, gT, HD], shg int64 [Z, gT, 1], K / V int32 [Z, S, HD] (any row strides, e.g. the reference Cache
[B, HKV, L, HD] viewed as [B * HKV, L, HD]), qpos int64 [Z, gT, 1] (key s visible iff s <= qpos) ->
num int64 [Z, gT, HD], den int64 [Z, gT, 1].
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op


def _aligned_rows(t):
    """The kernel reads 16-byte row pieces: rows must start 16-byte aligned (else a contiguous copy)."""
    ok = t.data_ptr() % 16 == 0 and t.stride(0) % 4 == 0 and t.stride(1) % 4 == 0
    return t if ok else t.contiguous()


def _prefill_fake(qg, shg, K, V, qpos, lut, l2e, planes):
    Z, gT, HD = qg.shape
    return empty((Z, gT, HD), torch.long, qg), empty((Z, gT, 1), torch.long, qg)


@op("attn_prefill(Tensor qg, Tensor shg, Tensor K, Tensor V, Tensor qpos, Tensor lut, int l2e, bool planes) -> "
    "(Tensor, Tensor)", _prefill_fake)
def _prefill(qg, shg, K, V, qpos, lut, l2e, planes):
    _hip.require_cuda(qg, shg, K, V, qpos, lut)
    Z, gT, HD = qg.shape
    S = K.shape[1]
    assert K.shape == V.shape and K.shape[0] == Z and K.shape[2] == HD
    assert qg.dtype == torch.int32 and K.dtype == torch.int32 and V.dtype == torch.int32
    assert qg.stride(2) == 1 and K.stride(2) == 1 and V.stride(2) == 1
    qg, K, V = (_aligned_rows(t) for t in (qg, K, V))
    shg = shg.reshape(Z, gT).contiguous().long()
    qpos = qpos.reshape(Z, gT).long()
    lut = lut.contiguous().long()
    num = torch.empty(Z, gT, HD, dtype=torch.long, device=qg.device)
    den = torch.empty(Z, gT, 1, dtype=torch.long, device=qg.device)
    need = _hip.lib().bx_attn_prefill_scratch(Z, S, HD) if planes else 0
    tmp, tmpb = _hip.scratch(qg.device, need) if need > 0 else (None, 0)
    _hip.call("bx_exact_attn_prefill", _hip.ptr(qg), qg.stride(0), qg.stride(1), _hip.ptr(shg), gT, _hip.ptr(qpos),
              qpos.stride(0), qpos.stride(1), _hip.ptr(K), K.stride(0), K.stride(1), _hip.ptr(V), V.stride(0),
              V.stride(1), S, _hip.ptr(lut), int(l2e), _hip.ptr(num), _hip.ptr(den), Z, gT, HD, _hip.ptr(tmp), tmpb,
              _hip.stream_of(qg))
    return num, den


def prefill(qg, shg, K, V, qpos, lut, l2e, planes=True):
    """planes=True: K / V split into int8 limb planes once (scratch) and streamed into LDS by the main kernel;
    False: the register-staged kernel (no scratch). Same integers."""
    return _prefill(qg, shg, K, V, qpos, lut, int(l2e), bool(planes))
