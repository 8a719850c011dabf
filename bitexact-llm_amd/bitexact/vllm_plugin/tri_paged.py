"""Paged limb-plane KV cache (src/bitexact/vllm_plugin/tri_paged.py:311-348).

Layout: int8 [nb, HKV, bs, 8 HD]; row (block, head, slot) holds K limbs 0, 1, 2 at bytes [0, 3 HD) and V limbs
at [3 HD, 6 HD) (the rest unused). store() writes tokens at their slots; to_limbs() converts an int32
[nb, HKV, bs, 2 HD] (K | V) cache into that layout (tests / reference conversions). attend() is the int8-mode
paged attention over that cache (one HIP kernel, two launches when the keys are split).
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op


@op("kv_store(Tensor(a!) c, Tensor slot, Tensor k, Tensor v) -> ()", lambda c, slot, k, v: None)
def store(c, slot, k, v):
    """K / V (int32 or int64 [N, HKV, HD], |.| within 3 limbs) of the tokens at cache slots slot [N] into the
    limb-plane cache c (int8 [nb, HKV, bs, 8 HD]); slot < 0 is skipped."""
    _hip.require_cuda(c, slot, k, v)
    N, hkv, hd = k.shape
    assert k.dtype == v.dtype and k.dtype in (torch.int32, torch.int64) and k.stride(2) == 1 and v.stride(2) == 1
    assert c.dtype == torch.int8 and c.shape[1] == hkv and c.shape[3] >= 6 * hd and c.stride(3) == 1
    if N == 0:
        return
    slot = slot.contiguous().long()
    _hip.call("bx_kv_store", _hip.ptr(c), c.stride(0), c.stride(1), c.stride(2), c.shape[2], _hip.ptr(slot), _hip.ptr(k),
              k.stride(0), k.stride(1), _hip.ptr(v), v.stride(0), v.stride(1), k.element_size(), N, hkv, hd,
              _hip.stream_of(c))


def to_limbs(c):
    """int32 cache [nb, HKV, bs, 2 HD] (K | V) -> int8 limb planes [nb, HKV, bs, 8 HD]."""
    nb, hkv, bs, two_hd = c.shape
    hd = two_hd // 2
    out = torch.zeros(nb, hkv, bs, 8 * hd, dtype=torch.int8, device=c.device)
    flat = c.permute(0, 2, 1, 3).reshape(nb * bs, hkv, two_hd)
    slot = torch.arange(nb * bs, device=c.device)
    store(out, slot, flat[..., :hd], flat[..., hd:])
    return out


FE, FP = 30, 20                 # exp table values, int8 attention weights (src/bitexact/int8/segs.py:22)
SM_TARGET = 256                 # blocks (of 8 waves) to aim for: 1 per MI355X compute unit


def weight_table(lut):
    """rsh(exp_lut, FE - FP) as int32 (src/bitexact/vllm_plugin/tri_paged.py:351-356); built once at load."""
    t = (lut + (1 << (FE - FP - 1))) >> (FE - FP)
    return t.to(torch.int32).contiguous()


def attend(q, qpos, cache, bt, ptab, nsplit=None, bm=None, bn=None, warps=4):
    """int8-mode paged attention (src/bitexact/vllm_plugin/tri_paged.py:363-401): q int64 [R, HKV, M, HD], qpos int64
    [R, M], cache int8 [nb, HKV, bs, 8 HD], bt int32 [R, *], ptab = weight_table(exp table) -> (num int64
    [R, HKV, M, HD], den int64 [R, HKV, M, 1]). bm / bn / warps are accepted for signature parity."""
    if nsplit is None:
        R, HKV, M, _ = q.shape
        tiles = max(1, R * HKV * ((M + 3) // 4))
        keys = max(1, bt.shape[1] * cache.shape[2])
        nsplit = 1 if tiles >= 128 else max(1, min(64, SM_TARGET // tiles, keys // 128))
    return _attend_int8(q, qpos, cache, bt, ptab, int(nsplit))


def _attend_int8_fake(q, qpos, cache, bt, ptab, nsplit):
    R, HKV, M, HD = q.shape
    return empty((R, HKV, M, HD), torch.long, q), empty((R, HKV, M, 1), torch.long, q)


@op("attend_int8(Tensor q, Tensor qpos, Tensor cache, Tensor bt, Tensor ptab, int nsplit) -> (Tensor, Tensor)",
    _attend_int8_fake)
def _attend_int8(q, qpos, cache, bt, ptab, nsplit):
    _hip.require_cuda(q, qpos, cache, bt, ptab)
    R, HKV, M, HD = q.shape
    assert cache.shape[1] == HKV and cache.shape[3] >= 6 * HD and cache.stride(3) == 1
    assert bt.shape[1] * cache.shape[2] < 43690
    assert cache.dtype == torch.int8 and bt.dtype == torch.int32 and ptab.dtype == torch.int32
    q, qpos, ptab = q.contiguous().long(), qpos.contiguous().long(), ptab.contiguous()
    num = torch.empty(R, HKV, M, HD, dtype=torch.long, device=q.device)
    den = torch.empty(R, HKV, M, 1, dtype=torch.long, device=q.device)
    ws, wsb = _hip.workspace(q.device, _hip.lib().bx_attn_paged_workspace(R, HKV, M, HD) if nsplit > 1 else 0)
    _hip.call("bx_int8_attn_paged", _hip.ptr(q), _hip.ptr(qpos), qpos.stride(0), _hip.ptr(cache), cache.stride(0),
              cache.stride(1), cache.stride(2), cache.shape[2], _hip.ptr(bt), bt.stride(0), bt.shape[1],
              _hip.ptr(ptab), ptab.numel(), _hip.ptr(num), _hip.ptr(den), R, HKV, M, HD, int(nsplit), _hip.ptr(ws),
              wsb, _hip.stream_of(q))
    return num, den
