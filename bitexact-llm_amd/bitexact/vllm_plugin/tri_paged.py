"""Paged limb-plane KV cache (src/bitexact/vllm_plugin/tri_paged.py:311-348).

Layout: int8 [nb, HKV, bs, 8 HD]; row (block, head, slot) holds K limbs 0, 1, 2 at bytes [0, 3 HD) and V limbs
at [3 HD, 6 HD) (the rest unused). store() writes tokens at their slots; to_limbs() converts an int32
[nb, HKV, bs, 2 HD] (K | V) cache into that layout (tests / reference conversions).
"""

import torch

from bitexact import _hip


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
