"""Llama-3.2-1B geometry, the contiguous integer KV cache and the geometry helper (src/bitexact/llama.py).

Cache holds K and V per layer as int32 [B, HKV, L, HD]; ExactLlama (bitexact.exact.model) writes a step's keys at
their positions and attends over cache[:, :, :S]. The paged limb-plane cache of the plugin path is
bitexact.vllm_plugin.tri_paged.
"""

import torch

from bitexact.exact.consts import dims   # noqa: F401  (the reference's llama.dims)

H, HKV, HD, D, FF = 32, 8, 64, 2048, 8192      # query heads, KV heads, head dim, hidden, MLP
V = 128256                                      # vocabulary


class Cache:
    """Integer K and V per layer, int32 [B, HKV, L, HD] on the device (values within 3 limbs, checked by the
    model's q_group stage). src/bitexact/llama.py:14-26."""

    def __init__(self, n_layers, B, L, device, hkv=HKV, hd=HD):
        dev = torch.device(device)
        if dev.type != "cuda":
            raise AssertionError("bitexact (MI355X) Cache lives on the GPU only")
        z = lambda: torch.zeros(B, hkv, L, hd, dtype=torch.int32, device=dev)
        self.k = [z() for _ in range(n_layers)]
        self.v = [z() for _ in range(n_layers)]

    def write(self, layer, k, v, pos):
        """k, v int64 [B, T, HKV, HD] at positions pos [B, T] (a copy with narrowing: values are within 3 limbs)."""
        assert k.shape == v.shape and k.shape[:2] == pos.shape
        b = torch.arange(k.shape[0], device=k.device)[:, None].expand_as(pos)
        self.k[layer].permute(0, 2, 1, 3)[b, pos] = k.to(torch.int32)
        self.v[layer].permute(0, 2, 1, 3)[b, pos] = v.to(torch.int32)
