"""Exact-mode attention on the paged limb-plane KV cache (src/bitexact/vllm_plugin/tri_exact_attn.py:138-165),
on one HIP kernel (two launches when the keys are split over blocks).

attend(q, sh, qpos, cache, bt, rmap, lut, l2e, nsplit=None) -> (num int64 [R, HKV, M, HD], den int64 [R, HKV, M, 1])
with the reference's argument meaning; bn / warps are accepted for signature parity (tiles never change the
integers).
"""

import torch

from bitexact import _hip
from bitexact._ops import empty, op

BQ = 4
BLOCK_TARGET = 256          # blocks (of 8 waves) to aim for: 1 per MI355X compute unit


def default_nsplit(R, HKV, nblk, bs):
    """Key splits: none once the (row, KV head) tiles alone cover half the device (one launch, K read once);
    otherwise enough blocks to fill it, at least 128 keys per split."""
    tiles = max(1, R * HKV)
    keys = max(1, nblk * bs)
    if tiles >= 128:
        return 1
    return max(1, min(64, BLOCK_TARGET // tiles, keys // 128))


def _attend_fake(q, sh, qpos, cache, bt, rmap, lut, l2e, nsplit):
    R, HKV, M, HD = q.shape
    return empty((R, HKV, M, HD), torch.long, q), empty((R, HKV, M, 1), torch.long, q)


@op("attend_exact(Tensor q, Tensor sh, Tensor qpos, Tensor cache, Tensor bt, Tensor rmap, Tensor lut, int l2e, "
    "int nsplit) -> (Tensor, Tensor)", _attend_fake)
def _attend(q, sh, qpos, cache, bt, rmap, lut, l2e, nsplit):
    _hip.require_cuda(q, sh, qpos, cache, bt, rmap, lut)
    R, HKV, M, HD = q.shape
    assert M <= BQ and cache.shape[1] == HKV and cache.shape[3] >= 6 * HD and cache.stride(3) == 1
    assert bt.shape[1] * cache.shape[2] < 43690
    assert q.dtype == torch.int32 and cache.dtype == torch.int8 and bt.dtype == torch.int32
    q, sh, qpos = q.contiguous(), sh.contiguous().long(), qpos.contiguous().long()
    rmap, lut = rmap.contiguous().long(), lut.contiguous().long()
    num = torch.empty(R, HKV, M, HD, dtype=torch.long, device=q.device)
    den = torch.empty(R, HKV, M, 1, dtype=torch.long, device=q.device)
    ws, wsb = _hip.workspace(q.device, _hip.lib().bx_attn_paged_workspace(R, HKV, M, HD) if nsplit > 1 else 0)
    _hip.call("bx_exact_attn_paged", _hip.ptr(q), _hip.ptr(sh), _hip.ptr(qpos), qpos.stride(0), _hip.ptr(cache),
              cache.stride(0), cache.stride(1), cache.stride(2), cache.shape[2], _hip.ptr(bt), bt.stride(0),
              bt.shape[1], _hip.ptr(rmap), _hip.ptr(lut), int(l2e), _hip.ptr(num), _hip.ptr(den), R, HKV, M, HD,
              int(nsplit), _hip.ptr(ws), wsb, _hip.stream_of(q))
    return num, den


def attend(q, sh, qpos, cache, bt, rmap, lut, l2e, nsplit=None, bn=64, warps=4):
    if nsplit is None:
        nsplit = default_nsplit(q.shape[0], q.shape[1], bt.shape[1], cache.shape[2])
    return _attend(q, sh, qpos, cache, bt, rmap, lut, int(l2e), int(nsplit))


def rope_fusable(N, HKV, H, nblk, bs):
    """Whether a decode step of N tokens (one per sequence) can take rope_attend: the attention would run
    unsplit (default_nsplit == 1), over at most 2048 keys per row, with at most 4 q heads per KV head."""
    return default_nsplit(N, HKV, nblk, bs) == 1 and nblk * bs <= 2048 and H % HKV == 0 and H // HKV <= 4


def _rope_attend_fake(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag):
    N = y.shape[0]
    G = H // HKV
    return empty((N, HKV, G, HD), torch.long, y), empty((N, HKV, G, 1), torch.long, y)


@op("attend_exact_rope(Tensor y, Tensor pos, Tensor cos, Tensor sin, int H, int HKV, int HD, Tensor(a!) cache, "
    "Tensor slot, Tensor bt, Tensor rmap, Tensor lut, int l2e, Tensor(b!) flag) -> (Tensor, Tensor)", _rope_attend_fake)
def _rope_attend(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag):
    from bitexact.exact.ops import FK, FR, FT, FV, FZ
    _hip.require_cuda(y, pos, cos, sin, cache, slot, bt, rmap, lut, flag)
    N = y.shape[0]
    G = H // HKV
    assert y.dtype == torch.int64 and y.stride(-1) == 1 and y.shape[1] >= (H + 2 * HKV) * HD
    assert cache.dtype == torch.int8 and cache.dim() == 4 and cache.shape[1] == HKV and cache.shape[3] >= 6 * HD
    assert cache.stride(3) == 1 and bt.dtype == torch.int32 and flag.dtype == torch.int32
    pos = pos.reshape(-1).contiguous().long()
    slot = slot.reshape(-1).contiguous().long()
    assert pos.shape[0] == N and slot.shape[0] == N
    cos, sin = cos.contiguous().long(), sin.contiguous().long()
    rmap, lut = rmap.contiguous().long(), lut.contiguous().long()
    num = torch.empty(N, HKV, G, HD, dtype=torch.long, device=y.device)
    den = torch.empty(N, HKV, G, 1, dtype=torch.long, device=y.device)
    _hip.call("bx_exact_attn_paged_rope", _hip.ptr(y), y.stride(0), _hip.ptr(pos), 1, _hip.ptr(cos), _hip.ptr(sin),
              cos.shape[0], H, FR, FT, FK, FV, FZ, _hip.ptr(slot), _hip.ptr(cache), cache.stride(0), cache.stride(1),
              cache.stride(2), cache.shape[2], _hip.ptr(bt), bt.stride(0), bt.shape[1], _hip.ptr(rmap), _hip.ptr(lut),
              int(l2e), _hip.ptr(num), _hip.ptr(den), N, HKV, HD, _hip.ptr(flag), _hip.stream_of(y))
    return num, den


def rope_attend(y, pos, cos, sin, dm, cache, slot, bt, rmap, lut, l2e, flag):
    """A decode step's exact_fuse.qkv (RoPE, q grouping, K / V into the cache at slot) and attend in one launch, for
    steps where every token is its own sequence's only one (rope_fusable). y int64 [N, (H + 2 HKV) HD] at FR, pos /
    slot int64 [N], dm = (H, HKV, HD) -> (num int64 [N, HKV, G, HD], den int64 [N, HKV, G, 1]); bound violations
    set flag[0]. The same integers as qkv_y(..., store=(cache, slot)) followed by attend(...)."""
    H, HKV, HD = (int(v) for v in dm)
    return _rope_attend(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, int(l2e), flag)


def _rope_attend_out_fake(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag):
    N = y.shape[0]
    return empty((N, H * HD), torch.int32, y), empty((N,), torch.long, y)


@op("attend_exact_rope_out(Tensor y, Tensor pos, Tensor cos, Tensor sin, int H, int HKV, int HD, Tensor(a!) cache, "
    "Tensor slot, Tensor bt, Tensor rmap, Tensor lut, int l2e, Tensor(b!) flag) -> (Tensor, Tensor)",
    _rope_attend_out_fake)
def _rope_attend_out(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag):
    return _rope_out_call(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag, False)


def _rope_out_call(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag, planes):
    from bitexact.exact.ops import FK, FR, FT, FV, FZ
    _hip.require_cuda(y, pos, cos, sin, cache, slot, bt, rmap, lut, flag)
    N = y.shape[0]
    assert y.dtype == torch.int64 and y.stride(-1) == 1 and y.shape[1] >= (H + 2 * HKV) * HD
    assert cache.dtype == torch.int8 and cache.dim() == 4 and cache.shape[1] == HKV and cache.shape[3] >= 6 * HD
    assert cache.stride(3) == 1 and bt.dtype == torch.int32 and flag.dtype == torch.int32
    pos = pos.reshape(-1).contiguous().long()
    slot = slot.reshape(-1).contiguous().long()
    assert pos.shape[0] == N and slot.shape[0] == N
    cos, sin = cos.contiguous().long(), sin.contiguous().long()
    rmap, lut = rmap.contiguous().long(), lut.contiguous().long()
    qo = torch.empty(N, H * HD, dtype=torch.int32, device=y.device)
    sho = torch.empty(N, dtype=torch.long, device=y.device)
    ws, wsb = _hip.workspace(y.device, _hip.lib().bx_attn_rope_out_workspace(N))
    tmp, tmpb = _hip.scratch(y.device, _hip.lib().bx_attn_rope_out_scratch(N, H, HD))
    head = (_hip.ptr(y), y.stride(0), _hip.ptr(pos), 1, _hip.ptr(cos), _hip.ptr(sin), cos.shape[0], H, FR, FT, FK,
            FV, FZ, _hip.ptr(slot), _hip.ptr(cache), cache.stride(0), cache.stride(1), cache.stride(2),
            cache.shape[2], _hip.ptr(bt), bt.stride(0), bt.shape[1], _hip.ptr(rmap), _hip.ptr(lut), int(l2e),
            _hip.ptr(qo), qo.stride(0), _hip.ptr(sho))
    tail = (N, HKV, HD, _hip.ptr(flag), _hip.ptr(ws), wsb, _hip.ptr(tmp), tmpb, _hip.stream_of(y))
    if not planes:
        _hip.call("bx_exact_attn_paged_rope_out", *head, *tail)
        return qo, sho
    pl = torch.empty(3, N, H * HD, dtype=torch.int8, device=y.device)
    _hip.call("bx_exact_attn_paged_rope_out_planes", *head, _hip.ptr(pl), *tail)
    return qo, sho, pl


def _rope_attend_out_planes_fake(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag):
    N = y.shape[0]
    return empty((N, H * HD), torch.int32, y), empty((N,), torch.long, y), empty((3, N, H * HD), torch.int8, y)


@op("attend_exact_rope_out_planes(Tensor y, Tensor pos, Tensor cos, Tensor sin, int H, int HKV, int HD, "
    "Tensor(a!) cache, Tensor slot, Tensor bt, Tensor rmap, Tensor lut, int l2e, Tensor(b!) flag) -> "
    "(Tensor, Tensor, Tensor)", _rope_attend_out_planes_fake)
def _rope_attend_out_planes(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag):
    return _rope_out_call(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, l2e, flag, True)


def rope_attend_out(y, pos, cos, sin, dm, cache, slot, bt, rmap, lut, l2e, flag, planes=False):
    """rope_attend with the attention output stage fused too (ops.attn_out over its num / den): -> (q int32
    [N, H HD], sh int64 [N]), the wo linear's input; the same integers as rope_attend then ops.attn_out.
    planes=True also returns q's int8 limb planes [3, N, H HD] (the exact linear's q_planes)."""
    H, HKV, HD = (int(v) for v in dm)
    f = _rope_attend_out_planes if planes else _rope_attend_out
    return f(y, pos, cos, sin, H, HKV, HD, cache, slot, bt, rmap, lut, int(l2e), flag)
