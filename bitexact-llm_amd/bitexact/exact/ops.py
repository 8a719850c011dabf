"""Exact-mode integer primitives and row stages on HIP (src/bitexact/exact/ops.py, src/bitexact/exact/segs.py).

The reference's primitives, same names and contracts (device tensors; the integers of the reference's CPU tensors):
rshc, div_round, combine, shift_round_hl, quant, rms, exp2neg_lut, silu_mul, softmax_w.

Stages with a bound check return err (a bool tensor, or'ed into the caller's `err`); with flag= (an int32 [1]
device tensor) they set that flag instead and pass err through, so a caller chaining many stages keeps one flag
and launches no extra kernels.

norm_quant(x, gm, ge, err)      segs.norm_quant: RMSNorm + quantization at -FN -> (q int32, sh, err)
softmax(raw, qpos, shg, lut, l2e) segs.softmax: masked weights at FP -> (p int32, den)
attn_out(num, den, T, hkv)      Segs.attn_out: div_round + regroup + quantization at -FR -> (q int32, sh)
qkv_y(y, pos, cos, sin, B, T, dm, err)  Segs.qkv_y: RoPE + q quantization + regroup -> (qg, shg, k, v, err)
add_norm_y(y, x, gm, ge, err)   Segs.add_norm_y: x += y in place, then norm_quant (gm None: the add alone)
embed_norm(emb, ids, gm, ge, err)  emb[ids] + pre_norm -> (x, q, sh, err)
gu_silu_y(y, lut, err)          Segs.gu_silu_y: silu(gate) up + quantization at -2 FR -> (q int32, sh, err)
"""

import torch

from bitexact import _elem, _hip
from bitexact._ops import empty, op
from bitexact.exact.consts import FR

QB = 22                         # activation rows: |q| <= 2^22 (3 int8 limbs)
FN = 40                         # normalized activations before quantization
FK, FV, FP = 17, 19, 22
FT = 30                         # cos / sin fractional bits (src/bitexact/exact/consts.py:24)
FT2 = 26                        # exponent argument t of 2^-t
FZ = 26                         # softmax z = score - max
L2E28 = 387270501               # round(log2(e) 2^28)
L2E30 = 1549082005              # round(log2(e) 2^30)
L2E28_HD = {64: L2E28, 128: 273841598}
EPS60 = 11529215046068          # round(1e-5 2^60)
NEG_BIG = -(1 << 20)


# ---- integer primitives (src/bitexact/exact/ops.py:25-143), element-wise and row kernels of csrc/bx_elem.hip ----
def rshc(x, s):
    """round(x / 2^s) for a tensor or int s (s <= 0: x 2^-s), shifts clamped to [-62, 62]
    (src/bitexact/exact/ops.py:25-34)."""
    return _elem.elem(_elem.RSHC, x, s)[0]


def div_round(a, p, r, chunk=28):
    """round(a 2^p / r), exact, for |a| < 2^62, 0 < r < 2^34 (src/bitexact/exact/ops.py:37-57: the 28-bit long
    division's value; the kernel takes its short form where that cannot wrap)."""
    assert chunk == 28, "the long division runs in 28-bit chunks"
    return _elem.elem(_elem.DIVROUND, a, p, r)[0]


def combine(T, d, B):
    """(H, L) with H 2^32 + L = T 2^d + B, 0 <= L < 2^32 (src/bitexact/exact/ops.py:60-66)."""
    H, L = _elem.elem(_elem.COMBINE, T, d, B)
    return H, L


def shift_round_hl(H, L, p):
    """round((H 2^32 + L) 2^p), 0 <= L < 2^32 (src/bitexact/exact/ops.py:69-79)."""
    return _elem.elem(_elem.SHRHL, H, L, p)[0]


def quant(P, eps):
    """Per-row power-of-two quantization of P 2^eps (P int64 [..., K], eps an int or a tensor broadcastable to P)
    -> (q int64, |q| <= 2^22, sh [...]) (src/bitexact/exact/ops.py:82-89)."""
    K = P.shape[-1]
    lead = P.shape[:-1]
    P2 = P.reshape(-1, K)
    if torch.is_tensor(eps):
        eps = eps.expand(P.shape).reshape(P2.shape)
    q, sh = _elem.row(_elem.R_QUANT, P2, eps)
    return q.view(P.shape), sh.view(lead)


def rms(x):
    """sqrt(mean(x^2) + 1e-5) of each row of x int64 [M, D] at FR as (r, er): r 2^er, 2^30 <= r < 2^31; D a power of
    two <= 4096 (src/bitexact/exact/ops.py:92-105)."""
    D = x.shape[-1]
    lg = D.bit_length() - 1
    assert D == 1 << lg and lg <= 12, "row length a power of two <= 4096"
    r, er = _elem.row(_elem.R_RMS, x, ia=(FR,))
    return r, er


def exp2neg_lut(t, lut, out_bits):
    """2^-t at out_bits for t >= 0 at FT2 bits: the 2^-f table (step 2^-14, at 2^60) and linear interpolation
    (src/bitexact/exact/ops.py:108-116)."""
    return _elem.elem(_elem.EXP2NEG, t, lut=lut, iarg=out_bits)[0]


def silu_mul(g, u, lut):
    """silu(g) u for g, u at FR -> (P, eps, ok): value P 2^eps, ok a bool device scalar (every |silu| |u| < 2^62 and
    |g| <= 2^32) (src/bitexact/exact/ops.py:119-130)."""
    fl = _elem.flag_for(g.device)
    P = _elem.elem(_elem.SILU_MUL, g, u, lut=lut, iarg=FR, flag=fl)[0]
    return P, -2 * FR, fl[0] == 0


def softmax_w(raw, ok, sh, kbits, lut, fp, l2e=None):
    """Attention weights at fp bits from exact scores raw [..., S] (value raw 2^(sh - kbits - 3), sh per row
    [..., 1]); ok marks visible keys -> (p int64 [..., S], 0 where masked, row sums [..., 1])
    (src/bitexact/exact/ops.py:133-143)."""
    S = raw.shape[-1]
    lead = raw.shape[:-1]
    r2 = raw.reshape(-1, S)
    okb = ok.expand(raw.shape).reshape(r2.shape)
    shb = sh.expand(*lead, 1).reshape(-1, 1) if torch.is_tensor(sh) else sh
    p, den = _elem.row(_elem.R_SOFTMAX_W, r2, okb, shb, lut=lut,
                       ia=(kbits, fp, L2E28 if l2e is None else int(l2e)))
    return p.view(raw.shape), den.view(*lead, 1)


def _flag(dev, flag):
    """The stage's bound flag: the caller's int32 [1] device tensor (set to 1 by the kernel, never cleared), or a
    fresh zero one."""
    if flag is not None:
        assert flag.dtype == torch.int32 and flag.is_cuda
        return flag
    return torch.zeros(1, dtype=torch.int32, device=dev)


def _or(err, flag, given):
    """err | flag as a bool tensor; with a caller's flag the flag itself carries it and err passes through."""
    if given is not None:
        return err
    e = flag[0].bool()
    return e if err is None else (err | e)


@op("norm_quant(Tensor x, Tensor gm, Tensor ge, Tensor(a!) flag) -> (Tensor, Tensor)",
    lambda x, gm, ge, flag: (empty(x.shape, torch.int32, x), empty(x.shape[:1], torch.long, x)))
def _norm_quant(x, gm, ge, flag):
    _hip.require_cuda(x, gm, ge)
    assert x.dtype == torch.int64 and x.stride(-1) == 1 and x.dim() == 2
    M, D = x.shape
    q = torch.empty(M, D, dtype=torch.int32, device=x.device)
    sh = torch.empty(M, dtype=torch.long, device=x.device)
    gm, ge = gm.contiguous().long(), ge.contiguous().long()     # kept alive until the launch is queued
    _hip.call("bx_rmsnorm_quant", _hip.ptr(x), x.stride(0), _hip.ptr(gm), _hip.ptr(ge), _hip.ptr(q), D, _hip.ptr(sh),
              M, D, FR, FN, _hip.ptr(flag), _hip.stream_of(x))
    return q, sh


@op("norm_planes(Tensor x, Tensor gm, Tensor ge, Tensor(a!) flag) -> (Tensor, Tensor, Tensor)",
    lambda x, gm, ge, flag: (empty(x.shape, torch.int32, x), empty((3, *x.shape), torch.int8, x),
                             empty(x.shape[:1], torch.long, x)))
def _norm_planes(x, gm, ge, flag):
    _hip.require_cuda(x, gm, ge)
    assert x.dtype == torch.int64 and x.stride(-1) == 1 and x.dim() == 2
    M, D = x.shape
    q = torch.empty(M, D, dtype=torch.int32, device=x.device)
    pl = torch.empty(3, M, D, dtype=torch.int8, device=x.device)
    sh = torch.empty(M, dtype=torch.long, device=x.device)
    gm, ge = gm.contiguous().long(), ge.contiguous().long()
    _hip.call("bx_add_rmsnorm_quant_planes", _hip.ptr(x), x.stride(0), None, 0, _hip.ptr(gm), _hip.ptr(ge),
              _hip.ptr(q), D, _hip.ptr(sh), _hip.ptr(pl), M, D, FR, FN, _hip.ptr(flag), _hip.stream_of(x))
    return q, pl, sh


def norm_quant(x, gm, ge, err=None, flag=None, planes=False):
    """segs.norm_quant -> (q, sh, err); planes=True: q is returned as (q, limb planes int8 [3, M, D]) for
    exact_linear's q_planes."""
    fl = _flag(x.device, flag)
    if planes:
        q, pl, sh = _norm_planes(x, gm, ge, fl)
        return (q, pl), sh, _or(err, fl, flag)
    q, sh = _norm_quant(x, gm, ge, fl)
    return q, sh, _or(err, fl, flag)


def _softmax_fake(raw, qpos, shg, lut, l2e, kbits, fp):
    return empty(raw.shape, torch.int32, raw), empty((*raw.shape[:-1], 1), torch.long, raw)


@op("softmax(Tensor raw, Tensor qpos, Tensor shg, Tensor lut, int l2e, int kbits, int fp) -> (Tensor, Tensor)",
    _softmax_fake)
def _softmax(raw, qpos, shg, lut, l2e, kbits, fp):
    _hip.require_cuda(raw, qpos, shg, lut)
    S = raw.shape[-1]
    lead = raw.shape[:-1]
    r2 = raw.reshape(-1, S)
    rows = r2.shape[0]
    qp = qpos.expand(*lead, 1).reshape(rows).contiguous().long()
    sh = shg.expand(*lead, 1).reshape(rows).contiguous().long()
    p = torch.empty(rows, S, dtype=torch.int32, device=raw.device)
    den = torch.empty(rows, dtype=torch.long, device=raw.device)
    if r2.stride(-1) != 1:
        r2 = r2.contiguous()
    lut = lut.contiguous().long()
    _hip.call("bx_softmax_w", _hip.ptr(r2), r2.stride(0), _hip.ptr(qp), _hip.ptr(sh), rows, S, kbits, _hip.ptr(lut),
              int(l2e), fp, _hip.ptr(p), S, _hip.ptr(den), _hip.stream_of(raw))
    return p.view(*lead, S), den.view(*lead, 1)


def softmax(raw, qpos, shg, lut, l2e, kbits=FK, fp=FP):
    """raw int64 [..., S] scores, qpos / shg broadcastable [..., 1] -> (p int32 [..., S], den int64 [..., 1])."""
    return _softmax(raw, qpos, shg, lut, int(l2e), int(kbits), int(fp))


def _attn_out_fake(num, den, T, hkv):
    Z, gT, HD = num.shape
    rows = (Z // hkv) * T
    return empty((rows, hkv * (gT // T) * HD), torch.int32, num), empty((rows,), torch.long, num)


@op("attn_out(Tensor num, Tensor den, int T, int hkv) -> (Tensor, Tensor)", _attn_out_fake)
def _attn_out(num, den, T, hkv):
    _hip.require_cuda(num, den)
    Z, gT, HD = num.shape
    g = gT // T
    B = Z // hkv
    assert num.stride(2) == 1
    den2 = den.reshape(Z, gT).contiguous().long()
    rows = B * T
    q = torch.empty(rows, hkv * g * HD, dtype=torch.int32, device=num.device)
    sh = torch.empty(rows, dtype=torch.long, device=num.device)
    _hip.call("bx_attn_out", _hip.ptr(num), num.stride(0), num.stride(1), _hip.ptr(den2), gT, rows, T, hkv, g, HD, FR,
              FV, _hip.ptr(q), q.stride(0), _hip.ptr(sh), _hip.stream_of(num))
    return q, sh


def attn_out(num, den, T, hkv):
    """num int64 [Z = B HKV, g T, HD], den [Z, g T, 1] -> (q int32 [B T, H HD], sh int64 [B T])."""
    return _attn_out(num, den, int(T), int(hkv))


def _qkv_fake(y, pos, cos, sin, B, T, H, HKV, HD, flag):
    g = H // HKV
    return (empty((B * HKV, g * T, HD), torch.int32, y), empty((B * HKV, g * T, 1), torch.long, y),
            empty((B, T, HKV, HD), torch.long, y), empty((B, T, HKV, HD), torch.long, y))


def _qkv_check(y, pos, cos, sin, B, T, H, HKV, HD):
    _hip.require_cuda(y, pos, cos, sin)
    assert y.dtype == torch.int64 and y.stride(-1) == 1 and y.shape[0] == B * T
    assert y.shape[1] >= (H + 2 * HKV) * HD and H % HKV == 0
    assert pos.dtype == torch.int64 and pos.dim() == 2
    assert cos.shape == sin.shape and cos.shape[1] == HD // 2


@op("qkv_y(Tensor y, Tensor pos, Tensor cos, Tensor sin, int B, int T, int H, int HKV, int HD, Tensor(a!) flag) -> "
    "(Tensor, Tensor, Tensor, Tensor)", _qkv_fake)
def _qkv_y(y, pos, cos, sin, B, T, H, HKV, HD, flag):
    _qkv_check(y, pos, cos, sin, B, T, H, HKV, HD)
    g = H // HKV
    dev = y.device
    cos, sin = cos.contiguous().long(), sin.contiguous().long()
    qg = torch.empty(B * HKV, g * T, HD, dtype=torch.int32, device=dev)
    shg = torch.empty(B * HKV, g * T, 1, dtype=torch.long, device=dev)
    k = torch.empty(B, T, HKV, HD, dtype=torch.long, device=dev)
    v = torch.empty(B, T, HKV, HD, dtype=torch.long, device=dev)
    _hip.call("bx_rope_qgroup", _hip.ptr(y), y.stride(0), _hip.ptr(pos), pos.stride(0), pos.stride(1),
              _hip.ptr(cos), _hip.ptr(sin), cos.shape[0], B, T, H, HKV, HD, FR, FT, FK, FV, FZ, _hip.ptr(qg),
              _hip.ptr(shg), _hip.ptr(k), _hip.ptr(v), _hip.ptr(flag), _hip.stream_of(y))
    return qg, shg, k, v


@op("qkv_y_store(Tensor y, Tensor pos, Tensor cos, Tensor sin, int B, int T, int H, int HKV, int HD, "
    "Tensor(a!) flag, Tensor(b!) cache, Tensor slot) -> (Tensor, Tensor)",
    lambda y, pos, cos, sin, B, T, H, HKV, HD, flag, cache, slot: _qkv_fake(y, pos, cos, sin, B, T, H, HKV, HD,
                                                                              flag)[:2])
def _qkv_y_store(y, pos, cos, sin, B, T, H, HKV, HD, flag, c, slot):
    _qkv_check(y, pos, cos, sin, B, T, H, HKV, HD)
    g = H // HKV
    dev = y.device
    cos, sin = cos.contiguous().long(), sin.contiguous().long()
    qg = torch.empty(B * HKV, g * T, HD, dtype=torch.int32, device=dev)
    shg = torch.empty(B * HKV, g * T, 1, dtype=torch.long, device=dev)
    _hip.require_cuda(c, slot)
    assert c.dtype == torch.int8 and c.dim() == 4 and c.shape[1] == HKV and c.shape[3] >= 6 * HD and c.stride(3) == 1
    slot = slot.reshape(-1).contiguous().long()
    assert slot.shape[0] == B * T
    _hip.call("bx_rope_qgroup_store", _hip.ptr(y), y.stride(0), _hip.ptr(pos), pos.stride(0), pos.stride(1),
              _hip.ptr(cos), _hip.ptr(sin), cos.shape[0], B, T, H, HKV, HD, FR, FT, FK, FV, FZ, _hip.ptr(qg),
              _hip.ptr(shg), None, None, _hip.ptr(c), c.stride(0), c.stride(1), c.stride(2), _hip.ptr(slot),
              c.shape[2], _hip.ptr(flag), _hip.stream_of(y))
    return qg, shg


def qkv_y(y, pos, cos, sin, B, T, dm, err=None, flag=None, store=None):
    """Segs.qkv_y (src/bitexact/exact/segs.py:170-173): y int64 [B T, (H + 2 HKV) HD] at FR, pos int64 [B, T],
    cos / sin int64 [n_pos, HD / 2] at FT, dm = (H, HKV, HD) -> qg int32 [B HKV, g T, HD], shg int64
    [B HKV, g T, 1], k / v int64 [B, T, HKV, HD], err (bool tensor, or'ed into `err`).
    store = (cache, slot): exact_fuse.qkv's fused store (src/bitexact/vllm_plugin/exact_fuse.py:372-386): K / V go
    straight into the limb-plane cache (int8 [nb, HKV, bs, 8 HD]) at slot [B T] (< 0: skipped), and k / v are
    returned as None."""
    H, HKV, HD = (int(v) for v in dm)
    fl = _flag(y.device, flag)
    pos = pos.long()
    if store is not None:
        c, slot = store
        qg, shg = _qkv_y_store(y, pos, cos, sin, int(B), int(T), H, HKV, HD, fl, c, slot)
        return qg, shg, None, None, _or(err, fl, flag)
    qg, shg, k, v = _qkv_y(y, pos, cos, sin, int(B), int(T), H, HKV, HD, fl)
    return qg, shg, k, v, _or(err, fl, flag)


@op("add_rows(Tensor y, Tensor(a!) x, Tensor(b!) flag) -> ()", lambda y, x, flag: None)
def _add_rows(y, x, flag):
    _hip.require_cuda(x, y)
    assert x.dtype == torch.int64 and y.dtype == torch.int64 and x.stride(-1) == 1 and y.stride(-1) == 1
    M, D = x.shape
    y = y.view(M, D) if y.dim() != 2 else y
    _hip.call("bx_add_rmsnorm_quant", _hip.ptr(x), x.stride(0), _hip.ptr(y), y.stride(0), None, None, None, D, None,
              M, D, FR, FN, _hip.ptr(flag), _hip.stream_of(x))


def _add_norm_fake(y, x, gm, ge, flag, planes):
    M, D = x.shape
    return (empty((M, D), torch.int32, x), empty((3, M, D) if planes else (0,), torch.int8, x),
            empty((M,), torch.long, x))


@op("add_norm(Tensor y, Tensor(a!) x, Tensor gm, Tensor ge, Tensor(b!) flag, bool planes) -> (Tensor, Tensor, Tensor)",
    _add_norm_fake)
def _add_norm(y, x, gm, ge, flag, planes):
    _hip.require_cuda(x, y)
    assert x.dtype == torch.int64 and y.dtype == torch.int64 and x.stride(-1) == 1 and y.stride(-1) == 1
    M, D = x.shape
    y = y.view(M, D) if y.dim() != 2 else y
    q = torch.empty(M, D, dtype=torch.int32, device=x.device)
    sh = torch.empty(M, dtype=torch.long, device=x.device)
    gm, ge = gm.contiguous().long(), ge.contiguous().long()
    if planes:
        pl = torch.empty(3, M, D, dtype=torch.int8, device=x.device)
        _hip.call("bx_add_rmsnorm_quant_planes", _hip.ptr(x), x.stride(0), _hip.ptr(y), y.stride(0), _hip.ptr(gm),
                  _hip.ptr(ge), _hip.ptr(q), D, _hip.ptr(sh), _hip.ptr(pl), M, D, FR, FN, _hip.ptr(flag),
                  _hip.stream_of(x))
        return q, pl, sh
    _hip.call("bx_add_rmsnorm_quant", _hip.ptr(x), x.stride(0), _hip.ptr(y), y.stride(0), _hip.ptr(gm), _hip.ptr(ge),
              _hip.ptr(q), D, _hip.ptr(sh), M, D, FR, FN, _hip.ptr(flag), _hip.stream_of(x))
    return q, torch.empty(0, dtype=torch.int8, device=x.device), sh


def add_norm_y(y, x, gm, ge, err=None, flag=None, planes=False):
    """Segs.add_norm_y (src/bitexact/exact/segs.py:175-178): x int64 [M, D] += y (in place, as exact_fuse.add_norm's
    store), then norm_quant of the sum. gm None: the add alone (returns q = sh = None). planes=True: q is returned
    as (q, limb planes int8 [3, M, D]) for exact_linear's q_planes (the limb split done by the norm kernel)."""
    fl = _flag(x.device, flag)
    if gm is None:
        _add_rows(y, x, fl)
        return x, None, None, _or(err, fl, flag)
    q, pl, sh = _add_norm(y, x, gm, ge, fl, bool(planes))
    return x, ((q, pl) if planes else q), sh, _or(err, fl, flag)


def _embed_fake(emb, ids, gm, ge, flag):
    M, D = ids.numel(), emb.shape[1]
    return empty((M, D), torch.long, emb), empty((M, D), torch.int32, emb), empty((M,), torch.long, emb)


@op("embed_norm_planes(Tensor emb, Tensor ids, Tensor gm, Tensor ge, Tensor(a!) flag) -> (Tensor, Tensor, Tensor, "
    "Tensor)", lambda emb, ids, gm, ge, flag: (*_embed_fake(emb, ids, gm, ge, flag)[:2],
                                               empty((3, ids.numel(), emb.shape[1]), torch.int8, emb),
                                               empty((ids.numel(),), torch.long, emb)))
def _embed_norm_planes(emb, ids, gm, ge, flag):
    _hip.require_cuda(emb, ids, gm, ge)
    assert emb.dtype == torch.int32 and emb.is_contiguous()
    ids = ids.reshape(-1).contiguous().long()
    M, D = ids.shape[0], emb.shape[1]
    x = torch.empty(M, D, dtype=torch.long, device=emb.device)
    q = torch.empty(M, D, dtype=torch.int32, device=emb.device)
    pl = torch.empty(3, M, D, dtype=torch.int8, device=emb.device)
    sh = torch.empty(M, dtype=torch.long, device=emb.device)
    gm, ge = gm.contiguous().long(), ge.contiguous().long()
    _hip.call("bx_embed_rmsnorm_quant_planes", _hip.ptr(emb), _hip.ptr(ids), _hip.ptr(x), D, _hip.ptr(gm),
              _hip.ptr(ge), _hip.ptr(q), D, _hip.ptr(sh), _hip.ptr(pl), M, D, FR, FN, _hip.ptr(flag),
              _hip.stream_of(emb))
    return x, q, pl, sh


@op("embed_norm(Tensor emb, Tensor ids, Tensor gm, Tensor ge, Tensor(a!) flag) -> (Tensor, Tensor, Tensor)",
    _embed_fake)
def _embed_norm(emb, ids, gm, ge, flag):
    _hip.require_cuda(emb, ids, gm, ge)
    assert emb.dtype == torch.int32 and emb.is_contiguous()
    ids = ids.reshape(-1).contiguous().long()
    M, D = ids.shape[0], emb.shape[1]
    x = torch.empty(M, D, dtype=torch.long, device=emb.device)
    q = torch.empty(M, D, dtype=torch.int32, device=emb.device)
    sh = torch.empty(M, dtype=torch.long, device=emb.device)
    gm, ge = gm.contiguous().long(), ge.contiguous().long()
    _hip.call("bx_embed_rmsnorm_quant", _hip.ptr(emb), _hip.ptr(ids), _hip.ptr(x), D, _hip.ptr(gm), _hip.ptr(ge),
              _hip.ptr(q), D, _hip.ptr(sh), M, D, FR, FN, _hip.ptr(flag), _hip.stream_of(emb))
    return x, q, sh


def embed_norm(emb, ids, gm, ge, err=None, flag=None, planes=False):
    """x = emb[ids].long() (emb int32 [V, D]) and its pre_norm (src/bitexact/exact/model.py:130-132) -> (x, q, sh, err);
    planes=True: q is returned as (q, limb planes int8 [3, M, D]) for exact_linear's q_planes."""
    fl = _flag(emb.device, flag)
    if planes:
        x, q, pl, sh = _embed_norm_planes(emb, ids, gm, ge, fl)
        return x, (q, pl), sh, _or(err, fl, flag)
    x, q, sh = _embed_norm(emb, ids, gm, ge, fl)
    return x, q, sh, _or(err, fl, flag)


SILU_SPLIT_ROWS = 128   # fewer rows than this: the stage is split over column chunks (bx_silu_quant_ws)


def _silu_fake(y, lut, flag, split, planes):
    M, ff = y.shape[0], y.shape[1] // 2
    return (empty((M, ff), torch.int32, y), empty((3, M, ff) if planes else (0,), torch.int8, y),
            empty((M,), torch.long, y))


@op("gu_silu(Tensor y, Tensor lut, Tensor(a!) flag, bool split, bool planes) -> (Tensor, Tensor, Tensor)", _silu_fake)
def _gu_silu(y, lut, flag, split, planes):
    _hip.require_cuda(y, lut)
    assert y.dtype == torch.int64 and y.stride(-1) == 1 and y.shape[1] % 2 == 0
    M, ff = y.shape[0], y.shape[1] // 2
    q = torch.empty(M, ff, dtype=torch.int32, device=y.device)
    sh = torch.empty(M, dtype=torch.long, device=y.device)
    lut = lut.contiguous().long()
    assert split or not planes, "limb planes come from the column-chunked path"
    pl = torch.empty((3, M, ff) if planes else (0,), dtype=torch.int8, device=y.device)
    if split and M > 0:
        tmp, tmpb = _hip.workspace(y.device, _hip.lib().bx_silu_quant_scratch(M, ff))   # zero-filled, kept so
        _hip.call("bx_silu_quant_ws", _hip.ptr(y), y.stride(0), ff, _hip.ptr(lut), FR, _hip.ptr(q), ff, _hip.ptr(sh),
                  _hip.ptr(pl) if planes else None, M, _hip.ptr(flag), _hip.ptr(tmp), tmpb, _hip.stream_of(y))
        return q, pl, sh
    _hip.call("bx_silu_quant", _hip.ptr(y), y.stride(0), ff, _hip.ptr(lut), FR, _hip.ptr(q), ff, _hip.ptr(sh), M,
              _hip.ptr(flag), _hip.stream_of(y))
    return q, pl, sh


def gu_silu_y(y, lut, err=None, flag=None, split=None, planes=False):
    """Segs.gu_silu_y (src/bitexact/exact/segs.py:180-182): y int64 [M, 2 ff] (gate | up) at FR ->
    (q int32 [M, ff], sh int64 [M], err | not ok). split: None picks by row count; True / False force the
    column-chunked or the row-per-block kernel (the same integers either way). planes=True (column-chunked path):
    q is returned as (q, limb planes int8 [3, M, ff]) for exact_linear's q_planes."""
    fl = _flag(y.device, flag)
    if split is None:
        split = y.shape[0] < SILU_SPLIT_ROWS or planes
    q, pl, sh = _gu_silu(y, lut, fl, bool(split), bool(planes))
    return ((q, pl) if planes else q), sh, _or(err, fl, flag)
