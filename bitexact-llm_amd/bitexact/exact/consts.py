"""Exact-mode weight format and tables (src/bitexact/exact/consts.py).

decompose() runs on the device (two HIP kernels, one block per output row) and returns the reference's
dict keys plus the ELL form of the residual that the fused linear reads. random_constants() builds a
constants dict with the reference's keys (src/bitexact/exact/consts.py:118-149) for a random-init model of
a given geometry: bf16 N(0, 0.02) weights drawn on the device, decomposed there, unit norm gammas, tied
lm_head. The RoPE and 2^-f tables are float64 constants computed once on the host, as the reference's
offline build computes them.
"""

import math

import torch

from bitexact import _hip

FR = 24                       # residual stream, linear outputs (src/bitexact/exact/consts.py:23)
FT = 30                       # cos / sin
MAX_POS = 4096                # RoPE table rows
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


def bf16_parts(w):
    """bf16 tensor -> (signed significand, exponent) int64: w = sm 2^ex exactly (src/bitexact/exact/consts.py:33-42)."""
    b = w.contiguous().view(torch.int16).long() & 0xFFFF
    e = (b >> 7) & 0xFF
    assert not bool((e == 255).any()), "inf/nan weight"
    m = b & 0x7F
    mag = torch.where(e > 0, m | 0x80, m)
    ex = torch.where(e > 0, e, torch.ones_like(e)) - 134
    return torch.where((b >> 15) == 1, -mag, mag), ex


def emb_fixed(w):
    """Embedding table bf16 [V, D] -> int32 at FR, each entry rounded once (half up) to 2^-FR
    (src/bitexact/exact/consts.py:131-135)."""
    sm, ex = bf16_parts(w)
    s = ex + FR
    e = torch.where(s >= 0, sm << s.clamp(min=0),
                    (sm + (1 << (-s - 1).clamp(min=0, max=62))) >> (-s).clamp(max=63))
    assert int(e.abs().max()) < 1 << 31
    return e.to(torch.int32)


def llama3_inv_freq(hd=64, theta=500000.0, factor=32.0, low=1.0, high=4.0, orig=8192):
    """Llama-3 scaled RoPE inverse frequencies: the transformers rule src/bitexact/llama.py:52-62 calls, in its
    float32 arithmetic, widened to float64. Wavelengths above orig / low are divided by factor, those below
    orig / high kept, the band between blended."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.int64).to(torch.float32) / hd))
    wl = 2 * math.pi / inv
    out = torch.where(wl > orig / low, inv / factor, inv)
    smooth = (orig / wl - low) / (high - low)
    mid = (1 - smooth) * out / factor + smooth * out
    return torch.where(~(wl < orig / high) & ~(wl > orig / low), mid, out).double()


def rope_tables(n_pos, bits, inv_freq):
    """Integer cos / sin [n_pos, HD / 2] at `bits` fractional bits, rounded once (src/bitexact/llama.py:65-68)."""
    ang = torch.arange(n_pos, dtype=torch.float64)[:, None] * inv_freq[None, :]
    return torch.round(torch.cos(ang) * 2.0 ** bits).long(), torch.round(torch.sin(ang) * 2.0 ** bits).long()


LLAMA_3_2_1B = {"hidden_size": 2048, "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 64,
                "intermediate_size": 8192, "vocab_size": 128256, "num_hidden_layers": 16, "rope_theta": 500000.0,
                "rope_scaling": {"factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                 "original_max_position_embeddings": 8192}}


def dims(cfg):
    """(H, HKV, HD, D, FF) of a HF Llama config dict (src/bitexact/llama.py:29-33); {} gives Llama-3.2-1B."""
    c = LLAMA_3_2_1B
    d = cfg.get("hidden_size", c["hidden_size"])
    h = cfg.get("num_attention_heads", c["num_attention_heads"])
    return (h, cfg.get("num_key_value_heads", c["num_key_value_heads"]), cfg.get("head_dim") or d // h, d,
            cfg.get("intermediate_size", c["intermediate_size"]))


def random_constants(cfg=None, n_layers=None, seed=0, device="cuda", keep_bf16=False, with_sha=False):
    """Constants dict (the reference's keys) of a random-init Llama: every linear weight bf16 N(0, 0.02) drawn on
    `device` from `seed`, decomposed there; norm gammas 1.0; lm_head tied to the embedding. keep_bf16 also keeps
    each weight's bf16 tensor under f"{name}.bf16" (checkers rebuild the decomposition from it). with_sha stores
    the model's identity under "sha256", as the reference's build does (it hashes every plane on the host)."""
    cfg = dict(LLAMA_3_2_1B if cfg is None else cfg)
    H, HKV, HD, D, FF = dims(cfg)
    V = cfg.get("vocab_size", LLAMA_3_2_1B["vocab_size"])
    L = cfg.get("num_hidden_layers", 16) if n_layers is None else n_layers
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    c = {"n_layers": L, "cfg": cfg}

    def draw(n, k):
        return (torch.randn(n, k, generator=gen, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)

    def put(name, w):
        dec = decompose(w)
        for k in ("limbs", "g", "d", "rr", "rc", "rv", "ell_cnt", "ell_col", "ell_val", "R"):
            c[f"{name}.{k}"] = dec[k]
        if keep_bf16:
            c[f"{name}.bf16"] = w

    emb = draw(V, D)
    c["emb"] = emb_fixed(emb)
    one = torch.ones(D, dtype=torch.bfloat16, device=dev)
    for i in range(L):
        put(f"{i}.wqkv", draw((H + 2 * HKV) * HD, D))
        put(f"{i}.wo", draw(D, H * HD))
        put(f"{i}.wgu", draw(2 * FF, D))
        put(f"{i}.wd", draw(D, FF))
        for n in ("ga", "gm"):
            c[f"{i}.{n}.m"], c[f"{i}.{n}.e"] = bf16_parts(one)
    c["gf.m"], c["gf.e"] = bf16_parts(one)
    put("lm", emb)
    if keep_bf16:
        c["emb.bf16"] = emb
    rs = cfg.get("rope_scaling") or {}
    inv = llama3_inv_freq(HD, cfg.get("rope_theta", 500000.0), rs.get("factor", 32.0), rs.get("low_freq_factor", 1.0),
                          rs.get("high_freq_factor", 4.0), rs.get("original_max_position_embeddings", 8192))
    c["cos"], c["sin"] = (t.to(dev) for t in rope_tables(MAX_POS, FT, inv))
    c["exp2"] = exp2_table(dev)
    if with_sha:
        c["sha256"] = sha256(c)
    return c


# keys this build adds to a constants dict (device-side ELL form, kept bf16 sources); they are derived data and
# stay out of the model's identity
_DERIVED = (".ell_cnt", ".ell_col", ".ell_val", ".R", ".bf16")


def sha256(c, skip=("cfg", "stats", "sha256")):
    """The model's identity: SHA-256 over every tensor and scalar of the constants dict in key order -- per key its
    name, then a tensor's dtype name and bytes or a scalar's repr (src/bitexact/llama.py:77-92 via
    src/bitexact/exact/consts.py:152-154). Keys in `skip` and this build's derived keys are left out."""
    import hashlib
    h = hashlib.sha256()
    for k in sorted(c):
        if k in skip or k.endswith(_DERIVED):
            continue
        v = c[k]
        h.update(k.encode())
        if torch.is_tensor(v):
            h.update(str(v.dtype).encode())
            h.update(v.detach().contiguous().cpu().numpy().tobytes())
        else:
            h.update(repr(v).encode())
    return h.hexdigest()


def save(c, path):
    """Write a constants dict as one safetensors file: every tensor under its key, every other entry (layer count,
    config, residual widths) as JSON in the file's metadata. Replaces the reference's pickle (torch.save) with a
    format that loads without executing anything."""
    import json

    from safetensors.torch import save_file
    tensors = {k: v.detach().contiguous().cpu() for k, v in c.items() if torch.is_tensor(v)}
    other = {k: v for k, v in c.items() if not torch.is_tensor(v)}
    save_file(tensors, path, metadata={"bitexact": json.dumps(other, sort_keys=True)})


def load(path, device="cpu"):
    """Read a constants dict written by save() (tensors moved to `device`)."""
    import json

    from safetensors import safe_open
    c = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        for k in f.keys():
            c[k] = f.get_tensor(k).to(device)
    c.update(json.loads(meta.get("bitexact", "{}")))
    return c
