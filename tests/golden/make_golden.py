"""Writes tests/golden/reference_vectors.npz: input/output vectors of the reference's CPU integer rules that
closed forms do not pin bit for bit (ops.rms, ops.exp2neg_lut, ops.softmax_w, segs.norm_quant, ops.div_round,
int8 ops.quant_rows, int8 segs.softmax, ops.silu_mul, segs.silu_y + quant_silu, llama.digest; int8 ops.rms, norm24,
exp_of, silu and segs.pre_norm, pre_plain, silu_mul, qkv, attn_out). Run in the development container only, where the reference checkout is present:

    python tests/golden/make_golden.py /root/reference

The reference's own functions compute the expected outputs (src/bitexact/exact/ops.py:92-143,
src/bitexact/exact/segs.py:59-63, 120-128, src/bitexact/int8/ops.py:24-35); the inputs are seeded here. Only the
resulting arrays are committed; nothing from the reference is copied.
"""

import os
import sys

import numpy as np
import torch


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "src"))
    from bitexact.exact import ops                     # noqa: E402  (reference, CPU paths only)
    from bitexact.exact import segs                    # noqa: E402
    from bitexact.int8 import ops as iops              # noqa: E402

    out = {}
    g = torch.Generator().manual_seed(20261201)
    f = torch.arange((1 << 14) + 1, dtype=torch.float64) / (1 << 14)
    lut = torch.round(torch.pow(2.0, -f) * 2.0 ** 60).long()

    # rms and norm_quant: rows of several magnitudes, widths 512 / 2048 / 4096
    for D in (512, 2048, 4096):
        x = torch.randint(-(200 << 24), 200 << 24, (6, D), generator=g)
        x[1] //= 1 << 12
        x[2] = (1 << 40) - 1
        x[3] = x[3] >> 20
        x[4, :] = 0
        x[4, 7] = 3
        x[5] = -x[5].abs() >> 3
        r, er = ops.rms(x)
        gm = torch.randint(-255, 256, (D,), generator=g)
        ge = torch.randint(-14, -6, (D,), generator=g)
        q, sh, err = segs.norm_quant(x, gm, ge, torch.zeros((), dtype=torch.bool))
        out[f"rms{D}_x"], out[f"rms{D}_r"], out[f"rms{D}_er"] = x.numpy(), r.numpy(), er.numpy()
        out[f"nq{D}_gm"], out[f"nq{D}_ge"] = gm.numpy(), ge.numpy()
        out[f"nq{D}_q"], out[f"nq{D}_sh"], out[f"nq{D}_err"] = q.numpy(), sh.numpy(), np.array(bool(err))

    # exp2neg_lut over its whole argument range and several output widths
    t = torch.cat([torch.randint(0, 60 << 26, (3000,), generator=g), torch.arange(0, 1 << 16),
                   torch.tensor([0, 1, (1 << 26) - 1, 1 << 26, (48 << 26) * 2])])
    for bits in (22, 30, 40):
        out[f"exp2_t"] = t.numpy()
        out[f"exp2_o{bits}"] = ops.exp2neg_lut(t, lut, bits).numpy()

    # softmax_w: scores with masks, per-row exponents, head_dim 64 and 128 constants
    for hd in (64, 128):
        raw = torch.randint(-(1 << 50), 1 << 50, (24, 300), generator=g)
        raw[3] = raw[3] >> 30
        raw[4] = 7
        sh = torch.randint(-40, -10, (24, 1), generator=g)
        qpos = torch.randint(-1, 300, (24, 1), generator=g)
        qpos[0] = -1                                             # no visible key
        qpos[1] = 299
        ok = torch.arange(300)[None, :] <= qpos
        p, den = ops.softmax_w(raw, ok, sh, 17, lut, 22, ops.L2E28_HD[hd])
        out[f"sm{hd}_raw"], out[f"sm{hd}_sh"], out[f"sm{hd}_qpos"] = raw.numpy(), sh.numpy(), qpos.numpy()
        out[f"sm{hd}_p"], out[f"sm{hd}_den"] = p.numpy(), den.numpy()

    # div_round as attn_div uses it, and quant at -FR
    num = torch.randint(-(1 << 60), 1 << 60, (2000,), generator=g)
    den = torch.randint(1 << 22, 1 << 34, (2000,), generator=g)
    out["dr_num"], out["dr_den"] = num.numpy(), den.numpy()
    out["dr_o"] = ops.div_round(num, 24 - 19, den).numpy()

    # int8 quant_rows with 2 limbs
    z = torch.randint(-(1 << 44), 1 << 44, (8, 256), generator=g)
    z[1] //= 1 << 40
    z[2] = 0
    q, as_, sh = iops.quant_rows(z, 2)
    out["qr_z"], out["qr_q"], out["qr_as"], out["qr_sh"] = z.numpy(), q.numpy(), as_.numpy(), sh.numpy()

    # int8 segs.softmax (score rule and exp table; head_dim 64 and 128)
    from bitexact.int8 import consts as iconsts           # noqa: E402
    from bitexact.int8 import segs as isegs               # noqa: E402
    expt = iconsts.exp_table()
    import hashlib
    out["i8_exp_sha256"] = np.frombuffer(hashlib.sha256(expt.numpy().astype("<i8").tobytes()).digest(), np.uint8)
    for hd in (64, 128):
        raw = torch.randint(-(1 << 36), 1 << 36, (2, 2, 12, 200), generator=g)
        raw[0, 0, 3] >>= 20
        raw[1, 1, 5] = 9
        qpos = torch.randint(-1, 200, (2, 1, 12, 1), generator=g)
        qpos[0, 0, 0] = -1
        qpos[1, 0, 1] = 199
        p, den = isegs.softmax(raw, qpos, expt, hd)
        out[f"i8sm{hd}_raw"], out[f"i8sm{hd}_qpos"] = raw.numpy(), qpos.numpy()
        out[f"i8sm{hd}_p"], out[f"i8sm{hd}_den"] = p.numpy(), den.numpy()

    # silu_mul and the gate/up stage (silu_y + quant_silu) over magnitudes up to and beyond the table clamp
    gate = torch.randint(-(1 << 31), 1 << 31, (6, 512), generator=g)
    gate[1] >>= 16
    gate[2] = torch.randint(-(80 << 24), 80 << 24, (512,), generator=g)      # beyond 64 at FR: clamped argument
    gate[3, :5] = torch.tensor([0, 1, -1, 1 << 32, -(1 << 32)])
    gate[4] = 0
    up = torch.randint(-(1 << 30), 1 << 30, (6, 512), generator=g)
    up[3] >>= 12
    P, eps, ok = ops.silu_mul(gate, up, lut)
    out["silu_g"], out["silu_u"], out["silu_P"], out["silu_ok"] = gate.numpy(), up.numpy(), P.numpy(), np.array(bool(ok))
    bad = gate.clone()
    bad[0, 0] = (1 << 32) + 1                                                # |g| > 2^32: not ok
    out["silu_bad_ok"] = np.array(bool(ops.silu_mul(bad, up, lut)[2]))
    gu = torch.cat([gate, up], 1)
    q, sh, err = segs.quant_silu(*segs.silu_y(gu, lut), torch.zeros((), dtype=torch.bool))
    out["gus_q"], out["gus_sh"], out["gus_err"] = q.numpy(), sh.numpy(), np.array(bool(err))

    # llama.digest: the constants dict's SHA-256 over sorted keys (tensors: name, dtype, bytes; scalars: repr)
    from bitexact.llama import digest                     # noqa: E402
    gd = torch.Generator().manual_seed(3)
    cdict = {"n_layers": 2, "cfg": {"hidden_size": 64}, "stats": {"x": 1},
             "0.wo.limbs": torch.randint(-128, 128, (3, 4, 8), dtype=torch.int8, generator=gd),
             "0.wo.g": torch.randint(-40, 0, (4,), generator=gd), "emb": torch.randint(-9, 9, (5, 8), dtype=torch.int32,
                                                                                       generator=gd),
             "gf.m": torch.randint(-255, 256, (8,), generator=gd)}
    for k, v in cdict.items():
        if torch.is_tensor(v):
            out["dg_" + k] = v.numpy()
    out["dg_sha"] = np.frombuffer(bytes.fromhex(digest(cdict)), np.uint8)

    # int8 RMSNorm front and the other int8 segments (src/bitexact/int8/ops.py:70-108, src/bitexact/int8/segs.py:47-118)
    gi = torch.Generator().manual_seed(20261202)
    x = torch.randint(-(1 << 26), 1 << 26, (9, 512), generator=gi)
    x = x >> torch.randint(0, 20, (9, 1), generator=gi)
    x[3] = 0
    x[3, 5] = -7
    x[4] = (1 << 40) - 1
    gamma = torch.randint(1, 1 << 13, (512,), generator=gi)
    r, shx = iops.rms(x)
    out["i8rms_x"], out["i8rms_r"], out["i8rms_shx"] = x.numpy(), r.numpy(), shx.numpy()
    out["i8pn_gamma"] = gamma.numpy()
    for nl in (1, 2, 3):
        q, mant, e = isegs.pre_norm(x, gamma, nl)
        out[f"i8pn{nl}_q"], out[f"i8pn{nl}_mant"], out[f"i8pn{nl}_e"] = q.numpy(), mant.numpy(), e.numpy()
        q, mant, e = isegs.pre_plain(x, nl)
        out[f"i8pp{nl}_q"], out[f"i8pp{nl}_mant"], out[f"i8pp{nl}_e"] = q.numpy(), mant.numpy(), e.numpy()
    mant = torch.randint(1, 1 << 40, (500,), generator=gi) >> torch.randint(0, 40, (500,), generator=gi)
    ee = torch.randint(-60, 20, (500,), generator=gi)
    m2, e2 = iops.norm24(mant, ee)
    out["n24_m"], out["n24_e"], out["n24_mo"], out["n24_eo"] = mant.numpy(), ee.numpy(), m2.numpy(), e2.numpy()
    z = torch.cat([torch.randint(-(40 << 12), 1, (3000,), generator=gi), torch.tensor([0, -1, -(32 << 12),
                                                                                       -(32 << 12) - 1])])
    out["i8eo_z"], out["i8eo_v"] = z.numpy(), iops.exp_of(z, expt).numpy()
    xs = torch.arange(-iconsts.SILU_LIM << iconsts.FA, (iconsts.SILU_LIM << iconsts.FA) + 1,
                      dtype=torch.float64) / (1 << iconsts.FA)
    silu_t = torch.round(xs / (1.0 + torch.exp(-xs)) * (1 << iconsts.FR)).long()
    out["i8silu_sha256"] = np.frombuffer(hashlib.sha256(silu_t.numpy().astype("<i8").tobytes()).digest(), np.uint8)
    gg = torch.cat([torch.randint(-(40 << 16), 40 << 16, (3000,), generator=gi),
                    torch.tensor([0, 1, -1, 32 << 16, (32 << 16) - 1, -(32 << 16), -(32 << 16) - 1])])
    out["i8silu_g"], out["i8silu_v"] = gg.numpy(), iops.silu(gg, silu_t).numpy()
    gu = torch.randint(-(1 << 22), 1 << 22, (5, 1024), generator=gi)
    gu[1] >>= 10
    gu[2, :512] = torch.randint(-(40 << 16), 40 << 16, (512,), generator=gi)
    for nl in (1, 2):
        q, mant, e, flag = isegs.silu_mul(gu, silu_t, nl)
        out[f"i8sm{nl}_q"], out[f"i8sm{nl}_mant"], out[f"i8sm{nl}_e"] = q.numpy(), mant.numpy(), e.numpy()
        out[f"i8sm{nl}_flag"] = np.array(bool(flag))
    out["i8sm_gu"] = gu.numpy()
    big = gu.clone()
    big[0, 0] = 1 << 40
    big[0, 600] = 1 << 30
    out["i8sm_big_gu"] = big.numpy()
    out["i8sm_big_flag"] = np.array(bool(isegs.silu_mul(big, silu_t, 2)[3]))
    B, T, dm = 2, 5, (8, 2, 16)
    y = torch.randint(-(1 << 30), 1 << 30, (B, T, (8 + 4) * 16), generator=gi)
    ang = torch.rand(B, T, 1, 8, generator=gi, dtype=torch.float64) * 6.283
    c = torch.round(torch.cos(ang) * (1 << 16)).long()
    sn = torch.round(torch.sin(ang) * (1 << 16)).long()
    qg, k, v, flag = isegs.qkv(y, c, sn, dm)
    out["i8qkv_y"], out["i8qkv_c"], out["i8qkv_s"] = y.numpy(), c.numpy(), sn.numpy()
    out["i8qkv_qg"], out["i8qkv_k"], out["i8qkv_v"], out["i8qkv_flag"] = qg.numpy(), k.numpy(), v.numpy(), \
        np.array(bool(flag))
    y2 = y.clone()
    y2[0, 0, 0] = 1 << 40
    out["i8qkv_big_flag"] = np.array(bool(isegs.qkv(y2, c, sn, dm)[3]))
    num = torch.randint(-(1 << 50), 1 << 50, (B, 2, 4 * T, 16), generator=gi)
    den = torch.randint(1 << 20, 1 << 30, (B, 2, 4 * T, 1), generator=gi)
    for nl in (1, 2):
        q, mant, e = isegs.attn_out(num, den, T, nl, dm)
        out[f"i8ao{nl}_q"], out[f"i8ao{nl}_mant"], out[f"i8ao{nl}_e"] = q.numpy(), mant.numpy(), e.numpy()
    out["i8ao_num"], out["i8ao_den"] = num.numpy(), den.numpy()

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
