"""Exact-bf16 Llama over a constants dict (src/bitexact/exact/model.py): Lin and ExactLlama, on the HIP kernels.

Lin(c, name, device, gemm) reads c[f"{name}.limbs" | ".g" | ".d" | ".rr" | ".rc" | ".rv"] (the reference's key
layout) and builds the ELL residual once (src/bitexact/exact/model.py:39-48). __call__(q) keeps the
reference's (C, rs, d, g) contract for segs.lin_y; y(q, sh, checked) is the fused HIP linear. gemm takes the
reference's values: "hip" (this build), and "triton" / "cublas" (the reference's CUDA backends), which this build
serves with the same HIP kernels (every backend gives the same integers). There is no CPU path: "cpu" and CPU
devices raise.

ExactLlama(c, device, n_layers, gemm, compiled, cpu_lazy) runs the reference's layer sequence
(src/bitexact/exact/model.py:107-157) through Segs over the contiguous int32 Cache; attention over the cache is
the fused prefill kernel (the same integers as bmm -> softmax -> bmm).
"""

import torch

from bitexact.exact import ops
from bitexact.exact.attention import prefill as attention_prefill
from bitexact.exact.consts import FR, dims
from bitexact.exact.segs import Segs
from bitexact.exact.wmm import wmm_hip
from bitexact.llama import Cache
from bitexact.vllm_plugin.exact_gemm import exact_linear

GEMMS = ("hip", "triton", "cublas")


def validate_ell(cnt, ec, R, K):
    """Load-time check of an ELL residual (cnt int32 [N], ec int32 [N, >= R]): counts in [0, R] and every listed
    column in [0, K). The kernels never read outside q on bad data (they raise the flag instead), but a damaged
    weight file must fail here, where it is loaded, with an AssertionError."""
    if R == 0:
        return
    cnt = cnt.long()
    assert int(cnt.min()) >= 0 and int(cnt.max()) <= R, "ELL residual: a row count outside [0, R]"
    assert ec.shape[1] >= R, "ELL residual: fewer column slots than R"
    used = torch.arange(ec.shape[1], device=ec.device)[None, :] < cnt[:, None]
    cols = ec.long()[used]
    assert cols.numel() == 0 or (int(cols.min()) >= 0 and int(cols.max()) < K), \
        "ELL residual: a column index outside [0, K)"


class Lin:
    def __init__(self, c, name, device, gemm="hip", ell=True, R=0, cpu_lazy=False):
        dev = torch.device(device)
        if dev.type != "cuda":
            raise AssertionError("bitexact (MI355X) Lin runs on the GPU only")
        assert gemm in GEMMS, f"gemm must be one of {GEMMS} (no CPU path)"
        t = lambda k: c[f"{name}.{k}"].to(dev)
        self.limbs = t("limbs").contiguous()
        self.N = self.limbs.shape[1]
        self.g, self.d = t("g").long(), t("d").long()
        self.rr, self.rc, self.rv = t("rr").long(), t("rc").long(), t("rv").long()
        self.gemm = gemm
        self.ell = True
        if f"{name}.ell_cnt" in c:                    # already in ELL form (consts.decompose on the device)
            self.R = max(R, int(c[f"{name}.R"]))
            self.cnt = t("ell_cnt").to(torch.int32).contiguous()
            ec, ev = t("ell_col").to(torch.int32), t("ell_val").long()
            if ec.shape[1] < max(self.R, 1):
                pad = max(self.R, 1) - ec.shape[1]
                ec = torch.nn.functional.pad(ec, (0, pad))
                ev = torch.nn.functional.pad(ev, (0, pad))
            self.ec, self.ev = ec.contiguous(), ev.contiguous()
            validate_ell(self.cnt, self.ec, self.R, self.limbs.shape[2])
            return
        rr = self.rr.cpu()
        cnt = torch.bincount(rr, minlength=self.N) if rr.numel() else torch.zeros(self.N, dtype=torch.long)
        self.R = max(R, int(cnt.max()) if rr.numel() else 0)
        start = torch.cumsum(cnt, 0) - cnt
        j = torch.arange(rr.numel()) - start[rr]
        ec = torch.zeros(self.N, max(self.R, 1), dtype=torch.int32)
        ev = torch.zeros(self.N, max(self.R, 1), dtype=torch.long)
        if rr.numel():
            ec[rr, j] = self.rc.cpu().to(torch.int32)
            ev[rr, j] = self.rv.cpu()
        validate_ell(cnt, ec, self.R, self.limbs.shape[2])
        self.cnt = cnt.to(torch.int32).to(dev)
        self.ec, self.ev = ec.to(dev), ev.to(dev)

    def __call__(self, q):
        """(C, rs, d, g) as the reference's Lin: C = exact dense products [1, M, N], rs = (q, ec, ev)."""
        return wmm_hip(q, self.limbs), (q, self.ec.long(), self.ev), self.d, self.g

    def y(self, q, sh, checked=True, flag=None):
        """The fused linear: (y int64 [M, N] at FR, flag int32 [1])."""
        if flag is None:
            flag = torch.zeros(1, dtype=torch.int32, device=q.device)
        return exact_linear(q, sh, self.limbs, self.d, self.g, self.cnt, self.ec, self.ev, self.R, flag,
                            checked), flag


class ExactLlama:
    """The reference's ExactLlama (src/bitexact/exact/model.py:73-157). gemm: "hip" / "triton" / "cublas" (all
    served by the HIP kernels); compiled: Segs(compiled) (same integers); cpu_lazy is accepted for signature
    parity (there is no CPU path)."""

    FR = FR

    def __init__(self, c, device, n_layers=None, gemm="hip", compiled=False, cpu_lazy=False):
        self.dev = torch.device(device)
        if self.dev.type != "cuda":
            raise AssertionError("bitexact (MI355X) ExactLlama runs on the GPU only")
        self.L = c["n_layers"] if n_layers is None else n_layers
        t = lambda k: c[k].to(self.dev)
        self.emb = t("emb").to(torch.int32).contiguous()
        self.layers = []
        for i in range(self.L):
            ly = {n: Lin(c, f"{i}.{n}", self.dev, gemm) for n in ("wqkv", "wo", "wgu", "wd")}
            for n in ("ga", "gm"):
                ly[n] = (t(f"{i}.{n}.m").long(), t(f"{i}.{n}.e").long())
            self.layers.append(ly)
        self.gf = (t("gf.m").long(), t("gf.e").long())
        self.lm = Lin(c, "lm", self.dev, gemm)
        self.cos, self.sin, self.exp2 = t("cos").long(), t("sin").long(), t("exp2").long()
        self.ln = c["ln"].to(self.dev) if "ln" in c else None
        self.err = torch.zeros((), dtype=torch.bool, device=self.dev)
        self.sha = c.get("sha256")
        self.H, self.HKV, self.HD, self.D, _ = dims(c.get("cfg", {}))
        assert self.emb.shape[1] == self.D, "constants config does not match the embedding width"
        self.sg = Segs(compiled, (self.H, self.HKV, self.HD))

    def _layer(self, i, x, q, sh, pos, cache, S, err):
        """One decoder layer from x and its normalized input (q, sh); returns the next (x, q, sh, err)."""
        B, T, _ = x.shape
        ly = self.layers[i]
        qg, shg, k, v, err = self.sg.qkv(*ly["wqkv"](q), sh, pos, self.cos, self.sin, B, T, err)
        cache.write(i, k, v, pos)
        Z, hd = B * self.HKV, self.HD
        Kc = cache.k[i][:, :, :S].reshape(Z, S, hd)
        Vc = cache.v[i][:, :, :S].reshape(Z, S, hd)
        g = qg.shape[1] // T
        qpos = pos[:, None, None, :].expand(B, self.HKV, g, T).reshape(Z, g * T, 1)
        num, den = attention_prefill(qg, shg, Kc, Vc, qpos, self.exp2, self.sg.l2e)
        qo, sho = self.sg.attn_out(num, den, T)
        x, q, sh, err = self.sg.add_norm(*ly["wo"](qo), sho, x, *ly["gm"], err)
        q, sh, err = self.sg.gu_silu(*ly["wgu"](q), sh, self.exp2, err)
        nxt = self.layers[i + 1]["ga"] if i + 1 < self.L else self.gf
        return self.sg.add_norm(*ly["wd"](q), sh, x, *nxt, err)

    def forward_q(self, ids, pos, cache, S=None):
        """ids, pos int64 [B, T]; writes K / V at pos. Returns the final residual stream [B, T, D] at FR and its
        final-norm quantization (q, sh). S: keys attended (default max(pos) + 1)."""
        B, T = ids.shape
        pos = pos.long()
        S = int(pos.max()) + 1 if S is None else S
        x, q, sh, err = ops.embed_norm(self.emb, ids, *self.layers[0]["ga"], self.err)
        x = x.view(B, T, self.D)
        for i in range(self.L):
            x, q, sh, err = self._layer(i, x, q, sh, pos, cache, S, err)
        self.err = err
        return x, q, sh

    def forward(self, ids, pos, cache, S=None):
        return self.forward_q(ids, pos, cache, S)[0]

    def logits_q(self, q, sh):
        """Final-norm rows (q, sh) -> logits int64 [M, V] at FR."""
        y, flag = self.sg.lin_out(*self.lm(q), sh)
        self.err = self.err | flag
        return y

    def logits(self, x):
        """Final residual rows [M, D] -> logits int64 [M, V] at FR."""
        return self.logits_q(*self.sg.pre_norm(x.reshape(-1, self.D), *self.gf))

    def new_cache(self, B, L):
        return Cache(self.L, B, L, self.dev, self.HKV, self.HD)

    def check(self):
        if bool(self.err):
            raise OverflowError("integer bound violated (exact/model.py)")
