"""Exact-mode linear layer over a constants dict (src/bitexact/exact/model.py:31-70), gemm = "hip".

Lin(c, name, device) reads c[f"{name}.limbs" | ".g" | ".d" | ".rr" | ".rc" | ".rv"] (the reference's key
layout) and builds the ELL residual once (src/bitexact/exact/model.py:39-48). __call__(q) keeps the
reference's (C, rs, d, g) contract for segs.lin_y; y(q, sh, checked) is the fused HIP linear.
"""

import torch

from bitexact.exact.wmm import wmm_hip
from bitexact.vllm_plugin.exact_gemm import exact_linear


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
        assert gemm == "hip", "this build has one backend: gemm='hip'"
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
