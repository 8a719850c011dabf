"""Exact-mode decode engine on the paged limb-plane KV cache (src/bitexact/vllm_plugin/exact_run.py:22-175).

Every token of the step is a row: it is embedded and normalised, goes through the fused exact linears, RoPE and
q quantization, is stored into its layer's paged cache (K at FK = 17, V at FV = 19 bits, 3 int8 limb planes)
and attends its own sequence's keys through its block-table row; attention output, residual adds, RMSNorms,
SiLU gating and the logits follow the reference's stages. Every rule is row-local, so the batch a token
shares a step with cannot change a bit of its logits. One HIP launch per stage; no host synchronisation, so a
step can be captured in a HIP graph.
"""

import torch

from bitexact import _hip
from bitexact._ops import op
from bitexact.exact import ops
from bitexact.exact.consts import FR, dims
from bitexact.exact.model import GEMMS, Lin
from bitexact.intops import first_argmax
from bitexact.vllm_plugin import tri_exact_attn, tri_paged
from bitexact.vllm_plugin.exact_gemm import FusedLin

NAMES = ("wqkv", "wo", "wgu", "wd")


class ExactEngine:
    """c: constants dict with the reference's keys (exact.consts.build, or random_constants here)."""

    def __init__(self, c, dev, compiled=False, gemm="triton"):
        """compiled / gemm: the reference's arguments (exact_run.py:24). Every stage here is already one HIP launch
        and every gemm value is served by the HIP linear (the same integers), so neither changes the kernels."""
        dev = torch.device(dev)
        if dev.type != "cuda":
            raise AssertionError("bitexact (MI355X) ExactEngine runs on the GPU only")
        assert gemm in GEMMS, f"gemm must be one of {GEMMS}"
        self.compiled, self.gemm = compiled, gemm
        self.dev = dev
        self.L = c["n_layers"]
        self.H, self.HKV, self.HD, self.D, self.FF = dims(c.get("cfg", {}))
        self.G = self.H // self.HKV
        self.FR = FR
        self.l2e = ops.L2E28_HD[self.HD]                        # KeyError: unsupported head_dim
        t = lambda k: c[k].to(dev)
        self.emb = t("emb").to(torch.int32).contiguous()
        assert self.emb.shape[1] == self.D, "constants config does not match the embedding width"
        self.fused = {(i, n): FusedLin(Lin(c, f"{i}.{n}", dev)) for i in range(self.L) for n in NAMES}
        self.fused["lm"] = FusedLin(Lin(c, "lm", dev))
        self.V = self.fused["lm"].N
        gam = lambda k: (t(f"{k}.m").long().contiguous(), t(f"{k}.e").long().contiguous())
        self.ga = [gam(f"{i}.ga") for i in range(self.L)]
        self.gm = [gam(f"{i}.gm") for i in range(self.L)]
        self.gf = gam("gf")
        self.cos, self.sin, self.exp2 = t("cos").long(), t("sin").long(), t("exp2").long()
        self.ln = c["ln"].to(dev) if "ln" in c else None
        self.sha = c.get("sha256")
        # one sticky int32 flag for every bound check of every stage (the reference's fl and err together)
        self.fl = torch.zeros(1, dtype=torch.int32, device=dev)

    @property
    def err(self):
        """The bound flag as a bool tensor (no host sync)."""
        return self.fl[0] != 0

    def new_cache(self, nblocks, bs=16):
        """One limb-plane cache per layer: int8 [nblocks, HKV, bs, 8 HD] (block 0 is the null block)."""
        return [torch.zeros(nblocks, self.HKV, bs, 8 * self.HD, dtype=torch.int8, device=self.dev)
                for _ in range(self.L)]

    def forward(self, kvs, ids, pos, slot, bt, rmap, one_per_seq=False):
        """ids, pos, slot [N]: the step's tokens (slot < 0: padding, redirected to the null block 0); bt [*, nblk]
        int32 block table and rmap [N] the table row of each token. kvs None: no cache (the reference's memory
        profiling run): nothing is stored and the attention output is 0. Returns the residual stream [N, D] int64
        at FR (src/bitexact/vllm_plugin/exact_run.py:55-128 with the fused stages of its 130-155).
        one_per_seq: every token is the only one of its sequence in this step (a decode step), so each layer's
        RoPE + KV store, attention and attention output stage run as one launch (tri_exact_attn.rope_attend_out)
        where the shapes allow; the integers are the same either way."""
        N, G, HKV, HD = ids.shape[0], self.G, self.HKV, self.HD
        pos = pos.long().contiguous()
        slot = slot.long().clamp(min=0)    # padding (slot < 0) -> the null block 0; one launch
        fl = self.fl
        pl = None                             # q's limb planes, when the norm before the layer wrote them
        if self.fused[0, "wqkv"].needs_planes(N):
            x, (q, pl), sh, _ = ops.embed_norm(self.emb, ids, *self.ga[0], flag=fl, planes=True)
        else:
            x, q, sh, _ = ops.embed_norm(self.emb, ids, *self.ga[0], flag=fl)
        fuse = (one_per_seq and kvs is not None and
                tri_exact_attn.rope_fusable(N, HKV, self.H, bt.shape[1], kvs[0].shape[2]))
        # the query positions per q head of a group (the split attention's input; the fused launch reads pos)
        qpos = None if fuse else pos.view(-1, 1).expand(-1, G).contiguous()
        for i in range(self.L):
            y = self.fused[i, "wqkv"](q, sh, fl, False, q_planes=pl)
            plo = None                        # the wo linear's limb planes, when the output stage writes them
            if fuse:   # RoPE + KV store + attention + the attention output stage in one launch
                if self.fused[i, "wo"].needs_planes(N):
                    qo, sho, plo = tri_exact_attn.rope_attend_out(y, pos, self.cos, self.sin, (self.H, HKV, HD),
                                                                  kvs[i], slot, bt, rmap, self.exp2, self.l2e, fl,
                                                                  planes=True)
                else:
                    qo, sho = tri_exact_attn.rope_attend_out(y, pos, self.cos, self.sin, (self.H, HKV, HD), kvs[i],
                                                             slot, bt, rmap, self.exp2, self.l2e, fl)
            elif kvs is None:
                ops.qkv_y(y, pos.view(N, 1), self.cos, self.sin, N, 1, (self.H, HKV, HD), flag=fl)
                num = torch.zeros(N, HKV, G, HD, dtype=torch.long, device=y.device)
                den = torch.ones(N, HKV, G, 1, dtype=torch.long, device=y.device)
            else:
                qg, shg, _, _, _ = ops.qkv_y(y, pos.view(N, 1), self.cos, self.sin, N, 1, (self.H, HKV, HD),
                                             flag=fl, store=(kvs[i], slot))   # K / V into the cache (exact_fuse.qkv)
                num, den = tri_exact_attn.attend(qg.view(N, HKV, G, HD), shg.view(N, HKV, G), qpos, kvs[i], bt,
                                                 rmap, self.exp2, self.l2e)
            if not fuse:
                qo, sho = ops.attn_out(num.view(N * HKV, G, HD), den.view(N * HKV, G, 1), 1, HKV)
            wgu = self.fused[i, "wgu"]
            if wgu.needs_planes(N):   # the norm kernel also writes q's limb planes for the MFMA path
                x, (q, pl), sh, _ = ops.add_norm_y(self.fused[i, "wo"](qo, sho, fl, True, q_planes=plo), x,
                                                   *self.gm[i], flag=fl, planes=True)
                y = wgu(q, sh, fl, False, q_planes=pl)
            else:
                x, q, sh, _ = ops.add_norm_y(self.fused[i, "wo"](qo, sho, fl, True, q_planes=plo), x, *self.gm[i],
                                             flag=fl)
                y = wgu(q, sh, fl, False)
            wd = self.fused[i, "wd"]
            # the column-chunked SiLU stage also writes q's limb planes for the MFMA path; measured only for the
            # few-row decode case (the chunked stage's own range), so prefill-sized steps keep the row kernel
            if N < ops.SILU_SPLIT_ROWS and wd.needs_planes(N):
                (q, pl), sh, _ = ops.gu_silu_y(y, self.exp2, flag=fl, planes=True)
                yd = wd(q, sh, fl, True, q_planes=pl)
            else:
                q, sh, _ = ops.gu_silu_y(y, self.exp2, flag=fl)
                yd = wd(q, sh, fl, True)
            nxt = self.ga[i + 1] if i + 1 < self.L else (None, None)
            pl = None
            if nxt[0] is not None and self.fused[i + 1, "wqkv"].needs_planes(N):
                x, (q, pl), sh, _ = ops.add_norm_y(yd, x, *nxt, flag=fl, planes=True)
            else:
                x, q, sh, _ = ops.add_norm_y(yd, x, *nxt, flag=fl)
        return x

    def logits(self, h):
        """Final residual rows [M, D] -> logits int64 [M, V] at FR (exact_run.py:157-175)."""
        lm = self.fused["lm"]
        if lm.needs_planes(h.shape[0]):   # the norm kernel writes q's limb planes: no split launch
            (q, pl), sh, _ = ops.norm_quant(h, *self.gf, flag=self.fl, planes=True)
            return lm(q, sh, self.fl, True, q_planes=pl)
        q, sh, _ = ops.norm_quant(h, *self.gf, flag=self.fl)
        return lm(q, sh, self.fl, True)

    def greedy(self, logits):
        """The greedy token of each logits row: its first maximum."""
        return first_argmax(logits)

    def advance(self, logits, ids, pos, slot, bt, rmap, bs=16):
        """A greedy decode step's next inputs, in place: ids = greedy(logits), pos += 1, slot = the new position's
        cache slot (bt[rmap, pos // bs] bs + pos % bs, bs the cache block size): the first-max kernels and one
        launch for the rest (the reference leaves this loop to its caller)."""
        _advance(self.greedy(logits), ids, pos, slot, bt, rmap, int(bs))

    def check(self):
        if bool(self.err):
            raise OverflowError("integer bound violated (exact/model.py)")


@op("decode_advance(Tensor nxt, Tensor(a!) ids, Tensor(b!) pos, Tensor(c!) slot, Tensor bt, Tensor rmap, int bs) -> ()",
    lambda nxt, ids, pos, slot, bt, rmap, bs: None)
def _advance(nxt, ids, pos, slot, bt, rmap, bs):
    _hip.require_cuda(nxt, ids, pos, slot, bt, rmap)
    N = ids.shape[0]
    for t in (nxt, ids, pos, slot, rmap):
        assert t.dtype == torch.int64 and t.is_contiguous() and t.shape == (N,)
    assert bt.dtype == torch.int32 and bt.dim() == 2 and bt.stride(1) == 1
    _hip.call("bx_decode_advance", _hip.ptr(nxt), _hip.ptr(ids), _hip.ptr(pos), _hip.ptr(slot), _hip.ptr(bt),
              bt.stride(0), bt.shape[1], _hip.ptr(rmap), bs, N, _hip.stream_of(ids))
