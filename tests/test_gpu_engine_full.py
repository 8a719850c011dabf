"""The config-5 engine at the full Llama-3.2-1B geometry (16 layers, D 2048, FF 8192, V 128256, random-init bf16
weights): a sequence's first decode logits hash is the same at batch 1, 8 and 32 (the reference's batch-invariance
guarantee, src/bitexact/vllm_plugin/exact_run.py:106-175), and the lm_head at M = 32 (the wide kernel) equals the
oracle on a column sample that covers every 64-column tile edge."""

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu

BS, CTX, B = 16, 64, 32


@pytest.fixture(scope="module")
def engine(dev):
    from bitexact.exact.consts import random_constants
    from bitexact.vllm_plugin.exact_run import ExactEngine
    c = random_constants(None, seed=0, device=dev, keep_bf16=True)
    lm_bf16 = c["lm.bf16"]
    eng = ExactEngine(c, dev)
    del c
    return eng, lm_bf16


def test_full_geometry_batch_invariance_and_lm_head(dev, engine):
    from bitexact.exact import ops
    from bitexact.generate import logits_sha
    from bitexact.vllm_plugin.exact_gemm import plan
    eng, lm_bf16 = engine
    assert (eng.L, eng.D, eng.V) == (16, 2048, 128256)
    nblk = -(-(CTX + 2) // BS)
    bt = (1 + torch.arange(B * nblk, device=dev, dtype=torch.int32)).view(B, nblk)
    kvs = eng.new_cache(1 + B * nblk, BS)
    g = torch.Generator().manual_seed(5)
    prompts = torch.randint(0, eng.V, (B, CTX), generator=g).to(dev)
    pos = torch.arange(CTX, device=dev).repeat(B)
    rmap = torch.arange(B, device=dev).repeat_interleave(CTX)
    slot = bt[rmap, pos // BS].long() * BS + pos % BS
    x = eng.forward(kvs, prompts.reshape(-1), pos, slot, bt, rmap)
    first = eng.greedy(eng.logits(x.view(B, CTX, -1)[:, -1].contiguous()))
    shas, h32 = {}, None
    for b in (1, 8, B):
        p = torch.full((b,), CTX, device=dev, dtype=torch.long)
        rm = torch.arange(b, device=dev)
        sl = bt[rm, p // BS].long() * BS + p % BS
        h = eng.forward(kvs, first[:b], p, sl, bt, rm)
        lg = eng.logits(h)
        shas[b] = logits_sha(lg[0])
        if b == B:
            h32, lg32 = h, lg
    assert len(set(shas.values())) == 1, shas
    assert not bool(eng.err)
    # the lm_head at M = 32 on the stream kernel against the oracle, columns at every 64-column tile edge + random
    assert plan(B, eng.V, eng.D)[0] == "stream"
    q, sh, _ = ops.norm_quant(h32, *eng.gf)
    cols = np.unique(np.concatenate([np.arange(0, eng.V, 64), np.arange(63, eng.V, 64),
                                     np.random.default_rng(2).integers(0, eng.V, 256)]))
    dec = R.decompose(lm_bf16[torch.from_numpy(cols).to(dev)].contiguous().view(torch.int16).cpu().numpy())
    qn, shn = q.cpu().numpy().astype(np.int64), sh.cpu().numpy()
    ref, _, _ = R.epilogue(R.wmm_f64(qn, dec["W"]), R.residual(qn, dec["rr"], dec["rc"], dec["rv"], len(cols)),
                           dec["d"], dec["g"], shn, R.FR, True)
    got = lg32[:, torch.from_numpy(cols).to(dev)].cpu().numpy()
    assert np.array_equal(got, ref), int((got != ref).sum())
