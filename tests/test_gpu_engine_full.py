"""The config-5 engine at the full Llama-3.2-1B geometry (16 layers, D 2048, FF 8192, V 128256, random-init bf16
weights) at config 5's context of 1024 tokens: batch-32 prefill, then a sequence's first decode logits hash is the
same at batch 1, 8 and 32 (the reference's batch-invariance guarantee, src/bitexact/vllm_plugin/exact_run.py:106-175),
and the lm_head at M = 32 (the stream kernel) equals the oracle on a column sample that covers every 64-column tile
edge. A one-layer model of the same geometry is checked against the oracle engine (oracle.engine_forward) on a
1024-token prefill and the decode step after it, residual stream bit for bit."""

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu

BS, CTX, B = 16, 1024, 32
CHUNK = 4                     # sequences per prefill call (4096 token rows)


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
    first = torch.empty(B, dtype=torch.long, device=dev)
    for s0 in range(0, B, CHUNK):
        seqs = torch.arange(s0, s0 + CHUNK, device=dev)
        pos = torch.arange(CTX, device=dev).repeat(CHUNK)
        rmap = seqs.repeat_interleave(CTX)
        slot = bt[rmap, pos // BS].long() * BS + pos % BS
        x = eng.forward(kvs, prompts[s0:s0 + CHUNK].reshape(-1), pos, slot, bt, rmap)
        first[s0:s0 + CHUNK] = eng.greedy(eng.logits(x.view(CHUNK, CTX, -1)[:, -1].contiguous()))
    shas, h32 = {}, None
    for b in (1, 8, B):
        p = torch.full((b,), CTX, device=dev, dtype=torch.long)
        rm = torch.arange(b, device=dev)
        sl = bt[rm, p // BS].long() * BS + p % BS
        h = eng.forward(kvs, first[:b], p, sl, bt, rm, one_per_seq=True)   # b = 32: the fused rope + attention
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


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


@pytest.mark.timeout(600)
def test_full_geometry_layer_against_oracle(dev):
    """One layer at the full geometry (D 2048, 32 / 8 heads of 64, FF 8192): a 1024-token prefill of one sequence
    and the decode step after it, the residual stream against the oracle engine bit for bit (the lm_head's columns
    are covered above; the engine reads the full 128256-row embedding, the oracle only the rows the steps use)."""
    from bitexact.exact.consts import random_constants
    from bitexact.vllm_plugin.exact_run import ExactEngine
    c = random_constants(None, n_layers=1, seed=3, device=dev, keep_bf16=True)
    eng = ExactEngine(c, dev)
    H, HKV, HD = eng.H, eng.HKV, eng.HD
    lin = {(0, n): _bits(c[f"0.{n}.bf16"]) for n in ("wqkv", "wo", "wgu", "wd")}
    gam = {k: (c[f"{k}.m"].cpu().numpy(), c[f"{k}.e"].cpu().numpy()) for k in ("0.ga", "0.gm", "gf")}
    g = torch.Generator().manual_seed(9)
    ids_all = torch.randint(0, eng.V, (CTX + 1,), generator=g)
    # the oracle gets only the embedding rows the two steps read (its table conversion is per row), ids remapped
    used, inv = torch.unique(ids_all, return_inverse=True)
    om = R.engine_constants(_bits(c["emb.bf16"][used.to(dev)]), lin, gam, c["cos"].cpu().numpy(),
                            c["sin"].cpu().numpy(), 1)
    del c
    nblk = -(-(CTX + 2) // BS)
    bt = (1 + torch.arange(nblk, dtype=torch.int32)).view(1, nblk)
    kvs = eng.new_cache(1 + nblk, BS)
    c32 = [np.zeros((1 + nblk, HKV, BS, 2 * HD), np.int64)]
    ids, oids = ids_all[:CTX], inv[:CTX]
    pos = torch.arange(CTX)
    rmap = torch.zeros(CTX, dtype=torch.long)
    for step in range(2):
        slot = bt[rmap, pos // BS].long() * BS + pos % BS
        print(f"layer check: step {step}, {ids.numel()} rows", flush=True)
        x = eng.forward(kvs, ids.to(dev), pos.to(dev), slot.to(dev), bt.to(dev), rmap.to(dev))
        xr, err = R.engine_forward(om, c32, oids.numpy(), pos.numpy(), slot.numpy(), bt.numpy(), rmap.numpy(),
                                   (H, HKV, HD))
        got = x.cpu().numpy()
        assert np.array_equal(got, xr), f"step {step}: {int((got != xr).any(1).sum())} rows differ"
        assert bool(eng.err) == err
        ids, oids = ids_all[CTX:], inv[CTX:]
        pos = torch.tensor([CTX])
        rmap = torch.zeros(1, dtype=torch.long)
