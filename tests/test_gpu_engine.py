"""The exact decode engine (ExactEngine: embedding, fused linears, RoPE, paged KV store and attention, attention
output, residual adds and norms, SiLU gating, tied lm_head, greedy first-max) against the oracle's restatement
of the reference's engine, bit for bit, on a small random-init Llama; and the batch invariance the reference
guarantees (a sequence's logits hash does not depend on the batch it is decoded in)."""

import numpy as np
import pytest
import torch

from oracle import bxref as R

pytestmark = pytest.mark.gpu

CFG = {"hidden_size": 256, "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 64,
       "intermediate_size": 512, "vocab_size": 300, "num_hidden_layers": 2}
BS, NBLK = 16, 4


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _oracle_model(c):
    L = c["n_layers"]
    lin = {(i, n): _bits(c[f"{i}.{n}.bf16"]) for i in range(L) for n in ("wqkv", "wo", "wgu", "wd")}
    lin["lm"] = _bits(c["lm.bf16"])
    gam = {k: (c[f"{k}.m"].cpu().numpy(), c[f"{k}.e"].cpu().numpy()) for k in
           [f"{i}.{n}" for i in range(L) for n in ("ga", "gm")] + ["gf"]}
    return R.engine_constants(_bits(c["emb.bf16"]), lin, gam, c["cos"].cpu().numpy(), c["sin"].cpu().numpy(), L)


def _rows(seqs, starts, lens, bt):
    """Token rows of a step: for each sequence j, positions starts[j] .. starts[j] + lens[j] - 1."""
    pos, slot, rmap = [], [], []
    for j, (s0, n) in enumerate(zip(starts, lens)):
        for p in range(s0, s0 + n):
            pos.append(p)
            slot.append(int(bt[seqs[j], p // BS]) * BS + p % BS)
            rmap.append(seqs[j])
    return torch.tensor(pos), torch.tensor(slot), torch.tensor(rmap)


@pytest.fixture(scope="module")
def model(dev):
    from bitexact.exact.consts import random_constants
    from bitexact.vllm_plugin.exact_run import ExactEngine
    c = random_constants(CFG, seed=11, device=dev, keep_bf16=True)
    return ExactEngine(c, dev), _oracle_model(c)


def test_engine_matches_oracle(dev, model):
    eng, om = model
    H, HKV, HD = eng.H, eng.HKV, eng.HD
    g = torch.Generator().manual_seed(3)
    lens = [5, 17, 1]
    nseq = len(lens)
    bt = (1 + torch.arange(nseq * NBLK).view(nseq, NBLK)).to(torch.int32)
    kvs = eng.new_cache(1 + nseq * NBLK, BS)
    c32 = [np.zeros((1 + nseq * NBLK, HKV, BS, 2 * HD), np.int64) for _ in range(eng.L)]
    ids = torch.randint(0, eng.V, (sum(lens),), generator=g)
    pos, slot, rmap = _rows(list(range(nseq)), [0] * nseq, lens, bt)
    last = np.cumsum(lens) - 1
    for step in range(3):
        x = eng.forward(kvs, ids.to(dev), pos.to(dev), slot.to(dev), bt.to(dev), rmap.to(dev))
        xr, err = R.engine_forward(om, c32, ids.numpy(), pos.numpy(), slot.numpy(), bt.numpy(), rmap.numpy(),
                                   (H, HKV, HD))
        assert np.array_equal(x.cpu().numpy(), xr), f"residual stream differs at step {step}"
        h = x[torch.as_tensor(last).to(dev)]
        lg = eng.logits(h)
        lr, f = R.engine_logits(om, xr[last])
        assert np.array_equal(lg.cpu().numpy(), lr), f"logits differ at step {step}"
        assert bool(eng.err) == (err or f)
        tok = eng.greedy(lg).cpu()
        assert np.array_equal(tok.numpy(), np.array([R.first_argmax(r) for r in lr]))
        # next step: one token per sequence at the next position
        starts = [int(pos[last[j]]) + 1 for j in range(nseq)]
        ids = tok
        pos, slot, rmap = _rows(list(range(nseq)), starts, [1] * nseq, bt)
        last = np.arange(nseq)


def test_batch_invariance(dev, model):
    """Sequence A decoded alone and inside a batch of 5 with padding rows: identical logits hashes."""
    from bitexact.generate import logits_sha
    eng, _ = model
    g = torch.Generator().manual_seed(8)
    prompt = torch.randint(0, eng.V, (9,), generator=g)
    others = [torch.randint(0, eng.V, (n,), generator=g) for n in (3, 12, 7, 1)]

    def run(batch):                         # batch: list of prompts; sequence 0 is A
        nseq = len(batch)
        bt = (1 + torch.arange(nseq * NBLK).view(nseq, NBLK)).to(torch.int32)
        bt = bt.flip(0).contiguous()                         # A's blocks differ between the runs
        kvs = eng.new_cache(1 + nseq * NBLK, BS)
        lens = [len(p) for p in batch]
        ids = torch.cat(batch)
        pos, slot, rmap = _rows(list(range(nseq)), [0] * nseq, lens, bt)
        # two padding rows (slot -1 -> null block 0)
        ids = torch.cat([ids, torch.tensor([0, 1])])
        pos, rmap = torch.cat([pos, torch.tensor([0, 0])]), torch.cat([rmap, torch.tensor([0, 0])])
        slot = torch.cat([slot, torch.tensor([-1, -1])])
        shas = []
        last = np.cumsum(lens) - 1
        for step in range(3):
            x = eng.forward(kvs, ids.to(dev), pos.to(dev), slot.to(dev), bt.to(dev), rmap.to(dev))
            lg = eng.logits(x[torch.as_tensor(last).to(dev)])
            shas.append(logits_sha(lg[0]))
            tok = eng.greedy(lg).cpu()
            starts = [int(pos[last[j]]) + 1 for j in range(nseq)]
            ids = tok
            pos, slot, rmap = _rows(list(range(nseq)), starts, [1] * nseq, bt)
            last = np.arange(nseq)
        return shas

    alone = run([prompt])
    batched = run([prompt] + others)
    assert alone == batched


def test_constants_file_roundtrip(dev, tmp_path):
    """A random-init constants dict saved to a safetensors file and loaded back gives the same identity and the
    same logits."""
    from bitexact.exact import consts
    from bitexact.vllm_plugin.exact_run import ExactEngine
    c = consts.random_constants(CFG, n_layers=1, seed=4, device=dev, with_sha=True)
    f = str(tmp_path / "m.safetensors")
    consts.save(c, f)
    c2 = consts.load(f, dev)
    assert c2["sha256"] == c["sha256"] == consts.sha256(c2)
    ids = torch.tensor([5, 7, 11], device=dev)
    pos = torch.arange(3, device=dev)
    bt = torch.arange(1, 1 + NBLK, dtype=torch.int32, device=dev).view(1, NBLK)
    slot = bt[0, pos // BS].long() * BS + pos % BS
    rmap = torch.zeros(3, dtype=torch.long, device=dev)
    out = []
    for cc in (c, c2):
        eng = ExactEngine(cc, dev)
        kvs = eng.new_cache(1 + NBLK, BS)
        out.append(eng.logits(eng.forward(kvs, ids, pos, slot, bt, rmap)).cpu())
    assert torch.equal(out[0], out[1])


def test_decode_advance(dev):
    """ExactEngine.advance (first-max tokens, pos + 1 and the new slot through the block table, one launch after
    the first-max kernels) against the same update in torch ops."""
    from bitexact.vllm_plugin.exact_run import ExactEngine
    g = torch.Generator().manual_seed(3)
    N, nblk, bs, V = 37, 9, 16, 3000
    logits = torch.randint(-1000, 1000, (N, V), generator=g).to(dev)
    logits[5, 17] = logits[5, 400] = 5000                 # ties: the first maximum
    bt = torch.randint(1, 500, (N + 3, nblk), generator=g).to(torch.int32).to(dev)
    rmap = torch.randperm(N + 3, generator=g)[:N].to(dev)
    pos = torch.randint(0, nblk * bs - 1, (N,), generator=g).to(dev)
    ids = torch.zeros(N, dtype=torch.long, device=dev)
    slot = torch.zeros(N, dtype=torch.long, device=dev)
    want_ids = torch.argmax(logits, dim=1)               # torch returns the first maximum
    want_pos = pos + 1
    want_slot = bt[rmap, want_pos // bs].long() * bs + want_pos % bs
    eng = ExactEngine.__new__(ExactEngine)               # advance uses no model state
    eng.advance(logits, ids, pos, slot, bt, rmap, bs)
    assert torch.equal(ids, want_ids) and torch.equal(pos, want_pos) and torch.equal(slot, want_slot)
