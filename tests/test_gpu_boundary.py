"""The reference's Python operator surface on the HIP kernels: ExactLlama through the reference's own call sequence
(Lin -> Segs.qkv -> Cache.write -> attention -> Segs.attn_out -> Segs.add_norm -> Segs.gu_silu -> ...) against the
oracle engine, bit for bit; Segs(compiled=True) and torch.compile(fullgraph=True) over the registered
torch.ops.bitexact_hip operators (no graph break, same integers); the wmm_* entry names; opcheck of operators."""

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


@pytest.fixture(scope="module")
def consts(dev):
    from bitexact.exact.consts import random_constants
    c = random_constants(CFG, seed=21, device=dev, keep_bf16=True)
    L = c["n_layers"]
    lin = {(i, n): _bits(c[f"{i}.{n}.bf16"]) for i in range(L) for n in ("wqkv", "wo", "wgu", "wd")}
    lin["lm"] = _bits(c["lm.bf16"])
    gam = {k: (c[f"{k}.m"].cpu().numpy(), c[f"{k}.e"].cpu().numpy()) for k in
           [f"{i}.{n}" for i in range(L) for n in ("ga", "gm")] + ["gf"]}
    om = R.engine_constants(_bits(c["emb.bf16"]), lin, gam, c["cos"].cpu().numpy(), c["sin"].cpu().numpy(), L)
    return c, om


def _oracle_steps(om, HKV, HD, L, ids_steps, pos_steps, dm):
    """The oracle engine over the same tokens (sequence b's blocks 1 + b NBLK ..): residual rows and logits."""
    B = ids_steps[0].shape[0]
    bt = (1 + np.arange(B * NBLK).reshape(B, NBLK)).astype(np.int32)
    c32 = [np.zeros((1 + B * NBLK, HKV, BS, 2 * HD), np.int64) for _ in range(L)]
    out = []
    for ids, pos in zip(ids_steps, pos_steps):
        T = ids.shape[1]
        rmap = np.repeat(np.arange(B), T)
        p = pos.reshape(-1)
        slot = bt[rmap, p // BS].astype(np.int64) * BS + p % BS
        x, err = R.engine_forward(om, c32, ids.reshape(-1), p, slot, bt, rmap, dm)
        lg, f = R.engine_logits(om, x)
        out.append((x, lg, err or f))
    return out


@pytest.mark.parametrize("compiled", [False, True])
def test_exact_llama_reference_sequence(dev, consts, compiled):
    """ExactLlama (contiguous Cache, Segs stages, fused attention) = the oracle engine: prefill 2 x 5 tokens, then
    two greedy decode steps; residual stream, logits, greedy tokens and the bound flag."""
    from bitexact.exact.model import ExactLlama
    c, om = consts
    m = ExactLlama(c, dev, compiled=compiled)
    assert m.sg.compiled == compiled
    cache = m.new_cache(2, 32)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 300, (2, 5), generator=g)
    pos = torch.arange(5).repeat(2, 1)
    ids_steps, pos_steps, got = [], [], []
    for step in range(3):
        ids_steps.append(ids.numpy())
        pos_steps.append(pos.numpy())
        x = m.forward(ids.to(dev), pos.to(dev), cache)
        lg = m.logits(x.reshape(-1, m.D))
        got.append((x.reshape(-1, m.D).cpu().numpy(), lg.cpu().numpy()))
        nxt = torch.from_numpy(np.array([R.first_argmax(r) for r in lg.view(2, -1, lg.shape[-1])[:, -1].cpu().numpy()]))
        ids = nxt.view(2, 1)
        pos = pos[:, -1:] + 1
    ref = _oracle_steps(om, m.HKV, m.HD, m.L, ids_steps, pos_steps, (m.H, m.HKV, m.HD))
    for step, ((x, lg), (xr, lr, _)) in enumerate(zip(got, ref)):
        assert np.array_equal(x, xr), f"residual stream differs at step {step}"
        assert np.array_equal(lg, lr), f"logits differ at step {step}"
    assert bool(m.err) == any(e for _, _, e in ref)
    m.check() if not bool(m.err) else None


def test_torch_compile_no_graph_break(dev, consts):
    """One decode step's stage chain under torch.compile(fullgraph=True): every kernel is a registered operator
    with a fake implementation, so the trace has no graph break, and the integers equal the eager ones."""
    from bitexact.exact import ops
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    from bitexact.exact.model import Lin
    c, _ = consts
    lin = Lin(c, "0.wo", dev)
    gm, ge = c["0.gm.m"].to(dev).long(), c["0.gm.e"].to(dev).long()
    g = torch.Generator().manual_seed(9)
    x0 = torch.randint(-(1 << 30), 1 << 30, (6, lin.N), generator=g).to(dev)
    q = torch.randint(-(1 << 22), 1 << 22, (6, lin.limbs.shape[2]), generator=g).to(torch.int32).to(dev)
    sh = torch.full((6,), -30, dtype=torch.long, device=dev)

    def chain(x, q, sh, flag):
        y = exact_linear(q, sh, lin.limbs, lin.d, lin.g, lin.cnt, lin.ec, lin.ev, lin.R, flag, True)
        x2, q2, sh2, err = ops.add_norm_y(y, x, gm, ge, flag=flag)
        return x2, q2, sh2, flag[0] != 0

    f_e = torch.zeros(1, dtype=torch.int32, device=dev)
    xe = x0.clone()
    eager = chain(xe, q, sh, f_e)
    f_c = torch.zeros(1, dtype=torch.int32, device=dev)
    xc = x0.clone()
    comp = torch.compile(chain, fullgraph=True, backend="aot_eager")(xc, q, sh, f_c)
    for a, b in zip(eager, comp):
        assert torch.equal(a, b)
    assert torch.equal(xe, xc) and torch.equal(f_e, f_c)


def test_wmm_entry_names(dev):
    """wmm_triton / wmm_cublas / residual / epilogue under the reference's names and contracts, against the oracle;
    wmm_cpu has no CPU path and raises."""
    from bitexact.exact.consts import decompose
    from bitexact.exact.wmm import epilogue, residual, wmm_cpu, wmm_cublas, wmm_triton
    N, K, M = 96, 256, 7
    g = torch.Generator().manual_seed(2)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    w[0, :3] = torch.tensor([1e-9, 2.0, -3e-8]).to(torch.bfloat16)
    ref = R.decompose(w.view(torch.int16).numpy())
    dec = decompose(w.to(dev))
    q = np.random.default_rng(3).integers(-(1 << 22), (1 << 22) + 1, (M, K))
    qd = torch.from_numpy(q).to(torch.int32).to(dev)
    T = R.wmm_f64(q, ref["W"])
    C = wmm_triton(qd, dec["limbs"])
    assert C.dim() == 3 and np.array_equal(C.sum(0).cpu().numpy(), T)
    assert np.array_equal(wmm_cublas(qd, dec["limbs"].reshape(3 * N, K)).cpu().numpy(), T)
    B = residual(qd, dec["rr"], dec["rc"], dec["rv"], N)
    Bref = R.residual(q, ref["rr"], ref["rc"], ref["rv"], N)
    assert np.array_equal(B.cpu().numpy(), Bref)
    sh = torch.full((M,), -30, dtype=torch.long, device=dev)
    y, flag = epilogue(C, B, dec["d"], dec["g"], sh, 24, checked=True)
    yr, fr, _ = R.epilogue(T, Bref, ref["d"], ref["g"], sh.cpu().numpy(), R.FR, True)
    assert np.array_equal(y.cpu().numpy(), yr) and bool(flag) == fr
    with pytest.raises(AssertionError):
        wmm_cpu(qd, None)


def test_opcheck_operators(dev):
    """torch.library.opcheck (schema, fake tensor, dispatch) on representative operators."""
    import bitexact.bmm  # noqa: F401  (registers bitexact_hip::bmm)
    from bitexact.exact.consts import decompose
    N, K, M = 64, 128, 5
    w = (torch.randn(N, K, generator=torch.Generator().manual_seed(1)) * 0.02).to(torch.bfloat16)
    dec = decompose(w.to(dev))
    q = torch.randint(-(1 << 22), 1 << 22, (M, K), device=dev).to(torch.int32)
    sh = torch.full((M,), -30, dtype=torch.long, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    ops = torch.ops.bitexact_hip
    torch.library.opcheck(ops.exact_linear, (q, sh, dec["limbs"], dec["d"], dec["g"], dec["ell_cnt"], dec["ell_col"],
                                             dec["ell_val"], dec["R"], flag, True, 24, None))
    a = torch.randint(-128, 128, (4, 3, 64), device=dev, dtype=torch.int32)
    b = torch.randint(-128, 128, (4, 64, 5), device=dev, dtype=torch.int32)
    torch.library.opcheck(ops.bmm, (a, b, 1, 1))
    x = torch.randint(-(1 << 40), 1 << 40, (3, 256), device=dev)
    gm = torch.randint(-255, 256, (256,), device=dev)
    ge = torch.full((256,), -8, dtype=torch.long, device=dev)
    torch.library.opcheck(ops.norm_quant, (x, gm, ge, flag))


def test_cache_write_and_lin_backends(dev, consts):
    """Cache.write puts k / v at their positions; Lin accepts the reference's gemm values (one HIP path) and no
    CPU device."""
    from bitexact.exact.model import Lin
    from bitexact.llama import Cache
    cache = Cache(2, 2, 8, dev, 2, 64)
    k = torch.randint(-1000, 1000, (2, 3, 2, 64), device=dev)
    v = torch.randint(-1000, 1000, (2, 3, 2, 64), device=dev)
    pos = torch.tensor([[0, 1, 2], [5, 6, 7]], device=dev)
    cache.write(1, k, v, pos)
    assert torch.equal(cache.k[1][0, :, 0:3].permute(1, 0, 2).long(), k[0])
    assert torch.equal(cache.v[1][1, :, 5:8].permute(1, 0, 2).long(), v[1])
    assert int(cache.k[0].abs().sum()) == 0
    c, _ = consts
    outs = [Lin(c, "lm", dev, gemm).y(torch.ones(2, 256, dtype=torch.int32, device=dev),
                                     torch.full((2,), -20, dtype=torch.long, device=dev))[0]
            for gemm in ("hip", "triton", "cublas")]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    with pytest.raises(AssertionError):
        Lin(c, "lm", "cpu")
