"""The C ABI library loads and exports every entry point include/*.h declares (no GPU call is made), and the
product package never reaches the oracle."""

import ctypes
import glob
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "bitexact-llm_amd", "bitexact", "_lib", "libbitexact_hip.so")


def declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(bx_[a-z0-9_]+)\s*\(", src))
    return names


def test_exports_every_declared_symbol():
    names = declared()
    assert {"bx_exact_linear", "bx_int8_gemm", "bx_int8_gemm_join"} <= names
    lib = ctypes.CDLL(LIB)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.bx_version() >= 1


def test_python_signatures_cover_header():
    from bitexact import _hip
    assert declared() <= set(_hip.SIGNATURES), declared() - set(_hip.SIGNATURES)


def test_product_never_imports_oracle():
    for f in glob.glob(os.path.join(ROOT, "bitexact-llm_amd", "**", "*.py"), recursive=True):
        src = open(f).read()
        assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", src, flags=re.M), f


def test_host_tables_match_oracle():
    """The product's RoPE tables, 2^-f table and embedding rounding are the oracle's (host float64 constants)."""
    import torch
    from bitexact.exact import consts
    from oracle import bxref as R
    inv = consts.llama3_inv_freq(64)
    assert np.array_equal(inv.numpy(), R.llama3_inv_freq(64))
    c, s = consts.rope_tables(4096, 30, inv)
    rc, rs = R.rope_tables(4096, 30, R.llama3_inv_freq(64))
    assert np.array_equal(c.numpy(), rc) and np.array_equal(s.numpy(), rs)
    assert np.array_equal(consts.exp2_table().numpy(), R.exp2_table())
    w = (torch.randn(64, 300, generator=torch.Generator().manual_seed(1)) * 0.02).to(torch.bfloat16)
    w[0, :4] = torch.tensor([0.0, -0.0, 1e-30, -3e-8])
    m = R.engine_constants(w.view(torch.int16).numpy(), {}, {}, c, s, 0)
    assert np.array_equal(consts.emb_fixed(w).numpy(), m["emb"])


def test_constants_digest_and_file_roundtrip(tmp_path):
    """sha256 equals the reference's llama.digest on the golden dict; save / load round-trips every entry and the
    digest; this build's derived keys do not change the identity."""
    import torch
    from bitexact.exact import consts
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))
    c = {"n_layers": 2, "cfg": {"hidden_size": 64}, "stats": {"x": 1}}
    for k in gold.files:
        if k.startswith("dg_") and k != "dg_sha":
            c[k[3:]] = torch.from_numpy(gold[k])
    assert bytes.fromhex(consts.sha256(c)) == gold["dg_sha"].tobytes()
    c2 = dict(c)
    c2["0.wo.ell_cnt"] = torch.zeros(4, dtype=torch.int32)
    c2["0.wo.R"] = 0
    assert consts.sha256(c2) == consts.sha256(c)
    f = str(tmp_path / "c.safetensors")
    consts.save(c, f)
    d = consts.load(f)
    assert set(d) == set(c) and d["n_layers"] == 2 and d["cfg"] == {"hidden_size": 64}
    assert all(torch.equal(d[k], c[k]) for k in c if torch.is_tensor(c[k]))
    assert consts.sha256(d) == consts.sha256(c)


def test_validate_ell_rejects_corrupt_lists():
    """The load-time ELL check: valid lists pass; a count outside [0, R] or a listed column outside [0, K) raises
    AssertionError (unused padding slots are not checked)."""
    import pytest
    import torch
    from bitexact.exact.model import validate_ell
    cnt = torch.tensor([0, 2, 1], dtype=torch.int32)
    ec = torch.tensor([[0, 0], [3, 63], [5, 999]], dtype=torch.int32)   # row 2's second slot is padding
    validate_ell(cnt, ec, 2, 64)
    for c2, e2 in ((torch.tensor([0, 3, 1], dtype=torch.int32), ec),
                   (torch.tensor([-1, 2, 1], dtype=torch.int32), ec),
                   (cnt, torch.tensor([[0, 0], [3, 64], [5, 0]], dtype=torch.int32)),
                   (cnt, torch.tensor([[0, 0], [-2, 1], [5, 0]], dtype=torch.int32))):
        with pytest.raises(AssertionError):
            validate_ell(c2, e2, 2, 64)


def test_torch_ops_registered_with_meta_shapes():
    """Every kernel entry is a torch.ops.bitexact_hip operator whose fake / meta kernel gives the output shapes
    and dtypes (what torch.compile traces with); no device is touched."""
    import torch
    import bitexact.bmm  # noqa: F401
    import bitexact.exact.attention  # noqa: F401
    import bitexact.exact.ops  # noqa: F401
    import bitexact.exact.wmm  # noqa: F401
    import bitexact.int8.gemm_skinny  # noqa: F401
    import bitexact.int8.segs  # noqa: F401
    import bitexact.intops  # noqa: F401
    import bitexact.vllm_plugin.exact_gemm  # noqa: F401
    import bitexact.vllm_plugin.tri_exact_attn  # noqa: F401
    import bitexact.vllm_plugin.tri_paged  # noqa: F401
    ops = torch.ops.bitexact_hip
    m = lambda *s, dt=torch.int64: torch.empty(*s, dtype=dt, device="meta")
    i32, i8 = torch.int32, torch.int8
    fl = m(1, dt=i32)
    y = ops.exact_linear(m(8, 64, dt=i32), m(8), m(3, 32, 64, dt=i8), m(32), m(32), None, None, None, 0, fl, True,
                         24, None)
    assert y.shape == (8, 32) and y.dtype == torch.int64
    assert ops.wmm(m(8, 64, dt=i32), m(3, 32, 64, dt=i8)).shape == (1, 8, 32)
    yy, f = ops.epilogue(m(2, 8, 32), None, m(8, 64, dt=i32), m(32, 2, dt=i32), m(32, 2), m(32), m(32), m(8), 24, True)
    assert yy.shape == (8, 32) and f.shape == (1,)
    assert ops.int_mm(m(16, 64, dt=i8), m(32, 64, dt=i8)).dtype == i32
    assert ops.int_mm_join(m(16, 64, dt=i8), m(32, 64, dt=i8), 8, 2).shape == (8, 32)
    assert ops.bmm(m(4, 3, 64, dt=i32), m(4, 64, 5, dt=i32), 3, 3).shape == (4, 3, 5)
    q, sh = ops.norm_quant(m(5, 256), m(256), m(256), fl)
    assert q.dtype == i32 and sh.shape == (5,)
    p, den = ops.softmax(m(2, 3, 40), m(2, 3, 1), m(2, 3, 1), m(16385), 387270501, 17, 22)
    assert p.shape == (2, 3, 40) and p.dtype == i32 and den.shape == (2, 3, 1)
    qo, so = ops.attn_out(m(4, 12, 64), m(4, 12, 1), 3, 2)
    assert qo.shape == (6, 512) and so.shape == (6,)
    qg, shg, k, v = ops.qkv_y(m(6, 3072), m(2, 3), m(4096, 32), m(4096, 32), 2, 3, 32, 8, 64, fl)
    assert qg.shape == (16, 12, 64) and k.shape == (2, 3, 8, 64)
    qg2, _ = ops.qkv_y_store(m(6, 3072), m(2, 3), m(4096, 32), m(4096, 32), 2, 3, 32, 8, 64, fl,
                             m(9, 8, 16, 512, dt=i8), m(6))
    assert qg2.shape == qg.shape
    q, pl, sh = ops.add_norm(m(5, 64), m(5, 64), m(64), m(64), fl, True)
    assert pl.shape == (3, 5, 64)
    x, q, sh = ops.embed_norm(m(300, 64, dt=i32), m(7), m(64), m(64), fl)
    assert x.shape == (7, 64) and q.dtype == i32
    q, pl, sh = ops.gu_silu(m(5, 128), m(16385), fl, True, False)
    assert q.shape == (5, 64) and pl.numel() == 0
    assert ops.first_argmax(m(3, 100), False).shape == (3,)
    num, den = ops.attend_exact(m(2, 8, 4, 64, dt=i32), m(2, 8, 4), m(2, 4), m(9, 8, 16, 512, dt=i8),
                                m(2, 4, dt=i32), m(2), m(16385), 387270501, 1)
    assert num.shape == (2, 8, 4, 64) and den.shape == (2, 8, 4, 1)
    num, den = ops.attend_int8(m(2, 8, 4, 64), m(2, 4), m(9, 8, 16, 512, dt=i8), m(2, 4, dt=i32), m(4097, dt=i32), 1)
    assert num.shape == (2, 8, 4, 64)
    num, den = ops.attn_prefill(m(4, 12, 64, dt=i32), m(4, 12, 1), m(4, 3, 64, dt=i32), m(4, 3, 64, dt=i32),
                                m(4, 12, 1), m(16385), 387270501, True)
    assert num.shape == (4, 12, 64)
    a, as_, sh, mant, e = ops.int8_quant_rows(m(5, 64), 2, True)
    assert a.shape == (10, 64) and mant.shape == (5,)
    yp, f = ops.int8_post(m(5, 32), m(32), 3, m(5), m(5))
    assert yp.shape == (5, 32)


def test_no_cpu_path():
    """The product has no CPU fallback: device-less layers and the float64 product raise."""
    import pytest
    import torch
    from bitexact.exact.wmm import wmm_cpu
    from bitexact.llama import Cache
    with pytest.raises(AssertionError):
        wmm_cpu(torch.zeros(1, 16, dtype=torch.int32), None)
    with pytest.raises(AssertionError):
        Cache(1, 1, 4, "cpu")
