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
