"""The C ABI library loads and exports every entry point include/*.h declares (no GPU call is made), and the
product package never reaches the oracle."""

import ctypes
import glob
import os
import re

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
