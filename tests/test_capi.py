"""C-ABI checks that need no GPU: the kernel library loads, exports every symbol
include/ortmi_kernels.h declares, and rejects malformed calls on the host with the
reference's error wording before anything is launched."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
from conftest import PKG_DIR, ROOT, load_package

HEADER = os.path.join(ROOT, "include", "ortmi_kernels.h")


def _declared(header: str) -> set[str]:
    text = open(header).read()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(ortmi_\w+)\s*\(", text, re.M))


@pytest.fixture(scope="module")
def lib():
    pkg = load_package()
    return pkg.load_kernels()


def test_exports_every_declared_symbol(lib):
    names = _declared(HEADER)
    assert len(names) >= 15
    for name in sorted(names):
        assert hasattr(lib, name), f"{name} declared in ortmi_kernels.h but not exported"


def test_python_signatures_cover_header():
    pkg = load_package()
    assert _declared(HEADER) == set(pkg.SIGNATURES)


def test_abi_version(lib):
    assert lib.ortmi_abi_version() == 2


def _err(lib):
    return lib.ortmi_last_error().decode()


def test_matmul_nbits_rejects_unsupported_forms(lib):
    # bits outside {4, 8} (tests/ops/test_claim_diagnostics.py: bits=2 is declined)
    assert lib.ortmi_matmul_nbits(None, None, None, None, None, 1, 8, 32, 2, 32, 10, None) == 1
    assert "4-bit and 8-bit" in _err(lib)
    assert lib.ortmi_matmul_nbits(None, None, None, None, None, 1, 8, 32, 4, 48, 10, None) == 1
    assert "block_size" in _err(lib)
    p = ctypes.c_void_p(16)
    assert lib.ortmi_matmul_nbits(p, p, p, None, p, 1, 8, 32, 4, 32, 7, None) == 1
    assert "float" in _err(lib)
    # Empty output is a no-op success.
    assert lib.ortmi_matmul_nbits(None, None, None, None, None, 0, 8, 32, 4, 32, 10, None) == 0


def test_gqa_rejects_bad_heads(lib):
    rc = lib.ortmi_group_query_attention(None, None, None, None, None, 0, 1, None, None, 0, 0,
                                         None, None, None, 1, 1, 6, 4, 128, 0.0, 0, 10, None, 0,
                                         None)
    assert rc == 1 and "multiple of kv_num_heads" in _err(lib)


def test_paged_rejects_latent_mismatch(lib):
    p = ctypes.c_void_p(256)
    rc = lib.ortmi_paged_attention(p, p, None, p, p, 4, 16, p, p, p, 1, 4, 1, 64, None, None, 0,
                                   0, 0, 0, None, None, None, None, 1e-6, p, 4, 2, 128, 0, 0.0,
                                   10, p, 1 << 20, None)
    assert rc == 1 and "LATENT" in _err(lib)


def test_workspace_sizes_are_monotone(lib):
    a = lib.ortmi_group_query_attention_workspace_size(8, 1, 32, 128, 4097)
    b = lib.ortmi_group_query_attention_workspace_size(8, 1, 32, 128, 8193)
    assert 0 < a < b
    c = lib.ortmi_paged_attention_workspace_size(1052, 32, 32, 8, 128, 128, 8192)
    assert c > 0


def test_package_layout():
    assert os.path.isdir(os.path.join(PKG_DIR, "csrc"))
