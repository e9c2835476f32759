"""libhelm_amd.so loads and exports exactly the C-ABI of include/helm_amd.h.

No compute calls here (CPU-only environment): only symbol presence and the
pure host-side entry points (ABI version, workspace sizing, argument checks
that return before touching a device).
"""
import ctypes
import os
import re

import numpy as np
import pytest

from helm_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "helm_amd.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(helm_[a-z_0-9]+)\s*\(", src)))


def test_library_built():
    assert _native.LIB_PATH.exists(), "run python -m helm_amd.build"


def test_every_declared_symbol_exported_and_bound():
    lib = _native.load()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(declared)


def test_abi_version():
    assert _native.load().helm_abi_version() == _native.ABI_VERSION == 2


def test_struct_layouts_match_header():
    assert _native.PAGE_DTYPE.itemsize == 32
    assert _native.APPEND_DTYPE.itemsize == 64
    assert _native.BANDWIDTH_DTYPE.itemsize == 32


def test_workspace_sizing_host_only():
    lib = _native.load()
    # Qwen3-8B shape, 2048 pages of 16 tokens
    n = lib.helm_query_workspace_bytes(1, 32, 8, 1, 128, 2048, 16, 0)
    assert n > 0
    # grows with the context and stays a small fraction of the KV bytes it
    # serves (2 * 8 heads * 16 tokens * 128 dims * 2 B per page); invalid
    # shapes give 0
    sizes = [lib.helm_query_workspace_bytes(1, 32, 8, 1, 128, p, 16, 0)
             for p in (256, 1024, 2048, 8192, 65536)]
    assert sizes == sorted(sizes) and sizes[2] == n
    for pages, ws in zip((256, 1024, 2048, 8192, 65536), sizes):
        assert ws <= 0.05 * pages * 65536 + (1 << 20)
    assert lib.helm_query_workspace_bytes(1, 30, 8, 1, 128, 2048, 16, 0) == 0


def test_argument_errors_raise_before_device_work():
    lib = _native.load()
    # append with zero segments is a no-op
    assert lib.helm_page_append(None, 0, 8, 128, _native.HELM_BF16, None) == 0
    # unknown dtype is rejected with a message
    rc = lib.helm_page_append(None, 1, 8, 128, 7, None)
    assert rc == _native.HELM_E_INVALID
    assert b"dtype" in lib.helm_last_error_string()
    with pytest.raises(ValueError):
        _native.check("helm_page_append", rc)
    # null pointers in the pool entry point are rejected
    rc = lib.helm_paged_decode_attn(None, None, None, None, 0, 0, None, 0, None, 1, 32, 8, 1,
                                    128, 16, 1, 0, None, 1.0, 0.0, None, 0, 0, 0, 2, 1, 1, 0, None, 0,
                                    None)
    assert rc == _native.HELM_E_INVALID


def test_no_cpu_fallback_symbols():
    # the library has no host compute path: nothing but the declared ABI
    lib_syms = os.popen(f"nm -D --defined-only {_native.LIB_PATH}").read()
    exported = set(re.findall(r" T (helm_[a-z_0-9]+)", lib_syms))
    assert exported == set(_declared_functions())
