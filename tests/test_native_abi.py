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


def test_decode_step_argument_block_layout():
    """The fast decode path packs helm_decode_args with precompiled structs;
    every field lands where the struct (and the numpy record type that
    mirrors it) has it."""
    from helm_amd.runtime import kv_cache as KC
    arr, buf, addr = KC._decode_args()
    assert addr == arr.ctypes.data and buf.nbytes == 744
    KC._DA_HEAD.pack_into(buf, 0, 11, 12, 13, 14, 15, -16, 17)
    KC._DA_TAIL.pack_into(buf, KC._DA_TAIL_OFF, 3, 32, 8, 128, 16, 1, 2, 3, 1, 0, 0.25, 30.0)
    for b in range(3):
        KC._DA_U64.pack_into(buf, KC._DA_PAGES + 8 * b, 100 + b)
        KC._DA_U64.pack_into(buf, KC._DA_TOKK + 8 * b, 200 + b)
        KC._DA_U64.pack_into(buf, KC._DA_TOKV + 8 * b, 300 + b)
        KC._DA_I64.pack_into(buf, KC._DA_TOKHS + 8 * b, 400 + b)
        KC._DA_I32.pack_into(buf, KC._DA_NPAGES + 4 * b, 500 + b)
        KC._DA_I32.pack_into(buf, KC._DA_TOKENS + 4 * b, 600 + b)
    r = arr[0]
    assert [int(r[f]) for f in ("q", "out", "mask", "stream", "mask_bstride", "mask_hstride",
                                "mask_qstride")] == [11, 12, 13, 14, 15, -16, 17]
    assert [int(r[f]) for f in ("B", "Hq", "Hkv", "D", "page_tokens", "aligned16", "mask_dtype",
                                "kv_dtype", "append", "pad")] == [3, 32, 8, 128, 16, 1, 2, 3, 1, 0]
    assert float(r["scale"]) == 0.25 and float(r["softcap"]) == 30.0
    for f, base in (("seq_pages", 100), ("tok_k", 200), ("tok_v", 300),
                    ("tok_head_stride", 400), ("seq_npages", 500), ("seq_tokens", 600)):
        assert list(r[f][:3]) == [base, base + 1, base + 2]


def test_fast_env_lookup_follows_environ(monkeypatch):
    from helm_amd.runtime import kv_cache as KC
    name = "HELM_AMD_TEST_SWITCH"
    monkeypatch.delenv(name, raising=False)
    assert KC._env_get(name) is None
    monkeypatch.setenv(name, "0")
    assert KC._env_get(name) == "0"
    monkeypatch.setenv(name, "1")
    assert KC._env_get(name) == "1"
    monkeypatch.delenv(name)
    assert KC._env_get(name) is None
    monkeypatch.setenv("HELM_AMD_CHECK_RECORDS", "1")
    assert KC.check_records_enabled()
    monkeypatch.setenv("HELM_AMD_CHECK_RECORDS", "0")
    assert not KC.check_records_enabled()
