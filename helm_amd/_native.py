"""ctypes binding of libhelm_amd.so (C-ABI declared in include/helm_amd.h).

Loading fails loudly: there is no Python or CPU fallback for any entry point.
Build the library with ``python -m helm_amd.build`` first.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(os.environ.get("HELM_AMD_LIB", Path(__file__).resolve().parent / "libhelm_amd.so"))

HELM_F16, HELM_BF16, HELM_F32 = 0, 1, 2
HELM_OK = 0
HELM_E_INVALID, HELM_E_UNSUPPORTED, HELM_E_WORKSPACE = -1, -2, -3
HELM_PAGE_HOST = 1
HELM_STATIC_SCRATCH_BYTES = 16 << 20

# struct helm_page (32 bytes)
PAGE_DTYPE = np.dtype([
    ("k", "<u8"), ("v", "<u8"), ("used", "<i4"), ("tok_off", "<i4"),
    ("head_stride", "<i4"), ("flags", "<i4"),
])
assert PAGE_DTYPE.itemsize == 32

# struct helm_append_seg (64 bytes)
APPEND_DTYPE = np.dtype([
    ("dst_k", "<u8"), ("dst_v", "<u8"), ("src_k", "<u8"), ("src_v", "<u8"),
    ("src_head_stride", "<i8"), ("src_tok_stride", "<i8"),
    ("dst_head_stride", "<i4"), ("dst_tok", "<i4"), ("n_tok", "<i4"), ("pad", "<i4"),
])
assert APPEND_DTYPE.itemsize == 64

# struct helm_bandwidth (32 bytes)
BANDWIDTH_DTYPE = np.dtype([
    ("device_copy_bytes_per_s", "<f8"), ("h2d_bytes_per_s", "<f8"), ("d2h_bytes_per_s", "<f8"),
    ("copy_mismatched_words", "<i8"),
])
assert BANDWIDTH_DTYPE.itemsize == 32

# helm_decode_args (include/helm_amd.h); 744 bytes, no padding
DECODE_MAX_SEQS = 16
DECODE_ARGS_DTYPE = np.dtype([
    ("q", "<u8"), ("out", "<u8"), ("mask", "<u8"), ("stream", "<u8"),
    ("mask_bstride", "<i8"), ("mask_hstride", "<i8"), ("mask_qstride", "<i8"),
    ("seq_pages", "<u8", (DECODE_MAX_SEQS,)), ("tok_k", "<u8", (DECODE_MAX_SEQS,)),
    ("tok_v", "<u8", (DECODE_MAX_SEQS,)), ("tok_head_stride", "<i8", (DECODE_MAX_SEQS,)),
    ("seq_npages", "<i4", (DECODE_MAX_SEQS,)), ("seq_tokens", "<i4", (DECODE_MAX_SEQS,)),
    ("B", "<i4"), ("Hq", "<i4"), ("Hkv", "<i4"), ("D", "<i4"),
    ("page_tokens", "<i4"), ("aligned16", "<i4"), ("mask_dtype", "<i4"), ("kv_dtype", "<i4"),
    ("append", "<i4"), ("pad", "<i4"), ("scale", "<f4"), ("softcap", "<f4"),
])
assert DECODE_ARGS_DTYPE.itemsize == 744

_c_void_p = ctypes.c_void_p
_i32, _i64, _u64, _f32, _sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); must list every function of include/helm_amd.h
SIGNATURES = {
    "helm_last_error_string": (ctypes.c_char_p, []),
    "helm_abi_version": (ctypes.c_int, []),
    "helm_engine_create": (ctypes.c_int, [ctypes.c_int, _sz, ctypes.c_int, ctypes.POINTER(_c_void_p)]),
    "helm_engine_destroy": (ctypes.c_int, [_c_void_p]),
    "helm_engine_copy_stream": (_c_void_p, [_c_void_p]),
    "helm_query_workspace_bytes": (_sz, [ctypes.c_int] * 8),
    "helm_paged_decode_attn": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, ctypes.c_int,
        _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p, _f32, _f32, _c_void_p, _i64, _i64,
        _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p, _sz, _c_void_p]),
    "helm_paged_decode_attn_static": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, ctypes.c_int,
        _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p, _f32, _f32, _c_void_p, _i64, _i64,
        _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p]),
    "helm_stream_attn": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, _c_void_p, _c_void_p, _f32, _f32, _c_void_p, _i64, _i64,
        _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p]),
    "helm_paged_attn_seqs": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, _c_void_p, _c_void_p, _c_void_p, ctypes.c_int,
        ctypes.c_int, _f32, _f32, _c_void_p, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, _c_void_p]),
    "helm_paged_attn_seqs_append": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, _c_void_p, _c_void_p, _c_void_p, ctypes.c_int, ctypes.c_int, _f32, _f32, _c_void_p,
        _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _c_void_p, _c_void_p]),
    "helm_decode_step": (ctypes.c_int, [_c_void_p, _c_void_p]),
    "helm_upload": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _sz, _c_void_p]),
    "helm_host_pages_in_place": (ctypes.c_int, [_c_void_p, _c_void_p, ctypes.c_int,
                                                ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                _c_void_p]),
    "helm_page_append": (ctypes.c_int, [_c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, _c_void_p]),
    "helm_decode_front": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, ctypes.c_int, _f32,
        _c_void_p, _c_void_p, _i64, ctypes.c_int, _c_void_p, _c_void_p, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p]),
    "helm_profile_split_kernels": (ctypes.c_int, [ctypes.c_int]),
    "helm_profile_split_read": (ctypes.c_int, [_c_void_p, ctypes.c_int]),
    "helm_profile_workgroup_stamps": (ctypes.c_int, [_c_void_p, ctypes.c_int]),
    "helm_profile_read_pass": (ctypes.c_int, [_c_void_p, ctypes.c_int, _u64, ctypes.c_int, _u64,
                                              ctypes.c_int, ctypes.c_int, _c_void_p,
                                              _c_void_p]),
    "helm_measure_bandwidth": (ctypes.c_int, [ctypes.c_int, _u64, _u64, ctypes.c_int,
                                              _c_void_p]),
    "helm_evict_pages": (ctypes.c_int, [_c_void_p, ctypes.c_int, _c_void_p, _c_void_p,
                                        _c_void_p, ctypes.c_int, _c_void_p]),
    "helm_prefetch_pages": (ctypes.c_int, [_c_void_p, ctypes.c_int, _c_void_p, _c_void_p,
                                           _c_void_p, ctypes.c_int, _c_void_p]),
}

_lib = None
ABI_VERSION = 2   # HELM_AMD_ABI_VERSION of include/helm_amd.h


class HelmNativeError(RuntimeError):
    """A libhelm_amd.so entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (status {code}): {msg}")
        self.code = code


def load() -> ctypes.CDLL:
    """Loads libhelm_amd.so once; raises if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} not found: the HIP library is required (no fallback). "
            "Build it with `python -m helm_amd.build`.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.helm_abi_version() != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {lib.helm_abi_version()} != {ABI_VERSION}"
                          " (rebuild with `python -m helm_amd.build`)")
    _lib = lib
    return lib


def check(fn: str, rc: int) -> None:
    if rc != HELM_OK:
        msg = load().helm_last_error_string().decode(errors="replace")
        if rc in (HELM_E_INVALID, HELM_E_WORKSPACE):
            raise ValueError(f"{fn}: {msg}")
        if rc == HELM_E_UNSUPPORTED:
            raise NotImplementedError(f"{fn}: {msg}")
        raise HelmNativeError(fn, rc, msg)


def call(fn: str, *args) -> None:
    check(fn, getattr(load(), fn)(*args))


_entries = {}


def entry(fn: str):
    """Entry point `fn` of the loaded library, bound once (for the per-call
    paths: the caller checks the status with ``check``)."""
    f = _entries.get(fn)
    if f is None:
        f = _entries[fn] = getattr(load(), fn)
    return f


def ptr(a: np.ndarray) -> int:
    """Address of a C-contiguous numpy array's data."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def dtype_code(torch_dtype) -> int:
    import torch
    if torch_dtype == torch.float16:
        return HELM_F16
    if torch_dtype == torch.bfloat16:
        return HELM_BF16
    if torch_dtype == torch.float32:
        return HELM_F32
    raise TypeError(f"unsupported KV/query dtype {torch_dtype}")
