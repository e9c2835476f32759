"""ctypes binding of libhelm_cpu.so (C-ABI declared in include/helm_cpu.h).

The host-CPU library of HELM's CPU stages: the fp16 GEMV of their linears and
the streaming attention of a query on the CPU.  ``load()`` raises when the
library is missing or this CPU cannot run it; the attention path has no
other implementation to fall back to.  (``helm_amd.kernels`` keeps HELM's
own rule for its linears: an unusable library means plain ``F.linear``.)
Build the library with ``python -m helm_amd.build``.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional, Tuple

LIB_PATH = Path(__file__).resolve().parent / "libhelm_cpu.so"

HELM_CPU_OK, HELM_CPU_E_INVALID, HELM_CPU_E_UNSUPPORTED = 0, 1, 2
ISA_NAMES = {0: "none", 1: "avx2", 2: "avx512"}

_vp, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# name -> (restype, argtypes); every function of include/helm_cpu.h
SIGNATURES = {
    "helm_cpu_isa": (ctypes.c_int, []),
    "helm_cpu_last_error": (ctypes.c_char_p, []),
    "helm_cpu_fp16_gemv": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _i64, _i64, _i32]),
    "helm_cpu_fp16_gemv_batch": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64,
                                                _i32]),
    "helm_cpu_stream_attn": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                                            _f32, _f32, _vp, _i64, _i64, _i64, _i32, _i32,
                                            _i32, _i32]),
}

_lib = None
_error: Optional[str] = None


def _open() -> Tuple[Optional[ctypes.CDLL], Optional[str]]:
    global _lib, _error
    if _lib is not None or _error is not None:
        return _lib, _error
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.helm_cpu_isa() == 0:
            _error = "this CPU lacks AVX2 + F16C + FMA"
        else:
            _lib = lib
    except OSError as e:
        _error = f"{LIB_PATH}: {e} (build it with `python -m helm_amd.build`)"
    return _lib, _error


def try_load() -> Tuple[Optional[ctypes.CDLL], Optional[str]]:
    """(library, None) when it can run here, else (None, why not)."""
    return _open()


def load() -> ctypes.CDLL:
    """The library; raises RuntimeError when it is missing or cannot run."""
    lib, err = _open()
    if lib is None:
        raise RuntimeError(f"libhelm_cpu.so unavailable: {err}")
    return lib


def error_text(fn: str, rc: int) -> str:
    """`fn`'s failure with status `rc`, with the library's message."""
    msg = load().helm_cpu_last_error().decode(errors="replace")
    kind = "unsupported" if rc == HELM_CPU_E_UNSUPPORTED else "invalid argument"
    return f"{fn} ({kind}): {msg}"


def call(fn: str, *args) -> None:
    """Calls entry point `fn`; a non-zero status raises ValueError
    (invalid arguments) or NotImplementedError (unsupported)."""
    lib = load()
    rc = getattr(lib, fn)(*args)
    if rc != HELM_CPU_OK:
        msg = lib.helm_cpu_last_error().decode(errors="replace")
        if rc == HELM_CPU_E_UNSUPPORTED:
            raise NotImplementedError(f"{fn}: {msg}")
        raise ValueError(f"{fn}: {msg}")


def isa() -> str:
    lib, _ = _open()
    return ISA_NAMES[lib.helm_cpu_isa()] if lib is not None else "none"
