"""helm_amd.kernels — the fp16 linear of HELM's CPU stages (helm/kernels/__init__.py).

Same surface as HELM's module: ``fp16_linear(input, weight, bias=None)``,
``patch_cpu_linears(module)``, ``is_available()``, ``load_error()``.  A decode
step's GEMV (up to 8 tokens) runs in libhelm_cpu.so (helm_amd/cpu/gemv.cpp:
AVX-512 or AVX2 + F16C, fp32 accumulation, bias in fp32, one rounding to
fp16, the weight read once); more tokens take HELM's float32 GEMM branch,
``F.linear`` in fp32 then fp16 (helm/kernels/__init__.py:78-82).  As in HELM,
when the native library cannot be used (not built, or a CPU without AVX2 +
F16C + FMA) ``is_available()`` is False and every call takes ``F.linear`` —
this is HELM's own behaviour for its CPU stages (:86-88, :141-154), not a path
of the GPU attention, which has no CPU fallback.  ``HELM_DISABLE_AVX`` turns
the native GEMV off, as in HELM (:77).
"""
from __future__ import annotations

import ctypes
import logging
import os
from pathlib import Path
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

logger = logging.getLogger(__name__)

LIB_PATH = Path(__file__).resolve().parent.parent / "libhelm_cpu.so"
ISA_NAMES = {0: "none", 1: "avx2", 2: "avx512"}

_lib = None
_load_error: Optional[str] = None
_warned_unavailable = False


def _load():
    """Loads libhelm_cpu.so once (helm/kernels/__init__.py:35-51 builds HELM's)."""
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.helm_cpu_isa.restype = ctypes.c_int
        lib.helm_cpu_isa.argtypes = []
        lib.helm_cpu_last_error.restype = ctypes.c_char_p
        lib.helm_cpu_last_error.argtypes = []
        lib.helm_cpu_fp16_gemv.restype = ctypes.c_int
        lib.helm_cpu_fp16_gemv.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                           ctypes.c_int64, ctypes.c_int]
        lib.helm_cpu_fp16_gemv_batch.restype = ctypes.c_int
        lib.helm_cpu_fp16_gemv_batch.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                                 ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                                 ctypes.c_int]
        if lib.helm_cpu_isa() == 0:
            _load_error = "this CPU lacks AVX2 + F16C + FMA"
            return
        _lib = lib
    except OSError as e:
        _load_error = f"{LIB_PATH}: {e}"


def is_available() -> bool:
    """True when the native GEMV can run here (helm/kernels/__init__.py:92-95)."""
    _load()
    return _lib is not None


def load_error() -> Optional[str]:
    """Why the native GEMV cannot run, or None (helm/kernels/__init__.py:98-101)."""
    _load()
    return _load_error


def isa() -> str:
    """The instruction-set path the native GEMV takes on this CPU."""
    _load()
    return ISA_NAMES[_lib.helm_cpu_isa()] if _lib is not None else "none"


MAX_BATCH = 8      # vectors per native call (HELM_CPU_GEMV_MAX_BATCH)


def gemv_fp16(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
              threads: int = 0) -> torch.Tensor:
    """y = fp16(weight @ x + bias) through libhelm_cpu.so: x [K] or [M, K]
    fp16 (M <= 8 vectors, W read once), weight [N, K] fp16, bias [N] fp16 /
    fp32 or None; returns [N] (or [M, N]) fp16."""
    _load()
    if _lib is None:
        raise RuntimeError(f"native fp16 GEMV unavailable: {_load_error}")
    if weight.dim() != 2 or weight.dtype != torch.float16 or weight.device.type != "cpu":
        raise ValueError("weight must be a 2-D fp16 CPU tensor")
    N, K = weight.shape
    if x.dtype != torch.float16 or x.device.type != "cpu" or x.numel() % K or x.numel() == 0:
        raise ValueError(f"x must hold a multiple of {K} fp16 values on the CPU")
    M = x.numel() // K
    if M > MAX_BATCH:
        raise ValueError(f"at most {MAX_BATCH} vectors per call, got {M}")
    w = weight.contiguous()
    xv = x.reshape(M, K).contiguous()
    bdt, bptr, b = 0, None, None
    if bias is not None:
        if bias.numel() != N or bias.device.type != "cpu":
            raise ValueError(f"bias must hold {N} values on the CPU")
        b = bias.reshape(N).contiguous()
        if b.dtype == torch.float16:
            bdt = 1
        else:
            b, bdt = b.float(), 2
        bptr = b.data_ptr()
    y = torch.empty(M, N, dtype=torch.float16)
    rc = _lib.helm_cpu_fp16_gemv_batch(xv.data_ptr(), w.data_ptr(), bptr, bdt, y.data_ptr(), M,
                                       N, K, int(threads))
    if rc != 0:
        raise RuntimeError(f"helm_cpu_fp16_gemv_batch: {_lib.helm_cpu_last_error().decode()}")
    return y if x.dim() > 1 else y.reshape(N)


def fp16_linear(input: torch.Tensor, weight: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear for fp16 weights on the CPU (helm/kernels/__init__.py:58-89):
    a decode step (up to 8 tokens: all leading dims multiply to <= 8) runs the
    native GEMV, W read once; more tokens run F.linear in float32 and cast to
    fp16 (HELM's branch for every count above 1: the same float32 sums and
    one rounding, with W widened to float32 each call); anything else
    (non-fp16, not on the CPU) is plain F.linear."""
    _load()
    if (weight.dtype == torch.float16 and weight.device.type == "cpu"
            and input.dtype == torch.float16):
        b = 1
        for s in input.shape[:-1]:
            b *= s
        if b <= MAX_BATCH and _lib is not None and not os.environ.get("HELM_DISABLE_AVX"):
            if input.shape[-1] != weight.shape[1]:
                raise RuntimeError(f"fp16_linear: input last dim ({input.shape[-1]}) != "
                                   f"weight K ({weight.shape[1]})")
            y = gemv_fp16(input.reshape(b, -1), weight, bias)
            return y.reshape(*input.shape[:-1], weight.shape[0])
        bias_f32 = bias.float() if bias is not None else None
        return F.linear(input.float(), weight.float(), bias_f32).half()
    return F.linear(input, weight, bias)


class _AVXLinear(nn.Module):
    """nn.Linear wrapper that routes fp16 CPU forwards through fp16_linear
    (helm/kernels/__init__.py:108-131); shares the original parameters."""

    def __init__(self, linear: nn.Linear):
        super().__init__()
        self.weight = linear.weight
        self.bias = linear.bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if (self.weight.dtype == torch.float16 and self.weight.device.type == "cpu"
                and x.dtype == torch.float16):
            return fp16_linear(x, self.weight, self.bias)
        return F.linear(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.weight.shape[1]}, out_features={self.weight.shape[0]}, "
                f"bias={self.bias is not None}, avx=True")


def patch_cpu_linears(module: nn.Module, verbose: bool = False) -> int:
    """Replaces every nn.Linear with fp16 CPU weights under `module` by
    _AVXLinear; returns how many (helm/kernels/__init__.py:134-168).  Nothing
    is patched, with one warning per process, when the native GEMV is
    unavailable."""
    global _warned_unavailable
    _load()
    if _lib is None:
        if not _warned_unavailable:
            logger.warning("[helm_amd kernels] native fp16 GEMV unavailable; CPU layers use "
                           "plain PyTorch. Cause: %s", _load_error)
            _warned_unavailable = True
        elif verbose:
            logger.info("[helm_amd kernels] native GEMV unavailable (%s); skipping patch",
                        _load_error)
        return 0
    count = 0
    for name, child in list(module.named_children()):
        if isinstance(child, nn.Linear):
            if child.weight.dtype == torch.float16 and child.weight.device.type == "cpu":
                setattr(module, name, _AVXLinear(child))
                count += 1
        else:
            count += patch_cpu_linears(child, verbose=verbose)
    return count
