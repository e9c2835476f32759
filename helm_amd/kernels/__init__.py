"""helm_amd.kernels — the fp16 linear of HELM's CPU stages (helm/kernels/__init__.py).

Same surface as HELM's module: ``fp16_linear(input, weight, bias=None)``,
``patch_cpu_linears(module)``, ``is_available()``, ``load_error()``.  A decode
step's GEMV (1 to 8 tokens) runs in libhelm_cpu.so (helm_amd/cpu/gemv.cpp:
AVX-512 or AVX2 + F16C, fp32 accumulation, bias in fp32, one rounding to
fp16, the weight read once); other token counts take HELM's float32 GEMM
branch, ``F.linear`` in fp32 then fp16 (helm/kernels/__init__.py:78-82).  As
in HELM, when the native library cannot be used (not built, or a CPU without
AVX2 + F16C + FMA) ``is_available()`` is False and every call takes
``F.linear`` — HELM's own rule for its CPU-stage linears (:86-88, :141-154).
``HELM_DISABLE_AVX`` turns the native GEMV off, as in HELM (:77).

``patch_cpu_linears`` binds a native forward onto each fp16 CPU ``nn.Linear``
instance in place: the modules keep their class, parameters, state-dict keys
and position in the tree; the bound forward decides per call whether the
native GEMV applies (fp16 weight and input on the CPU) or ``F.linear`` does.
"""
from __future__ import annotations

import logging
import os
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from helm_amd import _cpu_native

logger = logging.getLogger(__name__)

LIB_PATH = _cpu_native.LIB_PATH
ISA_NAMES = _cpu_native.ISA_NAMES
MAX_BATCH = 8      # vectors per native call (HELM_CPU_GEMV_MAX_BATCH)

_warned = False


def is_available() -> bool:
    """True when the native GEMV can run here (helm/kernels/__init__.py:92-95)."""
    return _cpu_native.try_load()[0] is not None


def load_error() -> Optional[str]:
    """Why the native GEMV cannot run, or None (helm/kernels/__init__.py:98-101)."""
    return _cpu_native.try_load()[1]


def isa() -> str:
    """The instruction-set path the native GEMV takes on this CPU."""
    return _cpu_native.isa()


_F16 = torch.float16
_entry = None    # helm_cpu_fp16_gemv_batch, bound once the library has loaded


def _gemv_entry():
    global _entry
    if _entry is None:
        lib, why = _cpu_native.try_load()
        if lib is None:
            raise RuntimeError(f"native fp16 GEMV unavailable: {why}")
        _entry = lib.helm_cpu_fp16_gemv_batch
    return _entry


def _gemv_into(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor],
               M: int, N: int, K: int, threads: int) -> None:
    """One native call: y [M, N] = fp16(w x + bias) for contiguous x [M, K], w [N, K]."""
    code, ptr, b = 0, None, None
    if bias is not None:
        if bias.numel() != N or not bias.is_cpu:
            raise ValueError(f"bias must hold {N} values on the CPU")
        b = bias.reshape(N).contiguous()
        if b.dtype is not _F16:
            b = b.float()
        code, ptr = (1 if b.dtype is _F16 else 2), b.data_ptr()
    rc = _gemv_entry()(x.data_ptr(), w.data_ptr(), ptr, code, y.data_ptr(), M, N, K, threads)
    if rc:
        raise RuntimeError(_cpu_native.error_text("helm_cpu_fp16_gemv_batch", rc))


def gemv_fp16(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
              threads: int = 0) -> torch.Tensor:
    """y = fp16(weight @ x + bias) through libhelm_cpu.so: x [K] or [M, K]
    fp16 (M <= 8 vectors, W read once), weight [N, K] fp16, bias [N] fp16 /
    fp32 or None; returns [N] (or [M, N]) fp16."""
    if weight.dim() != 2 or weight.dtype is not _F16 or not weight.is_cpu:
        raise ValueError("weight must be a 2-D fp16 CPU tensor")
    N, K = weight.shape
    if x.dtype is not _F16 or not x.is_cpu or x.numel() % K or x.numel() == 0:
        raise ValueError(f"x must hold a multiple of {K} fp16 values on the CPU")
    M = x.numel() // K
    if M > MAX_BATCH:
        raise ValueError(f"at most {MAX_BATCH} vectors per call, got {M}")
    y = torch.empty(M, N, dtype=_F16)
    _gemv_into(y, x.reshape(M, K).contiguous(), weight.contiguous(), bias, M, N, K, int(threads))
    return y if x.dim() > 1 else y.reshape(N)


def fp16_linear(input: torch.Tensor, weight: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear for fp16 weights on the CPU (helm/kernels/__init__.py:58-89).

    Tokens = the product of the input's leading dims.  1 to 8 tokens (a decode
    step) run the native GEMV, the weight read once; any other count (prefill,
    or an empty input) runs F.linear in float32 and rounds to fp16 — HELM's
    branch for every count but 1, the same float32 sums and one rounding;
    inputs that are not fp16 on the CPU take plain F.linear.  The decode
    branch is one native call and one output allocation (a layer's seven
    linears are a few hundred microseconds in all, so per-call work counts)."""
    if not (weight.dtype is _F16 and input.dtype is _F16 and weight.is_cpu and input.is_cpu
            and weight.dim() == 2):
        return F.linear(input, weight, bias)
    N, K = weight.shape
    shape = input.shape
    if shape[-1] != K:
        raise RuntimeError(f"fp16_linear: input last dim ({shape[-1]}) != weight K ({K})")
    tokens = input.numel() // K
    if 1 <= tokens <= MAX_BATCH and not os.environ.get("HELM_DISABLE_AVX") and is_available():
        y = torch.empty(*shape[:-1], N, dtype=_F16)
        _gemv_into(y, input if input.is_contiguous() else input.contiguous(),
                   weight if weight.is_contiguous() else weight.contiguous(),
                   bias, tokens, N, K, 0)
        return y
    return F.linear(input.float(), weight.float(),
                    bias.float() if bias is not None else None).half()


class NativeLinear(nn.Linear):
    """nn.Linear routed through ``fp16_linear``: the native GEMV path when the
    weight and input are fp16 on the CPU at call time, else F.linear.
    ``patch_cpu_linears`` changes a linear's class to this one in place, so
    the module keeps its parameters, buffers, hooks and state_dict keys and
    pickles (torch.save) like any module defined at module level."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return fp16_linear(x, self.weight, self.bias)


def patch_cpu_linears(module: nn.Module, verbose: bool = False) -> int:
    """Routes every fp16 CPU nn.Linear below `module` through ``fp16_linear``
    and returns how many were newly routed (helm/kernels/__init__.py:134-168).
    As HELM's walk, it visits `module`'s children recursively and never
    `module` itself, so a bare nn.Linear passed in is left as it is (0).  A
    linear already routed is left as it is.  When the native GEMV is
    unavailable nothing is changed, with one warning per process."""
    global _warned
    if not is_available():
        if not _warned:
            logger.warning("[helm_amd kernels] native fp16 GEMV unavailable; CPU layers use "
                           "plain PyTorch. Cause: %s", load_error())
            _warned = True
        elif verbose:
            logger.info("[helm_amd kernels] native GEMV unavailable (%s); nothing patched",
                        load_error())
        return 0
    routed = 0
    for child in module.children():
        if isinstance(child, NativeLinear):
            continue
        if isinstance(child, nn.Linear):
            if child.weight.dtype == torch.float16 and child.weight.device.type == "cpu":
                child.__class__ = NativeLinear
                routed += 1
        else:
            routed += patch_cpu_linears(child, verbose=verbose)
    return routed
