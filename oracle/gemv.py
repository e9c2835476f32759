"""CPU oracle for HELM's fp16 GEMV (helm/kernels/fp16_gemv.cpp) — TEST
INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module, and only
as the reference results are compared with.  It states what helm_fp16_linear computes on its decode fast
path, in float64 numpy, without the kernel's structure:

    y = fp16( sum_j W[i, j] * x[j]  +  bias[i] )      (fp16_gemv.cpp:101-108, :137-151)

The kernel accumulates in float32 (F16C widening, FMA) in an order of its own,
so its result is within the float32 accumulation bound of this sum before the
one rounding to fp16: ``error_bound`` gives that bound.
"""
from __future__ import annotations

from typing import Optional

import numpy as np


def gemv_fp64(x, W, bias=None) -> np.ndarray:
    """The exact-in-float64 sum W @ x (+ bias), before any rounding to fp16.
    x [K], W [N, K], bias [N] or None (any float dtype)."""
    W64 = np.asarray(W, dtype=np.float64)
    y = W64 @ np.asarray(x, dtype=np.float64).reshape(-1)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(-1)
    return y


def error_bound(x, W, bias=None) -> np.ndarray:
    """Per-row bound on |kernel - fp16(exact)| in float64: one fp16 ulp of the
    exact value (the final rounding may land on either neighbour once the
    float32 sum is off by a little) plus the float32 accumulation bound
    gamma_{K+1} * (sum_j |W x| + |bias|), gamma_n = n u / (1 - n u), u = 2^-24."""
    W64 = np.abs(np.asarray(W, dtype=np.float64))
    s = W64 @ np.abs(np.asarray(x, dtype=np.float64).reshape(-1))
    if bias is not None:
        s = s + np.abs(np.asarray(bias, dtype=np.float64).reshape(-1))
    K = W64.shape[1]
    u = 2.0 ** -24
    gamma = (K + 1) * u / (1 - (K + 1) * u)
    exact = np.abs(gemv_fp64(x, W, bias))
    # fp16 ulp of the exact value (subnormal spacing 2^-24 below 2^-14)
    e = np.floor(np.log2(np.maximum(exact, 2.0 ** -14)))
    ulp16 = 2.0 ** (e - 10)
    return ulp16 + gamma * s


def fp16_linear_ref(x, W, bias=None) -> np.ndarray:
    """fp16(exact) of one decode-step linear: the oracle's output in fp16."""
    return gemv_fp64(x, W, bias).astype(np.float16)
