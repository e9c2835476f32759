"""Device and host-link profile — the measurements of HELM's device profiler
(helm/compiler/optimization/device_profiler.py) that feed its planner's
attention roofline (cost_model.py:639-691: KV bytes / bandwidth).

Same fields as HELM's ``_ProfilerResult`` (device_profiler.py:44-56), in
bytes/s or FLOP/s:

* ``gpu_mem_bw``: a 256 MB device copy counted as 2 x bytes per copy
  (``_bench_gpu``, :188-197) — here the native streaming-copy kernel of
  ``helm_measure_bandwidth`` (libhelm_amd.so), word-checked;
* ``pcie_h2d_bw`` / ``pcie_d2h_bw``: 64 MB copies between pinned host memory
  and the device (``_bench_pcie``, :217-240) — hipMemcpyAsync in the same
  native probe;
* ``gpu_flops_decode`` / ``gpu_flops_prefill``: HELM times torch matmuls of
  (1 | 128, H) x (H, H) in the model dtype (:199-211); the same timing here
  (the library has no GEMM of its own: these measure the device's BLAS);
* ``cpu_mem_bw`` / ``cpu_flops_decode`` / ``cpu_flops_prefill``: HELM's CPU
  probes (:120-185) — copies over many separately allocated buffers, decode
  FLOPS taken as the memory bandwidth (a GEMV at 1 FLOP/byte), fp32 GEMM at
  seq 128 — with torch on the host, as HELM measures them.

Results are cached per (hidden size, dtype, CPU units, device) as HELM
caches them; ``force=True`` measures again.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from helm_amd import _native

STREAM_BYTES = 256 * 1024 * 1024     # device copy (device_profiler.py:33)
PCIE_BYTES = 64 * 1024 * 1024        # host-link copies (:39)
PREFILL_SEQ = 128                    # GEMM rows of the prefill probe (:40)
TIMED_ITERS = 8                      # repetitions per probe (:42)
BUDGET_S = 0.4                       # wall-clock cap per timed probe (:43)


@dataclass
class ProfilerResult:
    cpu_mem_bw: float = 0.0
    cpu_flops_decode: float = 0.0
    cpu_flops_prefill: float = 0.0
    gpu_mem_bw: float = 0.0
    gpu_flops_decode: float = 0.0
    gpu_flops_prefill: float = 0.0
    pcie_h2d_bw: float = 0.0
    pcie_d2h_bw: float = 0.0


_cache: Dict[Tuple[int, str, int, Optional[int]], ProfilerResult] = {}


def measure_links(device: int = 0, stream_bytes: int = STREAM_BYTES,
                  link_bytes: int = PCIE_BYTES, iters: int = TIMED_ITERS) -> dict:
    """The native probe: device-copy, pinned H2D and D2H bandwidth of one
    device in bytes/s; raises when the copy did not move the bytes intact."""
    res = np.zeros(1, dtype=_native.BANDWIDTH_DTYPE)
    _native.call("helm_measure_bandwidth", int(device), int(stream_bytes), int(link_bytes),
                 int(iters), _native.ptr(res))
    r = {k: res[k][0].item() for k in res.dtype.names}
    if r["copy_mismatched_words"]:
        raise RuntimeError(f"device copy probe: {r['copy_mismatched_words']} words differ")
    return r


def _seconds_per_call(fn, sync) -> float:
    """Mean seconds per call after two warm-ups, as many calls (up to
    TIMED_ITERS) as fit BUDGET_S after a probe call (device_profiler.py:62-107)."""
    for _ in range(2):
        fn()
    sync()
    t = time.perf_counter()
    fn()
    sync()
    probe = time.perf_counter() - t
    n = max(1, min(TIMED_ITERS, int(BUDGET_S / max(probe, 1e-9))))
    t = time.perf_counter()
    for _ in range(n):
        fn()
    sync()
    return (time.perf_counter() - t) / n


def bench_gpu(hidden_size: int, dtype: torch.dtype, result: ProfilerResult,
              device: int = 0) -> None:
    """GPU fields of `result` (device_profiler.py:188-211)."""
    if not torch.cuda.is_available():
        return
    result.gpu_mem_bw = measure_links(device)["device_copy_bytes_per_s"]
    dev = torch.device("cuda", device)
    sync = torch.cuda.synchronize
    W = torch.randn(hidden_size, hidden_size, dtype=dtype, device=dev)
    x1 = torch.randn(1, hidden_size, dtype=dtype, device=dev)
    result.gpu_flops_decode = 2 * hidden_size * hidden_size / _seconds_per_call(
        lambda: torch.matmul(x1, W), sync)
    xp = torch.randn(PREFILL_SEQ, hidden_size, dtype=dtype, device=dev)
    result.gpu_flops_prefill = 2 * PREFILL_SEQ * hidden_size * hidden_size / _seconds_per_call(
        lambda: torch.matmul(xp, W), sync)


def bench_pcie(result: ProfilerResult, device: int = 0) -> None:
    """Host-link fields of `result` (device_profiler.py:217-240)."""
    if not torch.cuda.is_available():
        result.pcie_h2d_bw = result.pcie_d2h_bw = 0.0
        return
    r = measure_links(device, stream_bytes=1 << 20)
    result.pcie_h2d_bw = r["h2d_bytes_per_s"]
    result.pcie_d2h_bw = r["d2h_bytes_per_s"]


def bench_cpu(hidden_size: int, result: ProfilerResult, n_cpu_units: int = 0) -> None:
    """Host fields of `result` (device_profiler.py:120-185): copies over
    max(8, min(4 x units, 256)) separately allocated fp16 buffers of up to
    one H x H weight each (512 MB in all at most), counted as read + write;
    decode FLOPS = that bandwidth; fp32 GEMM at seq 128."""
    n_bufs = max(8, min(n_cpu_units * 4, 256))
    per_buf = max(1 << 20, min(hidden_size * hidden_size * 2, (512 << 20) // n_bufs))
    srcs = [torch.randn(per_buf // 2, dtype=torch.float16) for _ in range(n_bufs)]
    dst = torch.empty(per_buf // 2, dtype=torch.float16)

    def copy_all():
        for s in srcs:
            dst.copy_(s)
    result.cpu_mem_bw = 2 * n_bufs * per_buf / _seconds_per_call(copy_all, lambda: None)
    result.cpu_flops_decode = result.cpu_mem_bw
    W = torch.randn(hidden_size, hidden_size)
    xp = torch.randn(PREFILL_SEQ, hidden_size)
    result.cpu_flops_prefill = 2 * PREFILL_SEQ * hidden_size * hidden_size / _seconds_per_call(
        lambda: torch.matmul(xp, W), lambda: None)


def profile(hidden_size: int, dtype: torch.dtype, allow_gpu: bool = True,
            force: bool = False, n_cpu_units: int = 0) -> ProfilerResult:
    """Every probe, cached per (hidden size, dtype, CPU units, device)."""
    device = torch.cuda.current_device() if allow_gpu and torch.cuda.is_available() else None
    key = (hidden_size, str(dtype), n_cpu_units, device)
    if not force and key in _cache:
        return _cache[key]
    r = ProfilerResult()
    bench_cpu(hidden_size, r, n_cpu_units)
    if device is not None:
        bench_gpu(hidden_size, dtype, r, device)
        bench_pcie(r, device)
    _cache[key] = r
    return r
