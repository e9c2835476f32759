"""Per-device native engine handles (side stream, workspace, staging ring).

One `helm_engine` per HIP device, created on first use and destroyed at
interpreter exit.  The engine's side stream is what HELM's per-device
``_get_kv_copy_stream`` (helm/runtime/kv_cache.py:383-391) memoizes.
"""
from __future__ import annotations

import atexit
import ctypes
import os
from typing import Dict

import torch

from helm_amd import _native

_engines: Dict[int, ctypes.c_void_p] = {}
_copy_streams: Dict[int, torch.cuda.ExternalStream] = {}


def device_index(device: torch.device) -> int:
    if device.type != "cuda":
        raise ValueError(f"expected a HIP device, got {device}")
    return device.index if device.index is not None else torch.cuda.current_device()


def get_engine(device: torch.device) -> ctypes.c_void_p:
    idx = device.index if device.index is not None else device_index(device)
    eng = _engines.get(idx)
    if eng is None:
        _native.load()
        chunk = int(os.environ.get("HELM_AMD_CHUNK_MB", "64")) << 20
        slots = int(os.environ.get("HELM_AMD_RING_SLOTS", "2"))
        handle = ctypes.c_void_p()
        with torch.cuda.device(idx):
            _native.call("helm_engine_create", idx, chunk, slots, ctypes.byref(handle))
        _engines[idx] = eng = handle
    return eng


def copy_stream(device: torch.device) -> torch.cuda.ExternalStream:
    """The engine's side stream as a torch stream object (memoized per device)."""
    idx = device_index(device)
    s = _copy_streams.get(idx)
    if s is None:
        ptr = _native.load().helm_engine_copy_stream(get_engine(device))
        s = torch.cuda.ExternalStream(ptr, device=torch.device("cuda", idx))
        _copy_streams[idx] = s
    return s


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (torch's raw-stream
    query where this torch has it: no Stream object per call)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


@atexit.register
def _destroy_engines() -> None:
    if not _engines:
        return
    lib = _native.load()
    for eng in _engines.values():
        lib.helm_engine_destroy(eng)
    _engines.clear()
    _copy_streams.clear()
