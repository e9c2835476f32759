"""The device / host-link profile (HELM's device_profiler.py:188-240): the
native bandwidth probe on the GPU, HELM's CPU probes on the host."""
import numpy as np
import pytest
import torch

from helm_amd import _native
from helm_amd import device_profiler as DP


def test_probe_rejects_bad_arguments_before_touching_a_device():
    lib = _native.load()
    res = np.zeros(1, dtype=_native.BANDWIDTH_DTYPE)
    assert lib.helm_measure_bandwidth(0, 1 << 20, 1 << 20, 0, _native.ptr(res)) == \
        _native.HELM_E_INVALID
    assert lib.helm_measure_bandwidth(0, 100, 1 << 20, 1, _native.ptr(res)) == \
        _native.HELM_E_INVALID
    assert lib.helm_measure_bandwidth(0, 1 << 20, 1 << 20, 1, None) == _native.HELM_E_INVALID


def test_cpu_fields_and_cache():
    r = DP.profile(256, torch.float16, allow_gpu=False)
    assert r.cpu_mem_bw > 1e8 and r.cpu_flops_decode == r.cpu_mem_bw
    assert r.cpu_flops_prefill > 1e8
    assert DP.profile(256, torch.float16, allow_gpu=False) is r
    assert r.gpu_mem_bw == 0.0 and r.pcie_h2d_bw == 0.0


@pytest.mark.gpu
def test_gpu_and_link_bandwidth_are_measured():
    """HBM copy between 1 and 8.5 TB/s (MI355X peak 8 TB/s), the copy word-
    exact; pinned H2D / D2H between 5 and 70 GB/s (PCIe Gen5 x16: ~63)."""
    r = DP.measure_links(0, stream_bytes=DP.STREAM_BYTES, link_bytes=DP.PCIE_BYTES)
    assert r["copy_mismatched_words"] == 0
    assert 1e12 < r["device_copy_bytes_per_s"] < 8.5e12
    assert 5e9 < r["h2d_bytes_per_s"] < 70e9
    assert 5e9 < r["d2h_bytes_per_s"] < 70e9
    p = DP.profile(1024, torch.bfloat16, force=True)
    assert p.gpu_mem_bw > 1e12 and p.pcie_h2d_bw > 5e9 and p.pcie_d2h_bw > 5e9
    assert p.gpu_flops_decode > 0 and p.gpu_flops_prefill > p.gpu_flops_decode
