"""The library's HELM_AMD_* switches are read per call (GPU).  Every entry
point that plans a launch takes one pass over the environment for them, so a
switch set or cleared between two calls applies to the second: here
HELM_AMD_PPS (pages per split) changes the decode kernel's grid, counted by
the per-workgroup stamp probe (helm_profile_workgroup_stamps), on the pool
entry point and on the one-call decode step."""
import math

import pytest
import torch

from helm_amd import _native
from helm_amd import workloads as W
from helm_amd.paged import paged_decode_attention
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager
from helm_amd.runtime.kv_offload import _decode_batched

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NWG = 1 << 14


def _workgroups(fn):
    """Workgroups of the next matrix-core decode launch that `fn` makes."""
    buf = torch.zeros(NWG * 4, dtype=torch.int64, device=DEV)
    torch.cuda.synchronize()
    _native.call("helm_profile_workgroup_stamps", buf.data_ptr(), NWG)
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        _native.call("helm_profile_workgroup_stamps", None, 0)
    return int((buf.view(-1, 4)[:, 0] > 0).sum())


def test_pages_per_split_switch_applies_to_the_next_call(monkeypatch):
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=3, device=DEV)
    call = lambda: paged_decode_attention(case["q"], case["k_pool"], case["v_pool"],
                                          case["table"], case["lens"],
                                          max_pages=case["max_pages"])
    monkeypatch.delenv("HELM_AMD_PPS", raising=False)
    base = _workgroups(call)
    assert base == 32 * w.Hkv                       # 32 splits of 64 pages per KV head
    monkeypatch.setenv("HELM_AMD_PPS", "32")
    assert _workgroups(call) == 64 * w.Hkv
    monkeypatch.setenv("HELM_AMD_PPS", "128")
    assert _workgroups(call) == 16 * w.Hkv
    monkeypatch.delenv("HELM_AMD_PPS")
    assert _workgroups(call) == base


def test_switch_applies_to_the_one_call_decode_step(monkeypatch):
    Hq, Hkv, D, T = 32, 8, 128, 8180                # 512 pages of 16, room in the tail
    alloc = KVAllocator(1, Hkv, D, page_size=16, dtype=torch.bfloat16)
    mgr = KVCacheManager(alloc, gpu_high_watermark_bytes=1 << 40)
    g = torch.Generator(device=DEV).manual_seed(4)
    mgr.append_prefill(0, torch.randn((1, Hkv, T, D), generator=g, device=DEV,
                                      dtype=torch.bfloat16),
                       torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=torch.bfloat16))
    q = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
    k = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
    step = lambda: _decode_batched([mgr], q, k, k, 0, 1 / math.sqrt(D), None)
    counts = []
    for pps in (None, "8", None):
        if pps is None:
            monkeypatch.delenv("HELM_AMD_PPS", raising=False)
        else:
            monkeypatch.setenv("HELM_AMD_PPS", pps)
        counts.append(_workgroups(step))
    assert counts[1] == 64 * Hkv                    # 512 pages in splits of 8
    assert counts[0] == counts[2] and counts[0] != counts[1]
