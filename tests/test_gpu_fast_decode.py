"""The one-call decode step (helm_decode_step through the runtime's fast
path of _decode_batched) against the general path (HELM_AMD_FAST_DECODE=0)
on the GPU: the same output bits, the same page contents, the same paging
counters and page states, step after step, across page boundaries (where the
fast path hands over to the general one), under HELM's decode mask in bf16
and with a watermark that evicts; and the fast path is taken whenever its
conditions hold."""
import math

import pytest
import torch

from helm_amd import _native
from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager
from helm_amd.runtime.kv_offload import _decode_batched
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _managers(lens, page, watermark, seed, Hkv=8, D=128, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    alloc = KVAllocator(1, Hkv, D, page_size=page, dtype=dtype)
    mgrs = [KVCacheManager(alloc, gpu_high_watermark_bytes=watermark) for _ in lens]
    for m, T in zip(mgrs, lens):
        m.append_prefill(0, torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype),
                         torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype))
    return mgrs


def _kv(mgr):
    pages = [p for p in mgr.layers[0].pages if p.used_tokens > 0]
    return (torch.cat([p.k_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1),
            torch.cat([p.v_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1))


@pytest.mark.parametrize("lens,page,masked,watermark", [
    ([3000], 16, True, 1 << 40), ([3000], 16, False, 1 << 40), ([1000, 77, 2050], 16, True, 1 << 40),
    ([700], 64, True, 1 << 40), ([3000], 16, True, 2 * 1024 * 1024),
])
def test_fast_decode_equals_the_general_path(lens, page, masked, watermark, monkeypatch):
    Hq, Hkv, D = 32, 8, 128
    runs = {}
    calls = {"fast": 0}
    real = _native.entry("helm_decode_step")

    def counting(*a):
        calls["fast"] += 1
        return real(*a)

    for mode in ("fast", "general"):
        monkeypatch.setenv("HELM_AMD_FAST_DECODE", "1" if mode == "fast" else "0")
        if mode == "fast":
            monkeypatch.setitem(_native._entries, "helm_decode_step", counting)
        mgrs = _managers(lens, page, watermark, seed=5)
        g = torch.Generator(device=DEV).manual_seed(6)
        B = len(lens)
        outs = []
        KC.reset_paging_stats()
        for step in range(40):
            q = torch.randn((B, Hq, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
            kn = torch.randn((B, Hkv, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
            vn = torch.randn((B, Hkv, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
            mask = None
            if masked:
                T = max(lens) + step + 1
                mask = torch.zeros((B, 1, 1, T), device=DEV, dtype=torch.bfloat16)
                mask[..., 3:9] = torch.finfo(torch.bfloat16).min
            outs.append(_decode_batched(mgrs, q, kn, vn, 0, 1 / math.sqrt(D), mask).cpu())
        torch.cuda.synchronize()
        runs[mode] = (outs, [_kv(m) for m in mgrs], KC.get_paging_stats(),
                      [[p.state for p in m.layers[0].pages] for m in mgrs],
                      [m.layers[0].total_tokens for m in mgrs], q, mask)
        monkeypatch.undo()
    fast, gen = runs["fast"], runs["general"]
    for a, b in zip(fast[0], gen[0]):
        assert torch.equal(a, b)
    for (ka, va), (kb, vb) in zip(fast[1], gen[1]):
        assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert fast[2] == gen[2] and fast[3] == gen[3] and fast[4] == gen[4]
    # the fast path took the steps whose tail had room (all but the page
    # boundaries) unless pages live on the host
    if watermark > 1 << 30:
        assert calls["fast"] >= 40 - (40 // page + 2) * len(lens)
    # the last step against fp64
    q, mask = fast[5], fast[6]
    for b, (K, V) in enumerate(fast[1]):
        mk = None if mask is None else mask[b, :, :, :K.shape[1]].float().cpu()
        for kvh in (0, Hkv - 1):
            hs = slice(kvh * 4, (kvh + 1) * 4)
            ref = A.attention_fp64_batched(q[b, hs].float().cpu(), K[kvh:kvh + 1].float(),
                                           V[kvh:kvh + 1].float(), mask=mk)
            assert (fast[0][-1][b, hs].double() - ref).abs().max().item() <= 1e-2
