"""GPU parity at the benchmark configurations that hold pages in pinned host
memory, each at its stated full shape, through HELM's runtime API
(KVAllocator / KVCacheManager / perform_streaming_attention /
_decode_batched, kv_cache.py:405-662, kv_offload.py:86-186):

* Qwen3-8B, 32,768 tokens (2,048 pages of 16), bf16, the oldest 50% of the
  pages in pinned host memory;
* Llama-2-13B (MHA, 40 / 40 heads), 131,072 tokens (8,192 pages), fp16, the
  oldest 75% in pinned host memory;
* Qwen3-14B, 40 layers x 4 sequences x 65,536 tokens, bf16: the 64 GB device
  budget (nothing evicted) and a 32 GB budget (about a quarter of the pages
  in pinned host memory), three decode steps.

Outputs against the fp64 oracle (2e-3 fp16, 1e-2 bf16, the tolerances
HELM's tests use); page contents against the source tensors bit for bit.
Attention runs under HELM's decode mask (zeros, pipeline_runtime.py:79-92),
the production path, and also without a mask (Path 3) where noted.
"""
import math
import random

import numpy as np
import pytest
import torch

from helm_amd import _native
from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager, perform_streaming_attention
from helm_amd.runtime.kv_offload import _decode_batched
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _page_bytes(Hkv, D, P, es):
    return 2 * Hkv * P * D * es


def _layer_kv(mgr, lid):
    """The layer's K and V [Hkv, T, D] gathered from its pages (host and
    device), on the CPU."""
    pages = [p for p in mgr.layers[lid].pages if p.used_tokens > 0 and p.state != "DEAD"]
    K = torch.cat([p.k_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
    V = torch.cat([p.v_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
    return K, V


def _max_err(out, q, K, V, heads, G, mask=None):
    """Max |out - fp64| over the query heads of the given KV heads."""
    worst = 0.0
    for kvh in heads:
        hs = slice(kvh * G, (kvh + 1) * G)
        ref = A.attention_fp64_batched(q[hs].float(), K[kvh:kvh + 1].float(),
                                       V[kvh:kvh + 1].float(), mask=mask)
        worst = max(worst, (out[hs].double().cpu() - ref).abs().max().item())
    return worst


def _prefill_with_budget(Hkv, D, T, dtype, host_pages, seed):
    """One layer of T tokens appended page by page through append_prefill,
    with the watermark set so that exactly the oldest `host_pages` pages end
    up evicted (HELM's policy: the evictable excess over the watermark,
    oldest first, after every appended page)."""
    P = 16
    es = torch.tensor([], dtype=dtype).element_size()
    n = T // P
    watermark = (n - 1 - host_pages) * _page_bytes(Hkv, D, P, es)
    a = KVAllocator(1, Hkv, D, page_size=P, dtype=dtype)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=watermark)
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    v = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    mgr.append_prefill(0, k, v)
    pages = mgr.layers[0].pages
    states = [p.state for p in pages]
    assert states == ["CPU"] * host_pages + ["GPU"] * (n - host_pages)
    assert all(p.device.type == "cpu" and p.k_tensor.is_pinned() for p in pages[:host_pages])
    return mgr, k, v


@pytest.mark.parametrize("host_read", ["auto", "copy", "direct"])
def test_qwen3_8b_32k_half_offloaded(host_read, monkeypatch):
    """2,048 pages, the oldest 1,024 in pinned host memory: every query head
    of one decode call, masked (the loop) and unmasked (Path 3), host pages
    staged, read in place, or chosen per call; the gather is bit-exact."""
    if host_read != "auto":
        monkeypatch.setenv("HELM_AMD_HOST_READ", host_read)
    Hq, Hkv, D, T = 32, 8, 128, 32768
    mgr, k, v = _prefill_with_budget(Hkv, D, T, torch.bfloat16, 1024, seed=21)
    K, V = _layer_kv(mgr, 0)
    assert torch.equal(K, k[0].cpu()) and torch.equal(V, v[0].cpu())
    q = torch.randn((1, Hq, 1, D), generator=torch.Generator(device=DEV).manual_seed(22),
                    device=DEV, dtype=torch.bfloat16)
    KC.reset_paging_stats()
    mask = torch.zeros(1, 1, 1, T, device=DEV)
    out_m = perform_streaming_attention(q, mgr.iterate_layer_pages(0), attention_mask=mask)
    out_u = perform_streaming_attention(q, mgr.iterate_layer_pages(0))
    st = KC.get_paging_stats()
    assert (st["prefetch_calls"], st["pages_prefetched"]) == (2, 2048)
    assert st["bytes_prefetched"] == 2 * 1024 * _page_bytes(Hkv, D, 16, 2)
    G = Hq // Hkv
    assert _max_err(out_m[0], q[0].cpu(), K, V, range(Hkv), G) <= 1e-2
    assert _max_err(out_u[0], q[0].cpu(), K, V, range(Hkv), G) <= 1e-2
    mgr.clear()


def test_llama2_13b_128k_three_quarters_offloaded():
    """8,192 pages of 40 KV heads (fp16, MHA), the oldest 6,144 in pinned host
    memory: perform_streaming_attention over the layer's page list (records)
    and over a plain copy of the list (page by page), and one _decode_batched
    step (token append, residency, attention), against fp64 on four KV heads;
    the gather is bit-exact before and after the step."""
    Hq = Hkv = 40
    D, T = 128, 131072
    mgr, k, v = _prefill_with_budget(Hkv, D, T, torch.float16, 6144, seed=31)
    K, V = _layer_kv(mgr, 0)
    assert torch.equal(K, k[0].cpu()) and torch.equal(V, v[0].cpu())
    del k, v
    g = torch.Generator(device=DEV).manual_seed(32)
    q = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=torch.float16)
    heads = [0, 13, 27, 39]
    mask = torch.zeros(1, 1, 1, T, device=DEV)
    out = perform_streaming_attention(q, mgr.iterate_layer_pages(0), attention_mask=mask)
    assert _max_err(out[0], q[0].cpu(), K, V, heads, 1) <= 2e-3
    out_pl = perform_streaming_attention(q, list(mgr.iterate_layer_pages(0)),
                                         attention_mask=mask)
    assert _max_err(out_pl[0], q[0].cpu(), K, V, heads, 1) <= 2e-3
    # one decode step through the batched decode of the patched forwards
    kn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=torch.float16)
    vn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=torch.float16)
    q2 = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=torch.float16)
    mask2 = torch.zeros(1, 1, 1, T + 1, device=DEV)
    out2 = _decode_batched([mgr], q2, kn, vn, 0, 1 / math.sqrt(D), mask2)
    K2 = torch.cat([K, kn[0].cpu()], 1)
    V2 = torch.cat([V, vn[0].cpu()], 1)
    assert _max_err(out2[0], q2[0].cpu(), K2, V2, heads, 1) <= 2e-3
    Kg, Vg = _layer_kv(mgr, 0)
    assert torch.equal(Kg, K2) and torch.equal(Vg, V2)
    mgr.clear()


@pytest.mark.parametrize("budget_gb", [64, 32])
def test_qwen3_14b_40_layers_b4_64k_decode_steps(budget_gb):
    """The full decode step of the 40-layer configuration through
    _decode_batched, three steps, HELM's decode mask: four sequences of
    65,536 tokens per layer in pages from one shuffled free list (a random
    page table), the device budget split evenly over the sequences.  At 64
    GB nothing is evicted; at 32 GB a quarter of the pages sit in pinned host
    memory and are read back every step.  Sampled (layer, sequence) outputs
    of the last step against fp64 on all 8 KV heads, their pages bit-exact."""
    L, B, Hq, Hkv, D, T, P, steps = 40, 4, 40, 8, 128, 65536, 16, 3
    dtype = torch.bfloat16
    checked = [(0, 0), (17, 2), (39, 3)]
    a = KVAllocator(L, Hkv, D, page_size=P, dtype=dtype)
    a.reserve_batch(L * B * (T // P + 2), DEV)
    random.Random(5).shuffle(a.gpu_free_pool)
    per_item = budget_gb * 10 ** 9 // B
    mgrs = [KVCacheManager(a, gpu_high_watermark_bytes=per_item) for _ in range(B)]
    for m in mgrs:
        m.initialize_layer_caches(L)
    src = {}
    g = torch.Generator(device=DEV).manual_seed(41)
    for lid in range(L):
        for i, m in enumerate(mgrs):
            k = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
            v = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
            m.append_prefill(lid, k, v)
            if (lid, i) in checked:
                src[(lid, i)] = [k[0].cpu(), v[0].cpu()]
            del k, v
    host = sum(layer._n_host for m in mgrs for layer in m.layers.values())
    total = sum(len(layer.pages) for m in mgrs for layer in m.layers.values())
    if budget_gb == 64:
        assert host == 0
    else:
        assert 0.2 < host / total < 0.3
    scale = 1 / math.sqrt(D)
    outs, qs = {}, {}
    for step in range(steps):
        Tn = T + step + 1
        mask = torch.zeros(B, 1, 1, Tn, device=DEV)
        for lid in range(L):
            q = torch.randn((B, Hq, 1, D), generator=g, device=DEV, dtype=dtype)
            kn = torch.randn((B, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
            vn = torch.randn((B, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
            out = _decode_batched(mgrs, q, kn, vn, lid, scale, mask)
            for (cl, ci) in checked:
                if cl == lid:
                    src[(cl, ci)][0] = torch.cat([src[(cl, ci)][0], kn[ci].cpu()], 1)
                    src[(cl, ci)][1] = torch.cat([src[(cl, ci)][1], vn[ci].cpu()], 1)
                    outs[(cl, ci)] = out[ci].cpu()
                    qs[(cl, ci)] = q[ci].cpu()
    torch.cuda.synchronize()
    for (lid, i), (K, V) in src.items():
        Kg, Vg = _layer_kv(mgrs[i], lid)
        assert torch.equal(Kg, K) and torch.equal(Vg, V)
        assert _max_err(outs[(lid, i)], qs[(lid, i)], K, V, range(Hkv), Hq // Hkv) <= 1e-2
    for m in mgrs:
        m.clear()
    del mgrs, a
    torch.cuda.empty_cache()
