"""HELM's runtime unit-test cases, restated against this package.

Each test below checks the behaviour one of HELM's own unit tests checks
(tests/unit/runtime/test_streaming_attention.py, test_kv_cache.py,
test_kv_allocator.py, test_batch_kv_offload.py, test_kv_offload.py; where a
test here covers one HELM case it has that case's name, and neighbouring cases
are merged, each of them also under its own HELM name in
tests/test_helm_unit_names.py), through ``helm_amd.runtime`` instead of
``helm.runtime``, so
that a HELM user who swaps the modules finds the cases they rely on green.
HELM runs these on the CPU; so do they here: a query and pages on the CPU go
to the host-CPU attention of libhelm_cpu.so (no torch fallback).  The
streaming-attention cases also run on the GPU (marked ``gpu``) over device
pages.  References are plain float32 attention, as HELM's tests use.
"""
import copy
import math
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from helm_amd import _cpu_native
from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime import kv_offload as KO
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager, KVPage, LayerKVCache
from helm_amd.runtime.kv_cache import perform_streaming_attention

CPU = torch.device("cpu")
needs_host_kernel = pytest.mark.skipif(_cpu_native.try_load()[0] is None,
                                       reason="libhelm_cpu.so cannot run on this CPU")


def _devices():
    return [pytest.param("cpu", marks=needs_host_kernel),
            pytest.param("cuda", marks=pytest.mark.gpu)]


# ── streaming attention (HELM's test_streaming_attention.py) ─────────────────

def _page(k, v, page_id=0, start=0):
    """k / v [B, H, n, D] as one page holding n tokens, resident on their device."""
    state = "GPU" if k.device.type == "cuda" else "CPU"
    return KVPage(page_id=page_id, layer_id=0, start_token=start, used_tokens=k.size(2),
                  capacity_tokens=k.size(2), k_tensor=k.clone(), v_tensor=v.clone(),
                  device=k.device, state=state)


def _reference(q, k, v, scale=None, mask=None, softcap=None):
    """float32 softmax(q k^T * scale [cap] [+ mask]) v, KV heads expanded."""
    scale = 1.0 / math.sqrt(q.size(-1)) if scale is None else scale
    g = q.size(1) // k.size(1)
    k = k.float().cpu().repeat_interleave(g, dim=1)
    v = v.float().cpu().repeat_interleave(g, dim=1)
    w = q.float().cpu() @ k.transpose(-2, -1) * scale
    if softcap is not None:
        w = torch.tanh(w / softcap) * softcap
    if mask is not None:
        w = w + mask.float().cpu()
    return torch.softmax(w, dim=-1) @ v


def _pages(sizes, dev, B=1, H=2, D=8, Hkv=None, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    Hkv = Hkv or H
    pages, ks, vs, start = [], [], [], 0
    for i, n in enumerate(sizes):
        k = torch.randn(B, Hkv, n, D, generator=g).to(dtype)
        v = torch.randn(B, Hkv, n, D, generator=g).to(dtype)
        pages.append(_page(k.to(dev), v.to(dev), i, start))
        ks.append(k)
        vs.append(v)
        start += n
    return pages, torch.cat(ks, 2), torch.cat(vs, 2)


def _q(B, H, D, dev, dtype=torch.float32, seed=100):
    return torch.randn(B, H, 1, D, generator=torch.Generator().manual_seed(seed)).to(dtype).to(dev)


@pytest.mark.parametrize("dev", _devices())
@pytest.mark.parametrize("sizes,H,D", [([4], 2, 8), ([4, 3], 2, 8), ([3, 5, 2], 1, 16)],
                         ids=["test_single_page_matches_eager", "test_two_pages_match_eager",
                              "test_three_pages_match_eager"])
def test_pages_match_eager(sizes, H, D, dev):
    pages, K, V = _pages(sizes, dev, H=H, D=D)
    q = _q(1, H, D, dev)
    out = perform_streaming_attention(q, pages)
    assert out.shape == q.shape and out.device == q.device
    assert torch.allclose(out.cpu(), _reference(q, K, V), atol=1e-4)


@pytest.mark.parametrize("dev", _devices())
def test_no_pages_returns_zeros(dev):
    q = _q(1, 2, 8, dev)
    out = perform_streaming_attention(q, [])
    assert out.shape == (1, 2, 1, 8) and torch.all(out == 0)


@pytest.mark.parametrize("dev", _devices())
def test_page_with_zero_used_tokens_skipped(dev):
    pages, _, _ = _pages([4], dev)
    pages[0].used_tokens = 0
    out = perform_streaming_attention(_q(1, 2, 8, dev), pages)
    assert torch.allclose(out.cpu(), torch.zeros(1, 2, 1, 8), atol=1e-6)


@pytest.mark.parametrize("dev", _devices())
def test_mixed_empty_and_nonempty_page(dev):
    pages, _, _ = _pages([4, 4], dev)
    pages[0].used_tokens = 0
    q = _q(1, 2, 8, dev)
    assert torch.allclose(perform_streaming_attention(q, pages).cpu(),
                          perform_streaming_attention(q, pages[1:]).cpu(), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
def test_custom_scale(dev):
    pages, K, V = _pages([3], dev, H=1, D=4)
    q = _q(1, 1, 4, dev)
    out = perform_streaming_attention(q, pages, scale=0.25)
    assert torch.allclose(out.cpu(), _reference(q, K, V, scale=0.25), atol=1e-4)


@pytest.mark.parametrize("dev", _devices())
def test_default_scale_is_inv_sqrt_head_dim(dev):
    pages, _, _ = _pages([4], dev, H=1, D=16)
    q = _q(1, 1, 16, dev)
    assert torch.allclose(perform_streaming_attention(q, pages).cpu(),
                          perform_streaming_attention(q, pages, scale=0.25).cpu(), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16],
                         ids=["test_output_dtype_matches_query_float32",
                              "test_output_dtype_matches_query_float16"])
def test_output_dtype_matches_query(dtype, dev):
    pages, _, _ = _pages([4], dev, dtype=dtype)
    assert perform_streaming_attention(_q(1, 2, 8, dev, dtype), pages).dtype == dtype


@pytest.mark.parametrize("dev", _devices())
def test_output_shape_matches_query(dev):
    """Batch 2, one page holding both sequences' K/V ([2, H, n, D])."""
    pages, K, V = _pages([6], dev, B=2, H=4, D=16)
    q = torch.randn(2, 4, 1, 16, generator=torch.Generator().manual_seed(3)).to(dev)
    out = perform_streaming_attention(q, pages)
    assert out.shape == (2, 4, 1, 16)
    assert torch.allclose(out.cpu(), _reference(q, K, V), atol=1e-4)


@pytest.mark.parametrize("dev", _devices())
@pytest.mark.parametrize("sizes", [[6], [4, 3]],
                         ids=["test_gqa_matches_eager_expanded", "test_gqa_multi_page_matches_eager"])
def test_gqa_matches_eager(sizes, dev):
    pages, K, V = _pages(sizes, dev, H=4, Hkv=2, D=8)
    q = _q(1, 4, 8, dev)
    out = perform_streaming_attention(q, pages)
    assert out.shape == (1, 4, 1, 8)
    assert torch.allclose(out.cpu(), _reference(q, K, V), atol=1e-4)


@pytest.mark.parametrize("dev", _devices())
def test_large_logits_no_nan(dev):
    k = torch.full((1, 1, 8, 64), 100.0)
    v = torch.randn(1, 1, 8, 64, generator=torch.Generator().manual_seed(4))
    out = perform_streaming_attention(torch.full((1, 1, 1, 64), 100.0).to(dev),
                                      [_page(k.to(dev), v.to(dev))])
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("dev", _devices())
def test_online_softmax_zero_mask_matches_unmasked_eager(dev):
    pages, K, V = _pages([3, 5, 2], dev)
    q = _q(1, 2, 8, dev)
    out = perform_streaming_attention(q, pages, attention_mask=torch.zeros(1, 1, 1, 10).to(dev))
    assert torch.allclose(out.cpu(), _reference(q, K, V), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
def test_online_softmax_padding_mask_matches_masked_eager(dev):
    """-inf entries spanning a page boundary."""
    pages, K, V = _pages([4, 4, 3], dev, seed=1)
    q = _q(1, 2, 8, dev, seed=101)
    mask = torch.zeros(1, 1, 1, 11)
    mask[..., 2:6] = float("-inf")
    out = perform_streaming_attention(q, pages, attention_mask=mask.to(dev))
    assert torch.allclose(out.cpu(), _reference(q, K, V, mask=mask), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
def test_online_softmax_fully_masked_page_matches_eager(dev):
    """A whole page masked out contributes nothing."""
    pages, K, V = _pages([3, 4, 2], dev, seed=2)
    q = _q(1, 2, 8, dev, seed=102)
    mask = torch.zeros(1, 1, 1, 9)
    mask[..., 3:7] = float("-inf")
    out = perform_streaming_attention(q, pages, attention_mask=mask.to(dev))
    assert torch.allclose(out.cpu(), _reference(q, K, V, mask=mask), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
def test_online_softmax_softcap_matches_eager(dev):
    pages, K, V = _pages([5, 3], dev, seed=3)
    q = (_q(1, 2, 8, dev, seed=103) * 4).contiguous()
    out = perform_streaming_attention(q, pages, softcap=5.0)
    assert torch.allclose(out.cpu(), _reference(q, K, V, softcap=5.0), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
def test_online_softmax_gqa_expansion_with_mask(dev):
    pages, K, V = _pages([4, 4], dev, H=4, Hkv=2, seed=4)
    q = _q(1, 4, 8, dev, seed=104)
    mask = torch.zeros(1, 1, 1, 8)
    mask[..., 5] = float("-inf")
    out = perform_streaming_attention(q, pages, attention_mask=mask.to(dev))
    assert torch.allclose(out.cpu(), _reference(q, K, V, mask=mask), atol=1e-5)


@pytest.mark.parametrize("dev", _devices())
def test_online_softmax_fp16_query_matches_eager(dev):
    pages, K, V = _pages([3, 4], dev, dtype=torch.float16, seed=5)
    q = _q(1, 2, 8, dev, torch.float16, seed=105)
    out = perform_streaming_attention(q, pages, attention_mask=torch.zeros(1, 1, 1, 7).to(dev))
    assert out.dtype == torch.float16
    assert torch.allclose(out.float().cpu(), _reference(q, K, V), atol=2e-3)


# ── KV cache (HELM's test_kv_cache.py) ───────────────────────────────────────

H, D, P, L = 2, 8, 4, 4


@pytest.fixture()
def allocator():
    return KVAllocator(num_layers=L, num_kv_heads=H, head_dim=D, page_size=P, dtype=torch.float32)


@pytest.fixture()
def cache(allocator):
    mgr = KVCacheManager(allocator, gpu_high_watermark_bytes=0)
    mgr.initialize_layer_caches(num_layers=L)
    return mgr


def _kv(n, seed=0, heads=H, dim=D):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, heads, n, dim, generator=g), torch.randn(1, heads, n, dim, generator=g)


def test_layer_cache_append_page_and_tail_updates(allocator):
    layer = LayerKVCache(layer_id=0)
    p1, p2 = allocator.allocate(CPU), allocator.allocate(CPU)
    layer.append_page(p1)
    assert len(layer.pages) == 1 and layer.tail_page is p1
    layer.append_page(p2)
    assert layer.tail_page is p2


def test_initialize_creates_n_layers(cache):
    assert cache.num_layers() == L
    assert sorted(cache.layers_keys()) == list(range(L))
    assert cache.seq_len() == 0


@pytest.mark.parametrize("n,pages", [(3, 1), (P, 1), (3 * P + 1, 4)],
                         ids=["test_prefill_single_page_when_short", "test_prefill_exact_one_page",
                              "test_prefill_multiple_pages_when_long"])
def test_prefill_page_count(cache, n, pages):
    cache.append_prefill(0, *_kv(n))
    assert len(cache.layers[0].pages) == pages
    assert cache.layers[0].total_tokens == n


def test_prefill_data_preserved_and_start_tokens(cache):
    k, v = _kv(2 * P + 2, seed=1)
    cache.append_prefill(0, k, v)
    pages = cache.layers[0].pages
    assert [p.start_token for p in pages] == [0, P, 2 * P]
    got_k = torch.cat([p.k_tensor[:, :, :p.used_tokens] for p in pages], 2)
    got_v = torch.cat([p.v_tensor[:, :, :p.used_tokens] for p in pages], 2)
    assert torch.equal(got_k, k) and torch.equal(got_v, v)


def test_prefill_auto_creates_layer(allocator):
    mgr = KVCacheManager(allocator, gpu_high_watermark_bytes=0)
    mgr.append_prefill(7, *_kv(2))
    assert 7 in mgr.layers and mgr.layers[7].total_tokens == 2


def test_decode_increments_and_pages(cache):
    cache.append_prefill(0, *_kv(P - 1))
    cache.append_decode(0, *_kv(1, seed=2))
    assert cache.layers[0].total_tokens == P and len(cache.layers[0].pages) == 1
    assert cache.seq_len() == P
    cache.append_decode(0, *_kv(1, seed=3))             # tail full: a new page
    assert len(cache.layers[0].pages) == 2
    for s in range(2 * P):
        cache.append_decode(0, *_kv(1, seed=10 + s))
    assert cache.layers[0].total_tokens == 3 * P + 1 and len(cache.layers[0].pages) == 4


def test_iterate_layer_pages(cache):
    cache.append_prefill(0, *_kv(P + 1))
    pages = cache.iterate_layer_pages(0)
    assert isinstance(pages, list) and len(pages) == 2
    assert cache.iterate_layer_pages(99) == []


def test_seq_len_from_layer_0(allocator):
    mgr = KVCacheManager(allocator, gpu_high_watermark_bytes=0)
    assert mgr.seq_len() == 0
    mgr.append_prefill(1, *_kv(3))
    assert mgr.seq_len() == 0
    mgr.append_prefill(0, *_kv(5))
    assert mgr.seq_len() == 5


def test_report_bytes(cache):
    r = cache.report_bytes_per_tier()
    assert {"gpu_active_bytes", "cpu_active_bytes"} <= set(r)
    cache.append_prefill(0, *_kv(P + 1))
    r = cache.report_bytes_per_tier()
    assert r["gpu_active_bytes"] == 0
    assert r["cpu_active_bytes"] == 2 * (2 * H * P * D * 4)     # two whole pages, K and V


def test_clear_resets_layers_and_frees_pages(cache, allocator):
    cache.append_prefill(0, *_kv(2 * P))
    used = allocator.report_usage()["active_cpu_pages"]
    assert used > 0
    cache.clear()
    assert len(cache.layers) == 0
    assert allocator.report_usage()["active_cpu_pages"] == 0


def test_evict_and_watermark_no_crash_cpu_only(cache):
    cache.append_prefill(0, *_kv(3 * P))
    cache.evict_pages(10 ** 9)                          # no GPU pages: nothing moves
    cache.append_decode(0, *_kv(1, seed=5))             # watermark 0, CPU pages only
    assert all(p.state == "CPU" for p in cache.layers[0].pages)


def test_paging_stats_record_and_reset():
    KC.reset_paging_stats()
    assert all(v == 0 for v in KC.get_paging_stats().values())
    KC._record_eviction(2, 100)
    KC._record_eviction(1, 50)
    KC._record_prefetch(3, 300)
    KC._record_prefetch(0, 0)
    s = KC.get_paging_stats()
    assert (s["evict_calls"], s["pages_evicted"], s["bytes_evicted"]) == (2, 3, 150)
    assert (s["prefetch_calls"], s["pages_prefetched"], s["bytes_prefetched"]) == (1, 3, 300)
    KC.reset_paging_stats()
    assert all(v == 0 for v in KC.get_paging_stats().values())


def test_build_contiguous_honors_small_capacities():
    a = KVAllocator(num_layers=2, num_kv_heads=H, head_dim=D, page_size=P, dtype=torch.float32)
    for cap in (1, 5, 100):
        mgr = KVCacheManager(a, gpu_high_watermark_bytes=0)
        assert mgr.build_contiguous(2, H, D, cap, CPU, torch.float32)
        assert mgr.use_contiguous and mgr.cont_capacity == cap


@pytest.mark.gpu
def test_evict_gpu_pages_to_cpu_tail_protected_and_counted():
    DEV = torch.device("cuda:0")
    a = KVAllocator(num_layers=1, num_kv_heads=H, head_dim=D, page_size=P, dtype=torch.float32)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    k, v = _kv(3 * P + 1, seed=6)
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    KC.reset_paging_stats()
    page_bytes = 2 * H * P * D * 4
    mgr.evict_pages(10 ** 9)
    states = [p.state for p in mgr.layers[0].pages]
    assert states == ["CPU", "CPU", "CPU", "GPU"]           # the tail stays
    s = KC.get_paging_stats()
    assert (s["pages_evicted"], s["bytes_evicted"]) == (3, 3 * page_bytes)
    q = torch.randn(1, H, 1, D, device=DEV)
    out = perform_streaming_attention(q, mgr.iterate_layer_pages(0))
    assert KC.get_paging_stats()["pages_prefetched"] == 3
    assert torch.allclose(out.cpu(), _reference(q, k, v), atol=1e-4)
    mgr.clear()


# ── allocator (HELM's test_kv_allocator.py) ──────────────────────────────────

def _alloc(**kw):
    args = dict(num_layers=2, num_kv_heads=2, head_dim=8, page_size=4, dtype=torch.float32)
    args.update(kw)
    return KVAllocator(**args)


def test_allocate_state_metadata_and_reserve():
    a = _alloc()
    assert a.cpu_total_pages == 0
    page = a.allocate(CPU)
    assert page.state == "CPU" and page.device.type == "cpu"
    assert a.cpu_total_pages > 1                         # a batch was reserved
    page.layer_id, page.start_token, page.used_tokens = 99, 500, 3
    a.free(page)
    assert page.state == "FREE"
    again = a.allocate(CPU)
    assert again is page                                 # LIFO reuse
    assert (again.layer_id, again.start_token, again.used_tokens) == (-1, 0, 0)


def test_page_shape_dtype_and_ids():
    a = KVAllocator(num_layers=2, num_kv_heads=3, head_dim=16, page_size=8)
    p = a.allocate(CPU)
    assert p.k_tensor.shape == p.v_tensor.shape == (1, 3, 8, 16)
    assert _alloc(dtype=torch.float16).allocate(CPU).k_tensor.dtype == torch.float16
    assert a.allocate(CPU).page_id != p.page_id


def test_free_returns_to_pool_and_reserve_batch():
    a = _alloc()
    page = a.allocate(CPU)
    before = len(a.cpu_free_pool)
    a.free(page)
    assert len(a.cpu_free_pool) == before + 1
    b = _alloc()
    b.reserve_batch(5, CPU)
    assert b.cpu_total_pages == 5 and len(b.cpu_free_pool) == 5
    b.reserve_batch(4, CPU)
    assert b.cpu_total_pages == 9


def test_move_page_same_device_and_report_usage():
    a = _alloc()
    page = a.allocate(CPU)
    page.used_tokens = 2
    page.k_tensor[:, :, :2] = 42.0
    page.v_tensor[:, :, :2] = 99.0
    moved = a.move_page(page, CPU)
    assert moved is page
    assert torch.all(moved.k_tensor[:, :, :2] == 42.0) and torch.all(moved.v_tensor[:, :, :2] == 99.0)
    r = a.report_usage()
    for key in ("gpu_pool_size", "cpu_pool_size", "active_gpu_pages", "active_cpu_pages",
                "gpu_free_pages", "cpu_free_pages", "gpu_reserved_bytes", "cpu_reserved_bytes",
                "gpu_used_bytes", "cpu_used_bytes"):
        assert key in r
    assert r["active_cpu_pages"] >= 1 and r["cpu_used_bytes"] <= r["cpu_reserved_bytes"]


@pytest.mark.gpu
def test_gpu_allocate_and_move_page_cpu_to_gpu():
    DEV = torch.device("cuda:0")
    a = _alloc()
    assert a.allocate(DEV).state == "GPU"
    page = a.allocate(CPU)
    page.layer_id, page.start_token, page.used_tokens = 2, 8, 3
    page.k_tensor[:, :, :3] = 7.0
    page.v_tensor[:, :, :3] = 8.0
    before = len(a.cpu_free_pool)
    new = a.move_page(page, DEV)
    assert new.device.type == "cuda" and (new.layer_id, new.start_token, new.used_tokens) == (2, 8, 3)
    assert torch.equal(new.k_tensor[:, :, :3].cpu(), torch.full((1, 2, 3, 8), 7.0))
    assert torch.equal(new.v_tensor[:, :, :3].cpu(), torch.full((1, 2, 3, 8), 8.0))
    assert len(a.cpu_free_pool) == before + 1            # the old page went back
    empty = a.allocate(CPU)
    assert a.move_page(empty, DEV).used_tokens == 0


# ── batch of managers (HELM's test_batch_kv_offload.py) ──────────────────────

@pytest.fixture()
def balloc():
    return KVAllocator(num_layers=4, num_kv_heads=2, head_dim=16, page_size=8, dtype=torch.float32)


def test_batch_kvcm_independent_layers_and_counts(balloc):
    kvcms = [KVCacheManager(balloc, gpu_high_watermark_bytes=0) for _ in range(3)]
    kvcms[0].append_prefill(0, *_kv(4, heads=2, dim=16))
    kvcms[1].append_prefill(0, *_kv(8, heads=2, dim=16))
    assert 0 in kvcms[0].layers and 0 not in kvcms[2].layers
    assert (kvcms[0].layers[0].total_tokens, kvcms[1].layers[0].total_tokens) == (4, 8)
    kvcms[1].append_decode(0, *_kv(1, heads=2, dim=16))
    assert (kvcms[0].layers[0].total_tokens, kvcms[1].layers[0].total_tokens) == (4, 9)


def test_batch_reset_returns_pages_to_pool(balloc):
    kvcms = [KVCacheManager(balloc, gpu_high_watermark_bytes=0) for _ in range(2)]
    for m in kvcms:
        m.append_prefill(0, *_kv(4, heads=2, dim=16))
    assert balloc.report_usage()["active_cpu_pages"] > 0
    for m in kvcms:
        m.clear()
    assert all(len(m.layers) == 0 for m in kvcms)
    assert balloc.report_usage()["active_cpu_pages"] == 0


@needs_host_kernel
def test_streaming_attention_batch_shape_and_independent(balloc):
    """Per-item decode attention over each item's own pages: shapes, and each
    item equal to attention over its own K/V only."""
    B, n = 3, 12
    kvcms = [KVCacheManager(balloc, gpu_high_watermark_bytes=0) for _ in range(B)]
    K, V = [], []
    for i, m in enumerate(kvcms):
        k, v = _kv(n, seed=20 + i, heads=2, dim=16)
        m.append_prefill(0, k, v)
        K.append(k)
        V.append(v)
    q = torch.randn(B, 2, 1, 16, generator=torch.Generator().manual_seed(30))
    outs = []
    for i, m in enumerate(kvcms):
        kd, vd = _kv(1, seed=40 + i, heads=2, dim=16)
        m.append_decode(0, kd, vd)
        outs.append(perform_streaming_attention(q[i:i + 1], m.iterate_layer_pages(0)))
        K[i], V[i] = torch.cat([K[i], kd], 2), torch.cat([V[i], vd], 2)
    out = torch.cat(outs, 0)
    assert out.shape == (B, 2, 1, 16)
    for i in range(B):
        assert torch.allclose(out[i:i + 1], _reference(q[i:i + 1], K[i], V[i]), atol=1e-4)


# ── offload manager and forwards (HELM's test_kv_offload.py) ─────────────────

def _tiny(arch="llama"):
    kw = dict(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
              num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
              attention_dropout=0.0)
    if arch == "mistral":
        from transformers.models.mistral import MistralConfig, MistralForCausalLM
        cfg = MistralConfig(sliding_window=None, **kw)
        cfg._attn_implementation = "eager"
        return MistralForCausalLM(cfg).eval()
    from transformers.models.llama import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(**kw)
    cfg._attn_implementation = "eager"
    return LlamaForCausalLM(cfg).eval()


def _single_decode(attn, model):
    hidden = torch.randn(1, 1, model.config.hidden_size)
    pos = torch.tensor([[0]])
    with torch.no_grad():
        attn(hidden, position_embeddings=model.model.rotary_emb(hidden, position_ids=pos),
             attention_mask=torch.zeros(1, 1, 1, 1), cache_position=torch.tensor([0]))


def _count_decodes(kvcm):
    calls = []
    orig = kvcm.append_decode

    def counting(*a, **kw):
        calls.append(1)
        return orig(*a, **kw)
    kvcm.append_decode = counting
    return calls


@needs_host_kernel
def test_mistral_patches_mistral_attention_not_llama():
    import transformers.models.mistral.modeling_mistral as mm
    model = _tiny("mistral")
    mgr = KO.KVOffloadManager(model, KO.KVOffloadConfig.from_model(model), batch_size=1)
    try:
        assert mgr._patched["mistral"][0] is mm.MistralAttention
        calls = _count_decodes(mgr.kvcms[0])
        _single_decode(model.model.layers[0].self_attn, model)
        assert len(calls) == 1
    finally:
        mgr.restore()


@needs_host_kernel
def test_patch_module_roots_rebinds_shadowed_attention_forward():
    torch.manual_seed(0)
    base = _tiny()
    shadow = copy.deepcopy(base)
    shadow_attn = shadow.model.layers[0].self_attn
    shadow_attn.forward = shadow_attn.forward             # an instance-level bound forward
    mgr = KO.KVOffloadManager(base, KO.KVOffloadConfig.from_model(base), batch_size=1)
    try:
        calls = _count_decodes(mgr.kvcms[0])
        _single_decode(shadow_attn, shadow)
        assert len(calls) == 0
        mgr.patch_module_roots(shadow)
        _single_decode(shadow_attn, shadow)
        assert len(calls) == 1
    finally:
        mgr.restore()


class _RecordingDecodeCache:
    """A duck-typed cache: append_decode / iterate_layer_pages /
    all_gpu_resident only, pages as plain namespaces."""
    use_contiguous = False

    def __init__(self):
        self.skip_residency_values = []
        self.pages = []

    def all_gpu_resident(self, layer_idx):
        return True

    def append_decode(self, layer_idx, k, v, skip_residency=False):
        self.skip_residency_values.append(skip_residency)
        self.pages.append(SimpleNamespace(used_tokens=1, k_tensor=k, v_tensor=v))

    def iterate_layer_pages(self, layer_idx):
        return list(self.pages)


@needs_host_kernel
def test_decode_batched_enforces_residency_even_when_pages_start_on_gpu():
    cache = _RecordingDecodeCache()
    q, k, v = (torch.randn(1, 1, 1, 4) for _ in range(3))
    out = KO._decode_batched([cache], q, k, v, layer_idx=0, scale=1.0)
    assert cache.skip_residency_values == [False]
    assert torch.allclose(out, v, atol=1e-6)              # one key: its value


def _padded_case():
    """Prompt of 3 real tokens + 2 pad tokens whose keys align with q (they
    would dominate an unmasked softmax) and whose values are far away."""
    torch.manual_seed(0)
    q = torch.randn(1, 1, 1, 4)
    real_k, real_v = torch.randn(1, 1, 3, 4), torch.randn(1, 1, 3, 4)
    pad_k, pad_v = q.expand(1, 1, 2, 4) * 50.0, torch.full((1, 1, 2, 4), 1000.0)
    k_dec, v_dec = torch.randn(1, 1, 1, 4), torch.randn(1, 1, 1, 4)
    a = KVAllocator(num_layers=1, num_kv_heads=1, head_dim=4, page_size=8, dtype=torch.float32)
    kvcm = KVCacheManager(a, gpu_high_watermark_bytes=0)
    kvcm.use_contiguous = False
    kvcm.append_prefill(0, torch.cat([real_k, pad_k], 2), torch.cat([real_v, pad_v], 2))
    mask = torch.zeros(1, 1, 1, 6)
    mask[..., 3:5] = float("-inf")
    expected = F.scaled_dot_product_attention(q, torch.cat([real_k, k_dec], 2),
                                              torch.cat([real_v, v_dec], 2), scale=1.0)
    return kvcm, q, k_dec, v_dec, mask, expected


@needs_host_kernel
def test_decode_batched_paged_path_masks_padded_prompt_tokens():
    kvcm, q, k, v, mask, expected = _padded_case()
    out = KO._decode_batched([kvcm], q, k, v, layer_idx=0, scale=1.0, attention_mask=mask)
    assert torch.allclose(out, expected, atol=1e-4)


@needs_host_kernel
def test_decode_batched_paged_path_without_mask_is_unaffected():
    kvcm, q, k, v, _, expected = _padded_case()
    out = KO._decode_batched([kvcm], q, k, v, layer_idx=0, scale=1.0)
    assert not torch.allclose(out, expected, atol=1e-4)


def test_config_from_model_contiguous_capacity():
    model = _tiny()
    assert KO.KVOffloadConfig.from_model(model).cont_capacity == 0
    assert KO.KVOffloadConfig.from_model(model, cont_capacity=128).cont_capacity == 128


class _PagedPrefillCache:
    use_contiguous = False

    def __init__(self):
        self.pages = []

    def append_prefill(self, layer_idx, k, v):
        start = sum(p.used_tokens for p in self.pages)
        self.pages.append(SimpleNamespace(used_tokens=k.shape[2], capacity_tokens=k.shape[2],
                                          start_token=start, k_tensor=k.clone(),
                                          v_tensor=v.clone(), device=k.device, state="CPU"))

    def iterate_layer_pages(self, layer_idx):
        return list(self.pages)


def _identity_attn(dim, head_dim):
    attn = nn.Module()
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        lin = nn.Linear(dim, dim, bias=False)
        with torch.no_grad():
            lin.weight.copy_(torch.eye(dim))
        setattr(attn, name, lin)
    attn.head_dim, attn.attention_dropout, attn.training, attn.layer_idx = head_dim, 0.0, False, 0
    return attn


def test_llama_prefill_with_past_streams_over_all_paged_kv(monkeypatch):
    """A second prompt chunk attends through perform_streaming_attention over
    every cached token (the first chunk's and its own), under the caller's
    mask; the first chunk attends locally."""
    import transformers.models.llama.modeling_llama as llama_modeling
    monkeypatch.setattr(llama_modeling, "apply_rotary_pos_emb", lambda q, k, cos, sin: (q, k))
    calls = []

    def fake(query, pages, scale=None, attention_mask=None, softcap=None):
        calls.append({"query_len": query.shape[2], "tokens": sum(p.used_tokens for p in pages),
                      "mask_shape": tuple(attention_mask.shape) if attention_mask is not None
                      else None})
        return torch.zeros_like(query)
    monkeypatch.setattr(KO, "perform_streaming_attention", fake)
    attn = _identity_attn(4, 2)
    cache = _PagedPrefillCache()
    forward = KO._make_llama_forward([cache])
    forward(attn, torch.randn(1, 2, 4), position_embeddings=(None, None),
            attention_mask=torch.zeros(1, 1, 2, 2), cache_position=torch.arange(2))
    assert calls == []
    forward(attn, torch.randn(1, 2, 4), position_embeddings=(None, None),
            attention_mask=torch.zeros(1, 1, 2, 4), cache_position=torch.arange(2, 4))
    assert calls == [{"query_len": 2, "tokens": 4, "mask_shape": (1, 1, 2, 4)}]


class _RecordingCache:
    def append_prefill(self, layer_idx, k, v):
        return None

    def append_decode(self, layer_idx, k, v):
        return None

    def iterate_layer_pages(self, layer_idx):
        return []


def test_gemma2_forward_enforces_sliding_window_mask(monkeypatch):
    """Window of 2: the third token sees the second and itself only — values
    1 and 2 with equal logits give 1.5 (HELM's known answer)."""
    import transformers.models.gemma2.modeling_gemma2 as gemma2_modeling
    monkeypatch.setattr(gemma2_modeling, "apply_rotary_pos_emb", lambda q, k, cos, sin: (q, k))
    attn = nn.Module()
    attn.q_proj = nn.Linear(3, 1, bias=False)
    attn.k_proj = nn.Linear(3, 1, bias=False)
    attn.v_proj = nn.Linear(3, 1, bias=False)
    attn.o_proj = nn.Linear(1, 1, bias=False)
    with torch.no_grad():
        attn.q_proj.weight.copy_(torch.tensor([[1.0, 0.0, 0.0]]))
        attn.k_proj.weight.copy_(torch.tensor([[0.0, 1.0, 0.0]]))
        attn.v_proj.weight.copy_(torch.tensor([[0.0, 0.0, 1.0]]))
        attn.o_proj.weight.fill_(1.0)
    attn.head_dim, attn.num_key_value_groups, attn.attention_dropout = 1, 1, 0.0
    attn.training, attn.layer_idx, attn.scaling = False, 0, 1.0
    attn.attn_logit_softcapping, attn.sliding_window = None, 2
    hidden = torch.tensor([[[1.0, 10.0, 100.0], [1.0, 0.0, 1.0], [1.0, 0.0, 2.0]]])
    causal = torch.triu(torch.full((3, 3), torch.finfo(torch.float32).min), diagonal=1)[None, None]
    out, _ = KO._make_gemma2_forward([_RecordingCache()])(
        attn, hidden, position_embeddings=(None, None), attention_mask=causal,
        cache_position=torch.arange(3))
    assert out[0, 2, 0].item() == pytest.approx(1.5, abs=1e-4)


@needs_host_kernel
@pytest.mark.parametrize("restore_first", [0, 1])
def test_managers_do_not_change_other_models_or_attention_class(restore_first):
    from transformers.models.llama.modeling_llama import LlamaAttention
    original = LlamaAttention.forward
    models = [_tiny() for _ in range(3)]
    managers = []
    try:
        for model in models[:2]:
            managers.append(KO.KVOffloadManager(model, KO.KVOffloadConfig.from_model(model)))
        assert LlamaAttention.forward is original
        assert models[2].model.layers[0].self_attn.forward.__func__ is original
        managers[restore_first].restore()
        other = 1 - restore_first
        _single_decode(models[other].model.layers[0].self_attn, models[other])
        assert managers[other].kvcms[0].seq_len() == 1
        assert LlamaAttention.forward is original
    finally:
        for m in managers:
            m.restore()
    assert all("forward" not in m.model.layers[0].self_attn.__dict__ for m in models)
