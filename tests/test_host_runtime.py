"""Host bookkeeping of helm_amd.runtime with host (CPU) pages — no GPU work.

Mirrors the CPU tests HELM holds for these classes
(tests/unit/runtime/test_kv_allocator.py, test_kv_cache.py,
test_batch_kv_offload.py) and cross-checks page metadata against the paging
model in oracle/paging.py.
"""
import numpy as np
import pytest
import torch

from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager, LayerKVCache
from helm_amd.runtime.kv_offload import KVOffloadConfig
from oracle.paging import AllocatorModel, CacheModel

CPU = torch.device("cpu")
NUM_HEADS, HEAD_DIM, PAGE_SIZE, NUM_LAYERS = 2, 8, 4, 4


@pytest.fixture()
def allocator():
    return KVAllocator(num_layers=NUM_LAYERS, num_kv_heads=NUM_HEADS, head_dim=HEAD_DIM,
                       page_size=PAGE_SIZE, dtype=torch.float32)


@pytest.fixture()
def cache(allocator):
    mgr = KVCacheManager(allocator, gpu_high_watermark_bytes=0)
    mgr.initialize_layer_caches(num_layers=NUM_LAYERS)
    return mgr


def _kv(n, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, NUM_HEADS, n, HEAD_DIM, generator=g),
            torch.randn(1, NUM_HEADS, n, HEAD_DIM, generator=g))


# ── allocator (test_kv_allocator.py) ──────────────────────────────────────────
def test_allocate_state_and_reserve(allocator):
    page = allocator.allocate(CPU)
    assert page.state == "CPU" and page.device.type == "cpu"
    assert allocator.cpu_total_pages == 16 and len(allocator.cpu_free_pool) == 15


def test_allocate_resets_metadata_and_lifo(allocator):
    p = allocator.allocate(CPU)
    p.layer_id, p.start_token, p.used_tokens = 99, 500, 3
    allocator.free(p)
    assert p.state == "FREE"
    p2 = allocator.allocate(CPU)
    assert p2 is p
    assert (p2.layer_id, p2.start_token, p2.used_tokens) == (-1, 0, 0)


def test_page_shape_dtype_and_ids():
    a = KVAllocator(num_layers=2, num_kv_heads=3, head_dim=16, page_size=8, dtype=torch.float16)
    p0, p1 = a.allocate(CPU), a.allocate(CPU)
    assert p0.k_tensor.shape == (1, 3, 8, 16) and p0.v_tensor.shape == (1, 3, 8, 16)
    assert p0.k_tensor.dtype == torch.float16
    assert p0.page_id != p1.page_id
    # K and V of a page are adjacent halves of one arena slot
    es = p0.k_tensor.element_size()
    assert p0.v_tensor.data_ptr() - p0.k_tensor.data_ptr() == 3 * 8 * 16 * es


def test_reserve_batch_accumulates(allocator):
    allocator.reserve_batch(3, CPU)
    allocator.reserve_batch(4, CPU)
    assert allocator.cpu_total_pages == 7 and len(allocator.cpu_free_pool) == 7


def test_move_page_same_device_and_data(allocator):
    page = allocator.allocate(CPU)
    page.used_tokens = 2
    page.k_tensor[:, :, :2, :] = 42.0
    page.v_tensor[:, :, :2, :] = 99.0
    res = allocator.move_page(page, CPU)
    assert res is page
    assert torch.all(res.k_tensor[:, :, :2, :] == 42.0)
    assert torch.all(res.v_tensor[:, :, :2, :] == 99.0)


def test_report_usage_matches_model(allocator):
    model = AllocatorModel(PAGE_SIZE, 2 * NUM_HEADS * PAGE_SIZE * HEAD_DIM * 4)
    for _ in range(5):
        allocator.allocate(CPU)
        model.allocate("cpu")
    assert allocator.report_usage() == model.report_usage()


# ── cache manager (test_kv_cache.py CPU part) ─────────────────────────────────
def test_layer_cache_tail(allocator):
    layer = LayerKVCache(0)
    p1, p2 = allocator.allocate(CPU), allocator.allocate(CPU)
    layer.append_page(p1)
    layer.append_page(p2)
    assert layer.tail_page is p2 and len(layer.pages) == 2


@pytest.mark.parametrize("n,pages", [(3, 1), (4, 1), (9, 3), (8, 2)])
def test_prefill_pages_and_start_tokens(cache, n, pages):
    k, v = _kv(n)
    cache.append_prefill(0, k, v)
    L = cache.layers[0]
    assert len(L.pages) == pages and L.total_tokens == n
    assert [p.start_token for p in L.pages] == list(range(0, n, PAGE_SIZE))
    got_k = torch.cat([p.k_tensor[:, :, :p.used_tokens] for p in L.pages], 2)
    got_v = torch.cat([p.v_tensor[:, :, :p.used_tokens] for p in L.pages], 2)
    assert torch.equal(got_k, k) and torch.equal(got_v, v)


def test_decode_tail_growth(cache):
    k, v = _kv(PAGE_SIZE)
    cache.append_prefill(0, k, v)
    kd, vd = _kv(1, seed=1)
    cache.append_decode(0, kd, vd)
    assert len(cache.layers[0].pages) == 2 and cache.layers[0].tail_page.used_tokens == 1
    assert torch.equal(cache.layers[0].tail_page.k_tensor[:, :, :1], kd)
    for i in range(PAGE_SIZE + 2):
        cache.append_decode(1, *_kv(1, seed=10 + i))
    assert len(cache.layers[1].pages) == 2 and cache.layers[1].total_tokens == PAGE_SIZE + 2
    assert cache.seq_len() == PAGE_SIZE + 1


def test_auto_create_layer_and_iterate(cache):
    del cache.layers[3]
    cache.append_prefill(3, *_kv(2))
    assert 3 in cache.layers
    assert isinstance(cache.iterate_layer_pages(3), list)
    assert cache.iterate_layer_pages(99) == []


def test_clear_returns_pages(cache):
    alloc = cache.allocator
    cache.append_prefill(0, *_kv(PAGE_SIZE))
    before = len(alloc.cpu_free_pool)
    cache.clear()
    assert len(alloc.cpu_free_pool) > before
    assert cache.num_layers() == 0 and cache.seq_len() == 0


def test_report_bytes_and_cpu_eviction_noop(cache):
    cache.append_prefill(0, *_kv(8))
    cache.evict_pages(99999)       # no GPU pages -> nothing moves
    r = cache.report_bytes_per_tier()
    assert r["gpu_active_bytes"] == 0
    assert r["cpu_active_bytes"] == 2 * 2 * NUM_HEADS * PAGE_SIZE * HEAD_DIM * 4


def test_metadata_matches_paging_model(allocator):
    mgr = KVCacheManager(allocator, gpu_high_watermark_bytes=0)
    model = CacheModel(AllocatorModel(PAGE_SIZE, 2 * NUM_HEADS * PAGE_SIZE * HEAD_DIM * 4), 0)
    ops = [("p", 0, 9), ("d", 0), ("d", 0), ("p", 1, 3), ("d", 1), ("d", 0), ("d", 0), ("d", 0)]
    for op in ops:
        if op[0] == "p":
            mgr.append_prefill(op[1], *_kv(op[2]))
            model.append_prefill(op[1], op[2], device="cpu")
        else:
            mgr.append_decode(op[1], *_kv(1))
            model.append_decode(op[1], device="cpu")
    for lid in (0, 1):
        got = [(p.page_id, p.start_token, p.used_tokens, p.state) for p in mgr.layers[lid].pages]
        ref = [(p.page_id, p.start_token, p.used_tokens, p.state) for p in model.layers[lid].pages]
        assert got == ref


def test_build_contiguous_small_capacities():
    for cap in (64, 640, 768, 2048):
        a = KVAllocator(num_layers=2, num_kv_heads=2, head_dim=8, page_size=4, dtype=torch.float32)
        m = KVCacheManager(a, gpu_high_watermark_bytes=0)
        assert m.build_contiguous(2, 2, 8, cap, CPU, torch.float32)
        assert m.use_contiguous and m.cont_capacity == cap
        assert m.cont_K[0].shape == (1, 2, cap, 8)


def test_build_contiguous_halves_on_oom(monkeypatch):
    # kv_cache.py:277-299: on allocation failure the capacity halves down to
    # a floor of min(capacity, 1024)
    real = KC.ContiguousKV._new_arena
    tried = []

    def flaky(shape, device, dtype):
        tried.append(shape[3])
        if shape[3] > 1024:
            raise RuntimeError("out of memory")
        return real(shape, device, dtype)

    a = KVAllocator(num_layers=1, num_kv_heads=2, head_dim=8, page_size=4, dtype=torch.float32)
    m = KVCacheManager(a)
    monkeypatch.setattr(KC.ContiguousKV, "_new_arena", staticmethod(flaky))
    assert m.build_contiguous(1, 2, 8, 4096, CPU, torch.float32)
    assert m.cont_capacity == 1024 and tried == [4096, 2048, 1024]
    assert m.cont_K[0].shape == (1, 2, 1024, 8) and m.cont_V[0].shape == (1, 2, 1024, 8)

    def oom(shape, device, dtype):
        raise RuntimeError("oom")
    monkeypatch.setattr(KC.ContiguousKV, "_new_arena", staticmethod(oom))
    assert not m.build_contiguous(1, 2, 8, 4096, CPU, torch.float32)
    assert not m.use_contiguous and m.cont_K == {}


def test_contiguous_buffers_and_migration_on_cpu():
    """prefill_contiguous / write_decode_contiguous / get_kv_contiguous /
    migrate_contiguous_to_pages (kv_cache.py:301-342): the buffers hold the
    prompt and the decoded tokens; migration appends only the decoded ones to
    the pages, after which pages hold every token and the buffers are gone."""
    a = KVAllocator(num_layers=2, num_kv_heads=2, head_dim=8, page_size=4, dtype=torch.float32)
    m = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 9)
    assert m.build_contiguous(2, 2, 8, 16, CPU, torch.float32)
    g = torch.Generator().manual_seed(3)
    K = torch.randn(1, 2, 13, 8, generator=g)
    V = torch.randn(1, 2, 13, 8, generator=g)
    for lid in range(2):
        m.append_prefill(lid, K[:, :, :10], V[:, :, :10])
        m.prefill_contiguous(lid, K[:, :, :10], V[:, :, :10])
    assert (m.cont_prefill_len, m.cont_seq_len) == (10, 10)
    for t in range(10, 13):
        for lid in range(2):
            m.write_decode_contiguous(lid, K[:, :, t:t + 1], V[:, :, t:t + 1])
            k, v = m.get_kv_contiguous(lid)
            assert torch.equal(k, K[:, :, :t + 1]) and torch.equal(v, V[:, :, :t + 1])
        m.advance_contiguous()
    m.migrate_contiguous_to_pages()
    assert not m.use_contiguous and m.cont_K == {}
    for lid in range(2):
        pages = m.layers[lid].pages
        assert [p.start_token for p in pages] == [0, 4, 8, 10]
        k = torch.cat([p.k_tensor[:, :, :p.used_tokens] for p in pages], 2)
        assert torch.equal(k, K)
    m.reset_contiguous()             # buffers dropped: stays off
    assert not m.use_contiguous


# ── counters (test_kv_cache.py:321-361) ───────────────────────────────────────
ZERO = {"evict_calls": 0, "pages_evicted": 0, "bytes_evicted": 0,
        "prefetch_calls": 0, "pages_prefetched": 0, "bytes_prefetched": 0}


def test_paging_counters():
    KC.reset_paging_stats()
    assert KC.get_paging_stats() == ZERO
    KC._record_eviction(2, 1000)
    KC._record_eviction(3, 1500)
    KC._record_prefetch(4, 4096)
    KC._record_eviction(0, 0)
    KC._record_prefetch(0, 0)
    s = KC.get_paging_stats()
    assert (s["evict_calls"], s["pages_evicted"], s["bytes_evicted"]) == (2, 5, 2500)
    assert (s["prefetch_calls"], s["pages_prefetched"], s["bytes_prefetched"]) == (1, 4, 4096)


def test_cpu_query_runs_the_host_kernel_without_a_torch_fallback(monkeypatch):
    """A CPU query attends on libhelm_cpu.so; when that library cannot be
    used the call raises instead of computing with torch."""
    from helm_amd import _cpu_native
    q = torch.randn(1, 2, 1, 8)
    page = KC.KVPage(0, 0, 0, 4, 4, torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8), CPU, "CPU")
    out = KC.perform_streaming_attention(q, [page])
    assert out.shape == q.shape and torch.isfinite(out).all()
    monkeypatch.setattr(_cpu_native, "_lib", None)
    monkeypatch.setattr(_cpu_native, "_error", "not built")
    with pytest.raises(RuntimeError, match="libhelm_cpu.so unavailable"):
        KC.perform_streaming_attention(q, [page])
    # no active pages -> zeros, as HELM
    assert torch.all(KC.perform_streaming_attention(q, []) == 0)


# ── batch managers (test_batch_kv_offload.py) ─────────────────────────────────
def test_batch_managers_independent(allocator):
    kvcms = [KVCacheManager(allocator, gpu_high_watermark_bytes=0) for _ in range(3)]
    kvcms[0].append_prefill(0, *_kv(4))
    kvcms[1].append_prefill(0, *_kv(8))
    assert 0 not in kvcms[2].layers
    assert kvcms[0].layers[0].total_tokens == 4 and kvcms[1].layers[0].total_tokens == 8
    kvcms[1].append_decode(0, *_kv(1))
    assert kvcms[1].layers[0].total_tokens == 9
    used = allocator.report_usage()["active_cpu_pages"]
    assert used > 0
    for m in kvcms:
        m.clear()
    assert allocator.report_usage()["active_cpu_pages"] == 0


def test_offload_config_defaults():
    cfg = KVOffloadConfig(num_layers=36, num_kv_heads=8, head_dim=128, dtype=torch.bfloat16)
    assert cfg.page_size == 64 and cfg.cont_capacity == 0
    assert cfg.gpu_watermark_bytes == 512 * 2 * 8 * 128 * 2 * 36


# ── residency bookkeeping at scale, on CPU ───────────────────────────────────
class _CpuBackedGpuAllocator(KVAllocator):
    """Hands the manager pages marked GPU-resident whose tensors live in CPU
    memory, so the residency and eviction bookkeeping runs without a GPU
    (evicted pages become real CPU pages)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self._moving = False

    def allocate(self, device):
        if self._moving:
            return super().allocate(device)
        page = super().allocate(CPU)
        page.device, page.state = torch.device("cuda", 0), "GPU"
        return page

    def move_pages(self, pages, target_device, sync=True):
        self._moving = True
        try:
            return super().move_pages(pages, target_device, sync)
        finally:
            self._moving = False


def _pos_kv(n, start, H, D):
    pos = torch.arange(start, start + n, dtype=torch.float32)
    k = pos.view(1, 1, n, 1).expand(1, H, n, D).contiguous()
    return k, -k


@pytest.mark.parametrize("seed,watermark_pages", [(0, 0), (1, 3), (2, 11), (3, 40)])
def test_eviction_order_matches_paging_model(seed, watermark_pages):
    """Oldest-first eviction across many layers, ties broken by layer then page
    order, equals the paging model's full rescan and stable sort
    (kv_cache.py:179-235) over a long random append sequence."""
    H, D, P, L = 2, 4, 4, 6
    page_bytes = 2 * H * P * D * 4
    wm = watermark_pages * page_bytes
    a = _CpuBackedGpuAllocator(L, H, D, page_size=P, dtype=torch.float32)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=wm)
    model = CacheModel(AllocatorModel(P, page_bytes), wm)
    KC.reset_paging_stats()
    rng = np.random.default_rng(seed)
    totals = [0] * L
    for _ in range(400):
        lid = int(rng.integers(0, L))
        if rng.random() < 0.2:
            n = int(rng.integers(1, 3 * P))
            mgr.append_prefill(lid, *_pos_kv(n, totals[lid], H, D))
            model.append_prefill(lid, n)
            totals[lid] += n
        else:
            mgr.append_decode(lid, *_pos_kv(1, totals[lid], H, D))
            model.append_decode(lid)
            totals[lid] += 1
    for lid in model.layers:
        got = [(p.start_token, p.used_tokens, p.state) for p in mgr.layers[lid].pages]
        ref = [(p.start_token, p.used_tokens, p.state) for p in model.layers[lid].pages]
        assert got == ref
        k = torch.cat([p.k_tensor[0, 0, :p.used_tokens, 0] for p in mgr.layers[lid].pages])
        assert torch.equal(k, torch.from_numpy(model.gathered(lid)).float())
    s = KC.get_paging_stats()
    assert (s["evict_calls"], s["pages_evicted"], s["bytes_evicted"]) == (
        model.stats["evict_calls"], model.stats["pages_evicted"], model.stats["bytes_evicted"])
    # the running total equals HELM's rescan of evictable bytes
    assert mgr._ev_bytes == page_bytes * len(mgr._evictable())


def test_layer_records_follow_pages():
    """Each layer's page records carry the pages' addresses, used counts and
    running token offsets through prefill, decode and eviction."""
    H, D, P = 2, 8, 4
    a = _CpuBackedGpuAllocator(2, H, D, page_size=P, dtype=torch.float16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=2 * (2 * H * P * D * 2))
    rng = np.random.default_rng(5)
    for _ in range(60):
        lid = int(rng.integers(0, 2))
        if rng.random() < 0.3:
            mgr.append_prefill(lid, *_kv(int(rng.integers(1, 10))))
        else:
            mgr.append_decode(lid, *_kv(1))
        for layer in mgr.layers.values():
            r = layer.records()
            pages = layer.pages
            assert r is not None and len(r) == len(pages)
            assert list(r["used"]) == [p.used_tokens for p in pages]
            assert list(r["tok_off"]) == list(np.cumsum([0] + [p.used_tokens for p in pages])[:-1])
            assert list(r["k"]) == [p.k_tensor.data_ptr() for p in pages]
            assert list(r["v"]) == [p.v_tensor.data_ptr() for p in pages]
            assert set(r["head_stride"]) == {P * D}
            assert layer._n_host == sum(p.state == "CPU" for p in pages)
            assert layer._host_bytes == sum(p.used_tokens * H * D * 2 * 2 for p in pages
                                            if p.state == "CPU")


def test_record_validation_mode(monkeypatch):
    """HELM_AMD_CHECK_RECORDS=1: records are validated against their pages
    whenever they are handed out (prefill, decode and eviction pass), and a
    record that no longer describes its page — wrong used count, token
    offset or address, or a page whose capacity reaches past its storage —
    raises RuntimeError naming the layer and page instead of reaching a
    kernel."""
    monkeypatch.setenv("HELM_AMD_CHECK_RECORDS", "1")
    H, D, P = 2, 8, 4
    a = _CpuBackedGpuAllocator(2, H, D, page_size=P, dtype=torch.float16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=2 * (2 * H * P * D * 2))
    rng = np.random.default_rng(9)
    for _ in range(40):
        lid = int(rng.integers(0, 2))
        if rng.random() < 0.3:
            mgr.append_prefill(lid, *_kv(int(rng.integers(1, 10))))
        else:
            mgr.append_decode(lid, *_kv(1))
        for layer in mgr.layers.values():
            assert layer.records() is not None        # validated, consistent
    layer = mgr.layers[0]
    assert len(layer.pages) >= 3
    for field, delta in (("used", -1), ("tok_off", 1), ("k", 64), ("head_stride", 1)):
        saved = int(layer._rec[field][1])
        layer._rec[field][1] = saved + delta
        with pytest.raises(RuntimeError, match=f"layer 0 page 1 .*{field}"):
            layer.records()
        layer._rec[field][1] = saved
    assert layer.records() is not None
    page = layer.pages[0]
    cap = page.capacity_tokens
    page.capacity_tokens = 10 ** 7     # past the end of the slot arena it lives in
    with pytest.raises(RuntimeError, match="outside its storage"):
        layer.records()
    page.capacity_tokens = cap
    monkeypatch.delenv("HELM_AMD_CHECK_RECORDS")
    layer._rec["used"][1] += 1
    assert layer.records() is not None                # not checked outside the mode


def test_external_layer_changes_rebuild_the_heap():
    H, D, P = 2, 4, 4
    a = _CpuBackedGpuAllocator(3, H, D, page_size=P, dtype=torch.float32)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 9)
    for lid in range(3):
        mgr.append_prefill(lid, *_pos_kv(3 * P, 0, H, D))
    assert mgr._ev_bytes == 6 * (2 * H * P * D * 4)
    del mgr.layers[1]
    mgr.append_decode(0, *_pos_kv(1, 3 * P, H, D))
    assert mgr._ev_bytes == (2 + 2) * (2 * H * P * D * 4) + (2 * H * P * D * 4)
    mgr.clear()
    assert mgr._ev_bytes == 0 and mgr._evq == []


def test_layer_page_list_link_follows_the_layer():
    """iterate_layer_pages returns a plain list (kv_cache.py:173-177) that stays
    linked to the layer's records only while it holds exactly the layer's
    pages: a token written into the tail keeps the link; a new page, an
    eviction, a clear or any in-place change of the list drops it."""
    H, D, P = 2, 4, 4
    page_bytes = 2 * H * P * D * 4
    a = _CpuBackedGpuAllocator(1, H, D, page_size=P, dtype=torch.float32)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 9)
    mgr.append_prefill(0, *_pos_kv(P + 2, 0, H, D))
    pages = mgr.iterate_layer_pages(0)
    assert isinstance(pages, list) and pages == mgr.layers[0].pages
    assert pages is not mgr.layers[0].pages
    layer = mgr.layers[0]
    assert pages._live_layer() is layer
    mgr.append_decode(0, *_pos_kv(1, P + 2, H, D))          # into the tail
    assert pages._live_layer() is layer and pages[-1].used_tokens == 3
    mgr.append_decode(0, *_pos_kv(1, P + 3, H, D))          # fills the tail
    assert pages._live_layer() is layer
    mgr.append_decode(0, *_pos_kv(1, P + 4, H, D))          # a new page
    assert pages._live_layer() is None and len(pages) == 2
    assert mgr.iterate_layer_pages(0)._live_layer() is layer
    for change in (lambda l: l.append(l[0]), lambda l: l.pop(), lambda l: l.reverse(),
                   lambda l: l.__setitem__(0, l[0]), lambda l: l.__delitem__(0),
                   lambda l: l.extend([]), lambda l: l.sort(key=lambda p: 0),
                   lambda l: l.insert(0, l[0]), lambda l: l.clear()):
        fresh = mgr.iterate_layer_pages(0)
        change(fresh)
        assert fresh._live_layer() is None
    fresh = mgr.iterate_layer_pages(0)
    fresh += []
    assert fresh._live_layer() is None
    assert type(mgr.iterate_layer_pages(0)[:1]) is list     # slices are plain lists
    # an eviction replaces a page object: older lists lose the link
    fresh = mgr.iterate_layer_pages(0)
    mgr.evict_pages(page_bytes)
    assert fresh[0].state == "DEAD" and fresh._live_layer() is None
    assert mgr.iterate_layer_pages(0)[0].state == "CPU"
    fresh = mgr.iterate_layer_pages(0)
    mgr.clear()
    assert fresh._live_layer() is None and mgr.iterate_layer_pages(0) == []


@pytest.mark.parametrize("mdtype", [torch.float32, torch.bfloat16, torch.float16])
def test_causal_mask_offset_recognises_only_exact_chunk_masks(mdtype):
    """HELM's chunk mask after `past` cached tokens (pipeline_runtime.py:94-113:
    key j visible to chunk row i iff j <= past + i, finfo.min elsewhere) is
    recognised with its offset; first chunks give 0; a diagonal off by one, a
    finite bias, a padded key, a mask narrower than the chunk and decode
    (one row) are not taken for causal; an in-place change is noticed."""
    from helm_amd.runtime.kv_offload import _causal_mask_offset
    neg = torch.finfo(mdtype).min

    def chunk_mask(past, S, shift=0):
        T = past + S
        allowed = torch.arange(T)[None, :] <= past + shift + torch.arange(S)[:, None]
        return torch.where(allowed, torch.zeros((), dtype=mdtype),
                           torch.full((), neg, dtype=mdtype))[None, None].contiguous()

    for past, S in [(0, 5), (0, 64), (3, 2), (1037, 300), (4096, 17)]:
        assert _causal_mask_offset(chunk_mask(past, S), S) == past
        assert _causal_mask_offset(chunk_mask(past, S).expand(3, 2, S, past + S), S) == past
    assert _causal_mask_offset(chunk_mask(10, 6, shift=1), 6) is None
    assert _causal_mask_offset(chunk_mask(10, 6, shift=-1), 6) is None
    m = chunk_mask(10, 6)
    m[0, 0, 2, 3] = -1.0                              # a finite bias on a visible key
    assert _causal_mask_offset(m, 6) is None
    m = chunk_mask(10, 6)
    m[0, 0, :, 0] = neg                               # key 0 padded away
    assert _causal_mask_offset(m, 6) is None
    assert _causal_mask_offset(torch.zeros(1, 1, 1, 40, dtype=mdtype), 1) is None
    assert _causal_mask_offset(torch.zeros(1, 1, 6, 4, dtype=mdtype), 6) is None
    assert _causal_mask_offset(chunk_mask(10, 6)[0], 6) is None      # not 4-D
    assert _causal_mask_offset(torch.zeros(1, 1, 6, 16, dtype=torch.bool), 6) is None
    m = chunk_mask(10, 6)
    assert _causal_mask_offset(m, 6) == 10
    m[0, 0, 5, 15] = neg                              # in place: the cached answer is dropped
    assert _causal_mask_offset(m, 6) is None


def test_causal_mask_offset_cache_follows_the_tensor_object():
    """The recognition is cached per mask object: a new mask whose memory and
    signature match a freed one's (address reuse, fresh version counter) is
    checked anew, and a view of a recognised mask is checked on its own."""
    from helm_amd.runtime import kv_offload as KO
    S, past = 8, 24
    T = past + S
    allowed = torch.arange(T)[None, :] <= past + torch.arange(S)[:, None]
    causal = torch.zeros(1, 1, S, T).masked_fill(~allowed, torch.finfo(torch.float32).min)
    assert KO._causal_mask_offset(causal, S) == past
    ptr = causal.data_ptr()
    buf = causal.view(-1)
    other = buf.view(1, 1, S, T)                   # same memory, shape and version
    assert KO._causal_mask_offset(other, S) == past
    del causal, other
    # the memory rewritten without a torch version bump, then a new tensor
    # over it: address, shape, strides, dtype and version (0) all equal the
    # freed mask's, as with a reused allocation
    arr = buf.numpy()
    arr[T - 1] = 0.0                               # row 0 sees the last key
    fresh = torch.from_numpy(arr).view(1, 1, S, T)
    assert fresh.data_ptr() == ptr and fresh._version == 0
    assert KO._causal_mask_offset(fresh, S) is None


def test_mask_fp32_converted_once_per_object_and_version():
    """A decode mask in the model's dtype is converted to fp32 once per mask
    object (HELM hands one mask to every layer of a step); an in-place change
    or a new object converts again, and a freed mask's entry goes away."""
    import gc
    from helm_amd.runtime import kv_cache as KC
    cpu = torch.device("cpu")
    m = torch.zeros(1, 1, 1, 40, dtype=torch.bfloat16)
    a = KC._mask_fp32(m, cpu)
    b = KC._mask_fp32(m, cpu)
    assert a is b and a.dtype == torch.float32 and torch.equal(a, m.float())
    m[..., 7] = -3.0                      # in place: version bump, converted anew
    c = KC._mask_fp32(m, cpu)
    assert c is not a and c[0, 0, 0, 7].item() == -3.0 and torch.equal(c, m.float())
    m2 = m.clone()                        # another object with equal values
    assert KC._mask_fp32(m2, cpu) is not c
    key = id(m)
    del m, a, b, c
    gc.collect()
    assert key not in KC._F32_MASKS
    saved = KC._F32_MASK_MAX_ELEMS, KC._F32_MASK_MAX_TOTAL
    KC._F32_MASKS.clear()
    try:
        KC._F32_MASK_MAX_ELEMS, KC._F32_MASK_MAX_TOTAL = 64, 100
        big = torch.zeros(1, 1, 1, 65, dtype=torch.float16)
        assert KC._mask_fp32(big, cpu) is not KC._mask_fp32(big, cpu)   # above one mask's cap
        keep = [torch.zeros(1, 1, 1, 40, dtype=torch.float16) for _ in range(3)]
        conv = [KC._mask_fp32(x, cpu) for x in keep]
        assert KC._mask_fp32(keep[0], cpu) is conv[0]        # 40 + 40 elements kept
        assert KC._mask_fp32(keep[1], cpu) is conv[1]
        assert KC._mask_fp32(keep[2], cpu) is not conv[2]    # past the total: per call
        assert torch.equal(KC._mask_fp32(keep[2], cpu), keep[2].float())
    finally:
        KC._F32_MASK_MAX_ELEMS, KC._F32_MASK_MAX_TOTAL = saved
        KC._F32_MASKS.clear()
