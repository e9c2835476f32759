"""Page append / evict / prefetch on the GPU: bit-exact data movement, HELM's
residency semantics (checked against oracle/paging.py), and attention over
mixed-residency pages (device + pinned host, staged through the copy ring)."""
import ctypes
import math

import numpy as np
import pytest
import torch

from helm_amd import _native
from helm_amd import workloads as W
from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager, perform_streaming_attention
from helm_amd.runtime.kv_offload import (KVOffloadConfig, KVOffloadManager, _decode_batched,
                                         _stream_prefill_batched)
from oracle import attention as A
from oracle.paging import AllocatorModel, CacheModel

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CPU = torch.device("cpu")


@pytest.fixture(params=["auto", "direct", "copy"])
def host_read(request, monkeypatch):
    """Host pages read in place by the kernel or staged through the device ring
    by hipMemcpyAsync: chosen per call (default), always in place when
    readable (HELM_AMD_HOST_READ=direct), always staged (=copy)."""
    if request.param == "auto":
        monkeypatch.delenv("HELM_AMD_HOST_READ", raising=False)
    else:
        monkeypatch.setenv("HELM_AMD_HOST_READ", request.param)
    return request.param


def _positional_kv(n, start, H=2, D=8, dtype=torch.float32, device=DEV):
    """K[h, t, d] = (start + t) * 1000 + h * 10 + d / 16 — every element names
    its token, head and dim exactly (bit-exact gather checks)."""
    t = torch.arange(start, start + n, dtype=torch.float64).view(1, 1, n, 1)
    h = torch.arange(H, dtype=torch.float64).view(1, H, 1, 1)
    d = torch.arange(D, dtype=torch.float64).view(1, 1, 1, D)
    k = (t * 1000 + h * 10 + d / 16).to(dtype)
    return k.to(device), (-k).to(device)


def _gather(mgr, lid):
    pages = [p for p in mgr.layers[lid].pages if p.used_tokens > 0 and p.state != "DEAD"]
    k = torch.cat([p.k_tensor[:, :, :p.used_tokens].to(CPU) for p in pages], 2)
    v = torch.cat([p.v_tensor[:, :, :p.used_tokens].to(CPU) for p in pages], 2)
    return k, v


def test_append_prefill_decode_bit_exact():
    a = KVAllocator(2, 8, 128, page_size=16, dtype=torch.bfloat16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator(device=DEV).manual_seed(0)
    # non-contiguous source like the projection output (transpose of [1,S,H,D])
    src = torch.randn(1, 37, 8, 128, generator=g, device=DEV).bfloat16()
    kp, vp = src.transpose(1, 2), (src * 2).transpose(1, 2)
    mgr.append_prefill(0, kp, vp)
    toks_k, toks_v = [kp.cpu()], [vp.cpu()]
    for i in range(20):
        kd = torch.randn(1, 8, 1, 128, generator=g, device=DEV).bfloat16()
        vd = torch.randn(1, 8, 1, 128, generator=g, device=DEV).bfloat16()
        mgr.append_decode(0, kd, vd)
        toks_k.append(kd.cpu())
        toks_v.append(vd.cpu())
    torch.cuda.synchronize()
    k, v = _gather(mgr, 0)
    assert torch.equal(k, torch.cat(toks_k, 2)) and torch.equal(v, torch.cat(toks_v, 2))
    L = mgr.layers[0]
    assert [p.start_token for p in L.pages] == [0, 16, 32, 48]
    # 37 prefill tokens -> pages of 16, 16, 5; 20 decode tokens fill the tail
    # page to 16 and open a fourth page holding 9
    assert [p.used_tokens for p in L.pages] == [16, 16, 16, 9]
    assert L.total_tokens == 57


def test_evict_round_trip_bit_exact_and_tail_protected():
    """test_kv_cache.py:260-311 on pooled pages."""
    a = KVAllocator(num_layers=2, num_kv_heads=2, head_dim=8, page_size=4, dtype=torch.float32)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    mgr.initialize_layer_caches(2)
    k, v = _positional_kv(10, 0)
    mgr.append_prefill(0, k, v)
    tail = mgr.layers[0].tail_page
    KC.reset_paging_stats()
    mgr.evict_pages(999999)
    s = KC.get_paging_stats()
    assert s["evict_calls"] == 1 and s["pages_evicted"] == 2
    assert s["bytes_evicted"] == 2 * 2 * 2 * 4 * 8 * 4
    assert tail is mgr.layers[0].tail_page and tail.state == "GPU"
    assert [p.state for p in mgr.layers[0].pages] == ["CPU", "CPU", "GPU"]
    assert all(p.k_tensor.is_pinned() for p in mgr.layers[0].pages[:2])
    gk, gv = _gather(mgr, 0)
    assert torch.equal(gk, k.cpu()) and torch.equal(gv, v.cpu())


def test_move_page_cpu_to_gpu_and_back():
    """test_kv_allocator.py:175-220 KATs (7.0 / 8.0) plus the DEAD transition."""
    a = KVAllocator(num_layers=2, num_kv_heads=2, head_dim=8, page_size=4, dtype=torch.float32)
    page = a.allocate(CPU)
    page.layer_id, page.start_token, page.used_tokens = 2, 8, 3
    page.k_tensor[:, :, :3, :] = 7.0
    page.v_tensor[:, :, :3, :] = 8.0
    free_before = len(a.cpu_free_pool)
    new = a.move_page(page, DEV)
    assert len(a.cpu_free_pool) == free_before + 1
    assert new.device.type == "cuda" and (new.layer_id, new.start_token, new.used_tokens) == (2, 8, 3)
    assert torch.all(new.k_tensor[:, :, :3].cpu() == 7.0) and torch.all(new.v_tensor[:, :, :3].cpu() == 8.0)
    gpu_before = a.gpu_total_pages
    back = a.move_page(new, CPU)
    assert new.state == "DEAD" and new.k_tensor.numel() == 0 and a.gpu_total_pages == gpu_before - 1
    assert torch.all(back.k_tensor[:, :, :3] == 7.0)
    empty = a.allocate(CPU)
    moved = a.move_page(empty, DEV)
    assert moved.used_tokens == 0 and moved.device.type == "cuda"


def test_copy_stream_memoized():
    s1 = KC._get_kv_copy_stream(DEV)
    s2 = KC._get_kv_copy_stream(DEV)
    assert s1 is s2 and s1.device == DEV


@pytest.mark.parametrize("watermark_pages", [0, 1, 3])
def test_residency_matches_paging_model(watermark_pages):
    """A mixed prefill/decode run over 3 layers with a small watermark:
    page ids, start tokens, fill, states, eviction counters and every byte
    of every page agree with the paging model."""
    H, D, P = 2, 8, 4
    page_bytes = 2 * H * P * D * 4
    wm = watermark_pages * page_bytes
    a = KVAllocator(3, H, D, page_size=P, dtype=torch.float32)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=wm)
    model = CacheModel(AllocatorModel(P, page_bytes), wm)
    KC.reset_paging_stats()
    rng = np.random.default_rng(watermark_pages)
    totals = [0, 0, 0]
    for step in range(40):
        lid = int(rng.integers(0, 3))
        if rng.random() < 0.25:
            n = int(rng.integers(1, 11))
            mgr.append_prefill(lid, *_positional_kv(n, totals[lid], H, D))
            model.append_prefill(lid, n)
            totals[lid] += n
        else:
            mgr.append_decode(lid, *_positional_kv(1, totals[lid], H, D))
            model.append_decode(lid)
            totals[lid] += 1
    torch.cuda.synchronize()
    for lid in range(3):
        if lid not in model.layers:
            continue
        got = [(p.page_id, p.start_token, p.used_tokens, p.state) for p in mgr.layers[lid].pages]
        ref = [(p.page_id, p.start_token, p.used_tokens, p.state) for p in model.layers[lid].pages]
        assert got == ref
        k, v = _gather(mgr, lid)
        pos = torch.from_numpy(model.gathered(lid))
        ek, ev = _positional_kv(len(pos), 0, H, D, device=CPU)
        assert torch.equal(k, ek[:, :, pos]) and torch.equal(v, ev[:, :, pos])
    s = KC.get_paging_stats()
    assert (s["evict_calls"], s["pages_evicted"], s["bytes_evicted"]) == (
        model.stats["evict_calls"], model.stats["pages_evicted"], model.stats["bytes_evicted"])
    assert a.report_usage() == model.alloc.report_usage()


@pytest.mark.parametrize("dtype,H,kvh", [(torch.bfloat16, 32, 8), (torch.float16, 40, 40),
                                        (torch.float32, 4, 2)])
def test_mixed_residency_attention(dtype, H, kvh, host_read):
    """Attention after evicting the oldest pages equals the fp64 oracle over
    the same tokens; the prefetch counters record the host pages."""
    D, P, T = 128, 16, 700
    a = KVAllocator(1, kvh, D, page_size=P, dtype=dtype)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator(device=DEV).manual_seed(1)
    k = torch.randn(1, kvh, T, D, generator=g, device=DEV).to(dtype)
    v = torch.randn(1, kvh, T, D, generator=g, device=DEV).to(dtype)
    mgr.append_prefill(0, k, v)
    q = torch.randn(1, H, 1, D, generator=g, device=DEV).to(dtype)
    full = perform_streaming_attention(q, mgr.iterate_layer_pages(0))
    page_bytes = 2 * kvh * P * D * k.element_size()
    mgr.evict_pages(20 * page_bytes)
    pages = mgr.iterate_layer_pages(0)
    n_cpu = sum(p.state == "CPU" for p in pages)
    assert n_cpu == 20
    KC.reset_paging_stats()
    mask = torch.zeros(1, 1, 1, T, device=DEV)
    mixed = perform_streaming_attention(q, pages, attention_mask=mask)
    unmasked = perform_streaming_attention(q, pages)
    s = KC.get_paging_stats()
    assert s["prefetch_calls"] == 2 and s["pages_prefetched"] == 40
    per_call = 20 * kvh * P * D * k.element_size() * 2      # K + V of 20 full pages
    assert s["bytes_prefetched"] == 2 * per_call
    ref = A.attention_fp64_batched(q[0].cpu(), k[0].cpu(), v[0].cpu())
    tol = {torch.bfloat16: 1e-2, torch.float16: 2e-3, torch.float32: 1e-5}[dtype]
    for out in (full, mixed, unmasked):
        assert (out[0].double().cpu() - ref).abs().max().item() <= tol


def _ring_engine(chunk, slots):
    lib = _native.load()
    h = ctypes.c_void_p()
    _native.call("helm_engine_create", 0, chunk, slots, ctypes.byref(h))
    return lib, h


@pytest.fixture(params=["side", "one"])
def stage_stream(request, monkeypatch):
    """Staging copies on the engine's side stream joined by events
    (HELM_AMD_STAGE_STREAM=side), or queued on the caller's stream (=one,
    the same as the default)."""
    monkeypatch.setenv("HELM_AMD_STAGE_STREAM", request.param)
    return request.param


_RING_OUTS = {}


def test_staging_ring_reuse_many_chunks(host_read, stage_stream):
    """More staged chunks than ring slots: every slot is reused several times
    in one call and across calls; results stay exact to the oracle, and the
    side-stream copies give the same bits as copies on the caller's stream."""
    w = W.Workload("t", 1, 32, 8, 128, torch.bfloat16, T=4096)
    n_pages = 256
    pool_h = torch.randn(n_pages, 2, 8, 16, 128, generator=torch.Generator().manual_seed(2)
                         ).bfloat16().pin_memory()
    g = torch.Generator().manual_seed(3)
    dev_pool = torch.randn(64, 2, 8, 16, 128, generator=g).bfloat16().to(DEV)
    q = torch.randn(1, 32, 1, 128, generator=g).bfloat16().to(DEV)
    es = 2
    slot_b = 2 * 8 * 16 * 128 * es
    pages = np.zeros(n_pages + 64, dtype=_native.PAGE_DTYPE)
    order = np.random.default_rng(0).permutation(n_pages + 64)  # token order mixes tiers
    for j, idx in enumerate(order):
        if idx < n_pages:
            base = pool_h.data_ptr() + int(idx) * slot_b
            pages[j] = (base, base + slot_b // 2, 16, 16 * j, 16 * 128, _native.HELM_PAGE_HOST)
        else:
            base = dev_pool.data_ptr() + int(idx - n_pages) * slot_b
            pages[j] = (base, base + slot_b // 2, 16, 16 * j, 16 * 128, 0)
    seq_off = np.array([0, len(pages)], dtype=np.int32)
    lib, eng = _ring_engine(1 << 20, 2)          # 1 MiB chunks (16 pages), 2 slots
    try:
        outs = []
        for _ in range(3):
            out = torch.empty_like(q)
            _native.call("helm_stream_attn", eng, q.data_ptr(), out.data_ptr(), 1, 32, 8, 1, 128,
                         _native.ptr(pages), _native.ptr(seq_off), 1 / math.sqrt(128), 0.0, None,
                         0, 0, 0, _native.HELM_F32, 0, _native.HELM_BF16, _native.HELM_BF16,
                         torch.cuda.current_stream().cuda_stream)
            outs.append(out)
        torch.cuda.synchronize()
    finally:
        lib.helm_engine_destroy(eng)
    K = torch.empty(8, 16 * len(pages), 128)
    V = torch.empty(8, 16 * len(pages), 128)
    for j, idx in enumerate(order):
        src = pool_h[idx] if idx < n_pages else dev_pool[idx - n_pages].cpu()
        K[:, 16 * j:16 * j + 16] = src[0].float()
        V[:, 16 * j:16 * j + 16] = src[1].float()
    ref = A.attention_fp64_batched(q[0].cpu(), K, V)
    for out in outs:
        assert (out[0].double().cpu() - ref).abs().max().item() <= 1e-2
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    # the same seeded inputs under the other stream mode give the same bits
    other = _RING_OUTS.get((host_read, "one" if stage_stream == "side" else "side"))
    if other is not None:
        assert torch.equal(other, outs[0].cpu())
    _RING_OUTS[(host_read, stage_stream)] = outs[0].cpu()


@pytest.mark.parametrize("writer", ["evict", "torch"])
@pytest.mark.parametrize("chunk_mb,slots", [(1, 2), (64, 2)])
def test_staged_copies_follow_callers_host_writes(stage_stream, chunk_mb, slots, writer,
                                                  monkeypatch):
    """Host pages rewritten on the caller's stream just before the call (a
    device-to-host copy queued behind a long matmul) are staged with their new
    contents.  Written by the engine's helm_evict_pages, as the runtime
    evicts, the side stream's copies wait for that eviction's event (and for
    the launches that last read their ring slots, here those of the call
    before); written by a torch copy on an engine that has never evicted,
    they wait for all of the caller's earlier work.  Two calls in a row with
    different contents."""
    monkeypatch.setenv("HELM_AMD_HOST_READ", "copy")
    g = torch.Generator().manual_seed(41)
    n_host, n_dev = 96, 32
    host = torch.randn(n_host, 2, 8, 16, 128, generator=g).bfloat16().pin_memory()
    dev_pool = torch.randn(n_dev, 2, 8, 16, 128, generator=g).bfloat16().to(DEV)
    q = torch.randn(1, 32, 1, 128, generator=g).bfloat16().to(DEV)
    slot_b = 2 * 8 * 16 * 128 * 2
    pages = np.zeros(n_host + n_dev, dtype=_native.PAGE_DTYPE)
    for j in range(n_host + n_dev):
        if j < n_host:
            base, flags = host.data_ptr() + j * slot_b, _native.HELM_PAGE_HOST
        else:
            base, flags = dev_pool.data_ptr() + (j - n_host) * slot_b, 0
        pages[j] = (base, base + slot_b // 2, 16, 16 * j, 16 * 128, flags)
    seq_off = np.array([0, len(pages)], dtype=np.int32)
    lib, eng = _ring_engine(chunk_mb << 20, slots)
    a = torch.randn(4096, 4096, device=DEV)
    outs, contents = [], []
    try:
        for call in range(2):
            new = torch.randn(n_host, 2, 8, 16, 128, generator=g).bfloat16().to(DEV)
            torch.cuda.synchronize()
            for _ in range(8):            # keep the caller's stream busy for a while
                a = (a @ a).clamp_(-1, 1)
            if writer == "torch":
                host.copy_(new, non_blocking=True)   # D2H behind the matmuls
            else:
                reg = [np.array([x], dtype=np.uint64) for x in
                       (new.data_ptr(), host.data_ptr(), new.numel() * new.element_size())]
                _native.call("helm_evict_pages", eng, 1, _native.ptr(reg[0]),
                             _native.ptr(reg[1]), _native.ptr(reg[2]), 0,
                             torch.cuda.current_stream().cuda_stream)
            out = torch.empty_like(q)
            _native.call("helm_stream_attn", eng, q.data_ptr(), out.data_ptr(), 1, 32, 8, 1, 128,
                         _native.ptr(pages), _native.ptr(seq_off), 1 / math.sqrt(128), 0.0,
                         None, 0, 0, 0, _native.HELM_F32, 0, _native.HELM_BF16, _native.HELM_BF16,
                         torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            outs.append(out.cpu())
            contents.append(new.cpu())
    finally:
        lib.helm_engine_destroy(eng)
    for out, new in zip(outs, contents):
        allp = torch.cat([new, dev_pool.cpu()])
        K = allp[:, 0].permute(1, 0, 2, 3).reshape(8, -1, 128).float()
        V = allp[:, 1].permute(1, 0, 2, 3).reshape(8, -1, 128).float()
        ref = A.attention_fp64_batched(q[0].cpu(), K, V)
        assert (out[0].double() - ref).abs().max().item() <= 1e-2


_QUEUED_ONE = {}


@pytest.mark.parametrize("ahead", ["0", "1", "2", "4"])
def test_side_stream_calls_queued_back_to_back(ahead, monkeypatch):
    """Six calls queued without a host wait, the host pages rewritten by
    helm_evict_pages on the caller's stream before each (1 MiB chunks, two
    ring slots: every slot is reused within a call and across calls).  With
    the copies on the side stream, whatever bound HELM_AMD_SIDE_AHEAD puts on
    how far the host runs ahead (0 = none), every call gives the bits of the
    same call with its copies on the caller's stream, and those equal the
    oracle."""
    monkeypatch.setenv("HELM_AMD_HOST_READ", "copy")
    g = torch.Generator().manual_seed(43)
    n_host, n_dev, calls = 96, 32, 6
    host = torch.zeros(n_host, 2, 8, 16, 128, dtype=torch.bfloat16).pin_memory()
    dev_pool = torch.randn(n_dev, 2, 8, 16, 128, generator=g).bfloat16().to(DEV)
    q = torch.randn(1, 32, 1, 128, generator=g).bfloat16().to(DEV)
    news = [torch.randn(n_host, 2, 8, 16, 128, generator=g).bfloat16().to(DEV)
            for _ in range(calls)]
    slot_b = 2 * 8 * 16 * 128 * 2
    pages = np.zeros(n_host + n_dev, dtype=_native.PAGE_DTYPE)
    for j in range(n_host + n_dev):
        if j < n_host:
            base, flags = host.data_ptr() + j * slot_b, _native.HELM_PAGE_HOST
        else:
            base, flags = dev_pool.data_ptr() + (j - n_host) * slot_b, 0
        pages[j] = (base, base + slot_b // 2, 16, 16 * j, 16 * 128, flags)
    seq_off = np.array([0, len(pages)], dtype=np.int32)
    stream = torch.cuda.current_stream().cuda_stream
    reg_dst = np.array([host.data_ptr()], dtype=np.uint64)
    reg_n = np.array([news[0].numel() * news[0].element_size()], dtype=np.uint64)

    def run(mode):
        monkeypatch.setenv("HELM_AMD_STAGE_STREAM", mode)
        monkeypatch.setenv("HELM_AMD_SIDE_AHEAD", ahead)
        lib, eng = _ring_engine(1 << 20, 2)
        outs = []
        try:
            torch.cuda.synchronize()
            for new in news:
                src = np.array([new.data_ptr()], dtype=np.uint64)
                _native.call("helm_evict_pages", eng, 1, _native.ptr(src), _native.ptr(reg_dst),
                             _native.ptr(reg_n), 0, stream)
                out = torch.empty_like(q)
                _native.call("helm_stream_attn", eng, q.data_ptr(), out.data_ptr(), 1, 32, 8, 1,
                             128, _native.ptr(pages), _native.ptr(seq_off), 1 / math.sqrt(128),
                             0.0, None, 0, 0, 0, _native.HELM_F32, 0, _native.HELM_BF16,
                             _native.HELM_BF16, stream)
                outs.append(out)
            torch.cuda.synchronize()
        finally:
            lib.helm_engine_destroy(eng)
        return [o.cpu() for o in outs]

    if "one" not in _QUEUED_ONE:
        one = run("one")
        for out, new in zip(one, news):
            allp = torch.cat([new.cpu(), dev_pool.cpu()])
            K = allp[:, 0].permute(1, 0, 2, 3).reshape(8, -1, 128).float()
            V = allp[:, 1].permute(1, 0, 2, 3).reshape(8, -1, 128).float()
            ref = A.attention_fp64_batched(q[0].cpu(), K, V)
            assert (out[0].double() - ref).abs().max().item() <= 1e-2
        _QUEUED_ONE["one"] = one
    side = run("side")
    for a, b in zip(side, _QUEUED_ONE["one"]):
        assert torch.equal(a, b)


def _kv_records(parts, Hkv, D, P):
    """helm_page records over [(slots tensor, slot index, host flag)], in order."""
    slot_b = 2 * Hkv * P * D * 2
    rec = np.zeros(len(parts), dtype=_native.PAGE_DTYPE)
    for j, (t, i, host) in enumerate(parts):
        base = t.data_ptr() + i * slot_b
        rec[j] = (base, base + slot_b // 2, P, P * j, P * D, _native.HELM_PAGE_HOST if host else 0)
    return rec


def test_host_pages_in_place_and_mixed_host_memory(host_read):
    """Pinned host pages are read in place, pageable ones staged: the in-place
    query says which; a call mixing device, pinned and pageable pages equals
    the oracle; a batched call is refused only when a page must be staged."""
    from helm_amd.runtime import engine
    Hkv, D, P, Hq = 8, 128, 16, 32
    g = torch.Generator().manual_seed(4)
    pinned = torch.randn(8, 2, Hkv, P, D, generator=g).bfloat16().pin_memory()
    pageable = torch.randn(8, 2, Hkv, P, D, generator=g).bfloat16()
    devp = torch.randn(8, 2, Hkv, P, D, generator=g).bfloat16().to(DEV)
    parts = []
    for i in range(8):
        parts += [(pinned, i, True), (devp, i, False), (pageable, i, True)]
    rec = _kv_records(parts, Hkv, D, P)
    eng = engine.get_engine(DEV)
    flags = np.zeros(len(rec), dtype=np.uint8)
    _native.call("helm_host_pages_in_place", eng, _native.ptr(rec), len(rec), Hkv, D,
                 _native.HELM_BF16, _native.ptr(flags))
    want = [1 if (t is pinned and host_read != "copy") else 0 for t, _, _ in parts]
    assert flags.tolist() == want
    q = torch.randn(2, Hq, 1, D, generator=g).bfloat16()
    K = torch.cat([t[i, 0].cpu().float() for t, i, _ in parts], 1)
    V = torch.cat([t[i, 1].cpu().float() for t, i, _ in parts], 1)
    ref = A.attention_fp64_batched(q[0].float(), K, V)
    stream = torch.cuda.current_stream().cuda_stream

    def call(recs, qd):
        B = qd.size(0)
        arr = np.concatenate(recs)
        off = np.cumsum([0] + [len(r) for r in recs]).astype(np.int32)
        out = torch.empty_like(qd)
        _native.call("helm_stream_attn", eng, qd.data_ptr(), out.data_ptr(), B, Hq, Hkv, 1, D,
                     _native.ptr(arr), _native.ptr(off), 1 / math.sqrt(D), 0.0, None, 0, 0, 0,
                     _native.HELM_F32, 0, _native.HELM_BF16, _native.HELM_BF16, stream)
        return out

    qd = q.to(DEV)
    out = call([rec], qd[:1])
    assert (out[0].double().cpu() - ref).abs().max().item() <= 1e-2
    with pytest.raises(NotImplementedError):
        call([rec, rec], qd)
    pin_only = _kv_records([p for p in parts if p[0] is not pageable], Hkv, D, P)
    K2 = torch.cat([t[i, 0].cpu().float() for t, i, _ in parts if t is not pageable], 1)
    V2 = torch.cat([t[i, 1].cpu().float() for t, i, _ in parts if t is not pageable], 1)
    if host_read != "copy":
        out = call([pin_only, pin_only], qd)
        for b in range(2):
            ref2 = A.attention_fp64_batched(q[b].float(), K2, V2)
            assert (out[b].double().cpu() - ref2).abs().max().item() <= 1e-2
    else:
        with pytest.raises(NotImplementedError):
            call([pin_only, pin_only], qd)
    torch.cuda.synchronize()


def test_large_contiguous_host_runs(host_read):
    """64 MiB of host pages in one address run (staged by default, in place
    with HELM_AMD_HOST_READ=direct) behind scattered device pages: both
    equal the oracle."""
    from helm_amd.runtime import engine
    Hkv, D, P, Hq, n = 8, 128, 16, 32, 1024
    g = torch.Generator().manual_seed(8)
    host = torch.randn(n, 2, Hkv, P, D, generator=g).bfloat16().pin_memory()
    devp = torch.randn(256, 2, Hkv, P, D, generator=g).bfloat16().to(DEV)
    perm = torch.randperm(256, generator=g).tolist()
    parts = [(host, i, True) for i in range(n)] + [(devp, i, False) for i in perm]
    rec = _kv_records(parts, Hkv, D, P)
    q = torch.randn(1, Hq, 1, D, generator=g).bfloat16()
    out = torch.empty(1, Hq, 1, D, dtype=torch.bfloat16, device=DEV)
    qd = q.to(DEV)
    off = np.array([0, len(rec)], dtype=np.int32)
    _native.call("helm_stream_attn", engine.get_engine(DEV), qd.data_ptr(), out.data_ptr(), 1,
                 Hq, Hkv, 1, D, _native.ptr(rec), _native.ptr(off), 1 / math.sqrt(D), 0.0, None,
                 0, 0, 0, _native.HELM_F32, 0, _native.HELM_BF16, _native.HELM_BF16,
                 torch.cuda.current_stream().cuda_stream)
    K = torch.cat([host[:, 0].permute(1, 0, 2, 3).reshape(Hkv, -1, D).float(),
                   devp[perm, 0].permute(1, 0, 2, 3).reshape(Hkv, -1, D).cpu().float()], 1)
    V = torch.cat([host[:, 1].permute(1, 0, 2, 3).reshape(Hkv, -1, D).float(),
                   devp[perm, 1].permute(1, 0, 2, 3).reshape(Hkv, -1, D).cpu().float()], 1)
    ref = A.attention_fp64_batched(q[0].float(), K, V)
    assert (out[0].double().cpu() - ref).abs().max().item() <= 1e-2


def test_in_place_query_forgets_freed_pinned_memory():
    """A pinned allocation that was released is no longer reported readable
    in place (the engine re-checks cached allocations on every call); no
    kernel runs on the released memory."""
    from helm_amd.runtime import engine
    if not hasattr(torch._C, "_host_emptyCache"):
        pytest.skip("torch cannot release cached pinned memory")
    Hkv, D, P = 2, 128, 16
    eng = engine.get_engine(DEV)
    t = torch.zeros(4, 2, Hkv, P, D, dtype=torch.bfloat16).pin_memory()
    rec = _kv_records([(t, i, True) for i in range(4)], Hkv, D, P)
    flags = np.zeros(4, dtype=np.uint8)
    _native.call("helm_host_pages_in_place", eng, _native.ptr(rec), 4, Hkv, D,
                 _native.HELM_BF16, _native.ptr(flags))
    assert flags.tolist() == [1, 1, 1, 1]
    del t
    torch.cuda.synchronize()
    torch._C._host_emptyCache()
    _native.call("helm_host_pages_in_place", eng, _native.ptr(rec), 4, Hkv, D,
                 _native.HELM_BF16, _native.ptr(flags))
    assert flags.tolist() == [0, 0, 0, 0]


def test_decode_batched_poison_pad_on_gpu():
    """test_kv_offload.py:168-245 on the GPU path."""
    torch.manual_seed(0)
    q = torch.randn(1, 1, 1, 4)
    real_k, real_v = torch.randn(1, 1, 3, 4), torch.randn(1, 1, 3, 4)
    pad_k = q.expand(1, 1, 2, 4) * 50.0
    pad_v = torch.full((1, 1, 2, 4), 1000.0)
    k_dec, v_dec = torch.randn(1, 1, 1, 4), torch.randn(1, 1, 1, 4)
    a = KVAllocator(1, 1, 4, page_size=8, dtype=torch.float32)
    for masked in (True, False):
        kvcm = KVCacheManager(a, gpu_high_watermark_bytes=0)
        kvcm.append_prefill(0, torch.cat([real_k, pad_k], 2).to(DEV),
                            torch.cat([real_v, pad_v], 2).to(DEV))
        mask = torch.zeros(1, 1, 1, 6)
        mask[..., 3:5] = float("-inf")
        out = _decode_batched([kvcm], q.to(DEV), k_dec.to(DEV), v_dec.to(DEV), 0, 1.0,
                              attention_mask=mask.to(DEV) if masked else None)
        exp = torch.nn.functional.scaled_dot_product_attention(
            q, torch.cat([real_k, k_dec], 2), torch.cat([real_v, v_dec], 2), scale=1.0)
        close = torch.allclose(out.cpu(), exp, atol=1e-4)
        assert close if masked else not close
        kvcm.clear()


def test_decode_batched_ragged_batch_and_offload(host_read):
    """Batched decode over per-item managers with ragged lengths (one kernel
    call) and with evicted pages (per-item streaming) agree with the oracle."""
    H, kvh, D = 8, 2, 64
    a = KVAllocator(1, kvh, D, page_size=16, dtype=torch.float16)
    g = torch.Generator().manual_seed(3)
    lens = [40, 75, 16]
    for evict in (False, True):
        kvcms = [KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12) for _ in lens]
        ks, vs = [], []
        for m, n in zip(kvcms, lens):
            k = torch.randn(1, kvh, n, D, generator=g).half()
            v = torch.randn(1, kvh, n, D, generator=g).half()
            m.append_prefill(0, k.to(DEV), v.to(DEV))
            ks.append(k)
            vs.append(v)
            if evict:
                m.evict_pages(10 ** 9)
        q = torch.randn(3, H, 1, D, generator=g).half()
        kd = torch.randn(3, kvh, 1, D, generator=g).half()
        vd = torch.randn(3, kvh, 1, D, generator=g).half()
        out = _decode_batched(kvcms, q.to(DEV), kd.to(DEV), vd.to(DEV), 0, 1 / math.sqrt(D))
        for i in range(3):
            K = torch.cat([ks[i], kd[i:i + 1]], 2)[0].float()
            V = torch.cat([vs[i], vd[i:i + 1]], 2)[0].float()
            ref = A.attention_fp64_batched(q[i].float(), K, V)
            assert (out[i].double().cpu() - ref).abs().max().item() <= 2e-3
        for m in kvcms:
            m.clear()


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("evict", [True, False])
@pytest.mark.parametrize("kernel", ["auto", "valu"])
def test_decode_from_layer_records_matches_page_list_path(masked, evict, kernel, monkeypatch,
                                                          host_read):
    """Decode steps over several layers, crossing page boundaries: with the
    watermark evicting a page at every boundary (layer-record path, host
    pages read in place or staged) or with every page resident (the layers'
    device-resident records, uploaded only when pages are added).  Both agree
    with HELM's page-list path (HELM_DISABLE_ASYNC_KV: host pages copied to
    the device first) and with the fp64 oracle, and record the same paging
    counters."""
    if kernel != "auto":
        monkeypatch.setenv("HELM_AMD_KERNEL", kernel)
    Hq, kvh, D, P, L = 8, 2, 128, 16, 3
    lens = [70, 45] if evict else [1100, 45, 301]
    B = len(lens)
    page_bytes = 2 * kvh * P * D * 2
    g = torch.Generator().manual_seed(11)
    pre = [[(torch.randn(1, kvh, n, D, generator=g).bfloat16(),
             torch.randn(1, kvh, n, D, generator=g).bfloat16()) for n in lens] for _ in range(L)]
    steps = 20
    qs = torch.randn(steps, L, B, Hq, 1, D, generator=g).bfloat16()
    kds = torch.randn(steps, L, B, kvh, 1, D, generator=g).bfloat16()
    vds = torch.randn(steps, L, B, kvh, 1, D, generator=g).bfloat16()
    results = {}
    for mode in ("records", "pages"):
        if mode == "pages":
            monkeypatch.setenv("HELM_DISABLE_ASYNC_KV", "1")
        a = KVAllocator(L, kvh, D, page_size=P, dtype=torch.bfloat16)
        wm = 3 * page_bytes if evict else 10 ** 12
        kvcms = [KVCacheManager(a, gpu_high_watermark_bytes=wm) for _ in lens]
        for lid in range(L):
            for m, (k, v) in zip(kvcms, pre[lid]):
                m.append_prefill(lid, k.to(DEV), v.to(DEV))
        KC.reset_paging_stats()
        outs = []
        for s in range(steps):
            for lid in range(L):
                mask = None
                if masked:
                    n = max(lens) + s + 1
                    mask = torch.zeros(B, 1, 1, n)
                    mask[..., ::7] = float("-inf")
                    mask = mask.to(DEV)
                outs.append(_decode_batched(kvcms, qs[s, lid].to(DEV), kds[s, lid].to(DEV),
                                            vds[s, lid].to(DEV), lid, 1 / math.sqrt(D),
                                            attention_mask=mask).cpu())
        results[mode] = (outs, KC.get_paging_stats())
        assert any(layer._n_host for m in kvcms for layer in m.layers.values()) == evict
        # the last step of every layer against the oracle
        for lid in range(L):
            for i, m in enumerate(kvcms):
                K, V = _gather(m, lid)
                n = K.size(2)
                mask = None
                if masked:
                    mask = torch.zeros(1, 1, n, dtype=torch.float64)
                    mask[..., ::7] = float("-inf")
                ref = A.attention_fp64_batched(qs[steps - 1, lid, i].float(), K[0].float(),
                                               V[0].float(), mask=mask)
                got = outs[(steps - 1) * L + lid][i].double()
                assert (got - ref).abs().max().item() <= 1e-2
        for m in kvcms:
            m.clear()
        monkeypatch.delenv("HELM_DISABLE_ASYNC_KV", raising=False)
    (o_rec, s_rec), (o_pg, s_pg) = results["records"], results["pages"]
    assert s_rec == s_pg and (s_rec["prefetch_calls"] > 0) == evict
    for x, y in zip(o_rec, o_pg):
        assert (x.float() - y.float()).abs().max().item() <= 1e-2


@pytest.mark.parametrize("evict", [False, True])
def test_decode_from_records_applies_softcap(evict):
    """The records decode path with a logit softcap (Gemma-2's decode,
    kv_cache.py:521-522): with every page resident (device-resident records)
    and with host pages, the output is tanh-capped attention, not plain
    attention."""
    from helm_amd.runtime.kv_offload import _decode_from_records
    Hq, kvh, D, P, cap = 8, 2, 128, 16, 2.0
    lens = [150, 77]
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    wm = 2 * (2 * kvh * P * D * 2) if evict else 10 ** 12
    kvcms = [KVCacheManager(a, gpu_high_watermark_bytes=wm) for _ in lens]
    g = torch.Generator().manual_seed(5)
    kv = [(torch.randn(1, kvh, n, D, generator=g).bfloat16(),
           torch.randn(1, kvh, n, D, generator=g).bfloat16()) for n in lens]
    for m, (k, v) in zip(kvcms, kv):
        m.append_prefill(0, k.to(DEV), v.to(DEV))
    assert any(L._n_host for m in kvcms for L in m.layers.values()) == evict
    # scores of a few units, so that a cap of 2 changes them
    q = (3 * torch.randn(len(lens), Hq, 1, D, generator=g)).bfloat16()
    out = _decode_from_records(kvcms, q.to(DEV), 0, kvh, D, 1 / math.sqrt(D), None, cap)
    assert out is not None
    torch.cuda.synchronize()
    for i, (k, v) in enumerate(kv):
        ref = A.attention_fp64_batched(q[i].float(), k[0].float(), v[0].float(), softcap=cap)
        plain = A.attention_fp64_batched(q[i].float(), k[0].float(), v[0].float())
        assert (ref - plain).abs().max().item() > 0.05
        assert (out[i].double().cpu() - ref).abs().max().item() <= 1e-2
    for m in kvcms:
        m.clear()


@pytest.mark.parametrize("B,T,steps", [(4, 16384, 18), (17, 600, 3)])
def test_decode_batched_many_pages_and_many_sequences(B, T, steps):
    """_decode_batched at scale: 4 sequences x 16k tokens (1,024 pages each,
    the device-resident records grown past their first capacity while steps
    cross a page boundary) and 17 sequences (more than one call carries by
    value, so the concatenated-records path runs); the last step equals the
    fp64 oracle."""
    Hq, kvh, D, P, L = 32, 8, 128, 16, 2
    a = KVAllocator(L, kvh, D, page_size=P, dtype=torch.bfloat16)
    kvcms = [KVCacheManager(a, gpu_high_watermark_bytes=10 ** 13) for _ in range(B)]
    g = torch.Generator(device=DEV).manual_seed(21)
    kv = {}
    for lid in range(L):
        for i, m in enumerate(kvcms):
            n = T + 7 * i
            k = torch.randn(1, kvh, n, D, generator=g, device=DEV).bfloat16()
            v = torch.randn(1, kvh, n, D, generator=g, device=DEV).bfloat16()
            m.append_prefill(lid, k, v)
            kv[lid, i] = [k, v]
    out = None
    for s in range(steps):
        for lid in range(L):
            q = torch.randn(B, Hq, 1, D, generator=g, device=DEV).bfloat16()
            kn = torch.randn(B, kvh, 1, D, generator=g, device=DEV).bfloat16()
            vn = torch.randn(B, kvh, 1, D, generator=g, device=DEV).bfloat16()
            out = _decode_batched(kvcms, q, kn, vn, lid, 1 / math.sqrt(D))
            for i in range(B):
                kv[lid, i][0] = torch.cat([kv[lid, i][0], kn[i:i + 1]], 2)
                kv[lid, i][1] = torch.cat([kv[lid, i][1], vn[i:i + 1]], 2)
    torch.cuda.synchronize()
    for i in sorted({0, B - 1}):
        K, V = kv[L - 1, i]
        ref = A.attention_fp64_batched(q[i].float().cpu(), K[0].float().cpu(),
                                       V[0].float().cpu())
        assert (out[i].double().cpu() - ref).abs().max().item() <= 1e-2
        k_pages, v_pages = _gather(kvcms[i], L - 1)
        assert torch.equal(k_pages, K.cpu()) and torch.equal(v_pages, V.cpu())
    for m in kvcms:
        m.clear()


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("evict", [False, True])
def test_stream_prefill_from_records_matches_page_list_path(masked, evict, monkeypatch):
    """A later prefill chunk (q_len 24) over every cached page, per item as
    HELM does (kv_offload.py:207-227): the layer-record path equals the
    page-list path (HELM_DISABLE_ASYNC_KV) and the fp64 oracle, with the same
    prefetch counters; unmasked all-device items get HELM's top-left causal."""
    Hq, kvh, D, P, S = 16, 4, 128, 16, 24
    lens = [200, 77, 130]
    B = len(lens)
    page_bytes = 2 * kvh * P * D * 2
    g = torch.Generator().manual_seed(17)
    kvs = [(torch.randn(1, kvh, n, D, generator=g).bfloat16(),
            torch.randn(1, kvh, n, D, generator=g).bfloat16()) for n in lens]
    q = torch.randn(B, Hq, S, D, generator=g).bfloat16()
    T = max(lens)
    mask = None
    if masked:
        mask = torch.zeros(B, 1, S, T)
        mask[..., 3::5] = float("-inf")
    results = {}
    for mode in ("records", "pages"):
        if mode == "pages":
            monkeypatch.setenv("HELM_DISABLE_ASYNC_KV", "1")
        a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
        kvcms = [KVCacheManager(a, gpu_high_watermark_bytes=2 * page_bytes if evict else 10 ** 12)
                 for _ in lens]
        for m, (k, v) in zip(kvcms, kvs):
            m.append_prefill(0, k.to(DEV), v.to(DEV))
        KC.reset_paging_stats()
        out = _stream_prefill_batched(kvcms, q.to(DEV), 0, 1 / math.sqrt(D),
                                      attention_mask=mask.to(DEV) if masked else None)
        torch.cuda.synchronize()
        results[mode] = (out.cpu(), KC.get_paging_stats())
        assert any(m.layers[0]._n_host for m in kvcms) == evict
        for m in kvcms:
            m.clear()
        monkeypatch.delenv("HELM_DISABLE_ASYNC_KV", raising=False)
    (o_rec, s_rec), (o_pg, s_pg) = results["records"], results["pages"]
    assert s_rec == s_pg
    assert (o_rec.float() - o_pg.float()).abs().max().item() <= 1e-2
    for i, n in enumerate(lens):
        mk = None
        if masked:
            mk = mask[i, :, :, :n].double()
        elif not evict:
            # top-left causal of HELM's Path 1: key t visible to row s iff t <= s
            mk = torch.zeros(1, S, n, dtype=torch.float64)
            mk[0][torch.arange(n)[None, :] > torch.arange(S)[:, None]] = float("-inf")
        ref = A.attention_fp64_batched(q[i].float(), kvs[i][0][0].float(), kvs[i][1][0].float(),
                                       mask=mk)
        assert (o_rec[i].double() - ref).abs().max().item() <= 1e-2


def _tiny_model(arch: str):
    """A tiny random model of `arch` (fp32, eager attention) and its twin."""
    import transformers.models as tm
    common = dict(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    if arch == "qwen2":
        cfg, cls = tm.qwen2.Qwen2Config(**common), tm.qwen2.Qwen2ForCausalLM
    elif arch == "qwen3":
        cfg, cls = tm.qwen3.Qwen3Config(head_dim=16, **common), tm.qwen3.Qwen3ForCausalLM
    elif arch == "mistral":
        cfg, cls = tm.mistral.MistralConfig(**common), tm.mistral.MistralForCausalLM
    elif arch == "olmo2":
        cfg, cls = tm.olmo2.Olmo2Config(**common), tm.olmo2.Olmo2ForCausalLM
    elif arch.startswith("gemma2"):
        # "gemma2-cap1": a logit softcap of 1, so that the tanh changes every score
        cap = 1.0 if arch == "gemma2-cap1" else 50.0
        cfg = tm.gemma2.Gemma2Config(head_dim=16, sliding_window=8, query_pre_attn_scalar=16,
                                      attn_logit_softcapping=cap, final_logit_softcapping=30.0,
                                      **common)
        cls = tm.gemma2.Gemma2ForCausalLM
    else:
        cfg, cls = tm.llama.LlamaConfig(**common), tm.llama.LlamaForCausalLM
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    ref = cls(cfg).eval().to(DEV)
    model = cls(cfg).eval().to(DEV)
    model.load_state_dict(ref.state_dict())
    return ref, model


@pytest.mark.parametrize("arch", ["llama", "qwen2", "qwen3", "mistral", "olmo2", "gemma2",
                                  "gemma2-cap1"])
def test_tiny_models_decode_logits_match_hf_with_eviction(arch):
    """Every architecture the paged forwards cover (kv_offload.py:291-651): a
    tiny random model prefills in two chunks and decodes through the paged,
    evicting cache with the same logits as HF's own full-recompute forward
    over the same tokens (teacher forced, so near-tied argmaxes cannot
    diverge the two runs)."""
    ref_model, model = _tiny_model(arch)
    conf = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=1024)
    mgr = KVOffloadManager(model, conf, batch_size=1)
    g = torch.Generator().manual_seed(2)
    S, steps = 12, 30
    ids = torch.randint(0, 97, (1, S + steps), generator=g).to(DEV)
    KC.reset_paging_stats()
    worst = 0.0
    with torch.no_grad():
        # the prompt in two chunks: the first attends over its own K/V, the
        # second over the cached pages with a chunk-causal additive mask
        # (HELM's pipeline chunk masks, pipeline_runtime.py:94-113)
        c1 = 8
        logits = model(ids[:, :c1], position_ids=torch.arange(c1, device=DEV)[None],
                       use_cache=False).logits
        ref = ref_model(ids[:, :S], use_cache=False).logits
        worst = max(worst, (logits - ref[:, :c1]).abs().max().item())
        n2 = S - c1
        chunk_mask = torch.zeros(1, 1, n2, S, device=DEV)
        chunk_mask[0, 0][torch.arange(S, device=DEV)[None, :] >
                         (c1 + torch.arange(n2, device=DEV))[:, None]] = torch.finfo(torch.float32).min
        logits = model(ids[:, c1:S], position_ids=torch.arange(c1, S, device=DEV)[None],
                       attention_mask=chunk_mask, use_cache=False,
                       cache_position=torch.arange(c1, S, device=DEV)).logits
        worst = max(worst, (logits - ref[:, c1:S]).abs().max().item())
        for t in range(steps):
            pos = S + t
            logits = model(ids[:, pos:pos + 1], position_ids=torch.tensor([[pos]], device=DEV),
                           attention_mask=None, use_cache=False,
                           cache_position=torch.tensor([pos], device=DEV)).logits
            ref = ref_model(ids[:, :pos + 1], use_cache=False).logits[:, -1:]
            worst = max(worst, (logits - ref).abs().max().item())
    mgr.restore()
    assert worst <= 2e-4, f"{arch}: max logit difference {worst}"
    assert KC.get_paging_stats()["pages_evicted"] > 0


def test_tiny_llama_greedy_matches_hf_with_eviction():
    """test_kv_eviction_e2e.py:10-66 pattern: a tiny random Llama generates the
    same greedy tokens through the paged, evicting cache as HF's own
    full-recompute forward."""
    from transformers.models.llama import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    cfg._attn_implementation = "eager"
    ref_model = LlamaForCausalLM(cfg).eval().to(DEV)
    model = LlamaForCausalLM(cfg).eval().to(DEV)
    model.load_state_dict(ref_model.state_dict())
    conf = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=1024)
    mgr = KVOffloadManager(model, conf, batch_size=1)
    prompt = torch.randint(0, 97, (1, 12), generator=torch.Generator().manual_seed(1)).to(DEV)
    steps = 40
    with torch.no_grad():
        ids = prompt.clone()
        for _ in range(steps):
            nxt = ref_model(ids, use_cache=False).logits[:, -1].argmax(-1, keepdim=True)
            ids = torch.cat([ids, nxt], 1)
        ref_tokens = ids[0, prompt.shape[1]:].tolist()

        KC.reset_paging_stats()
        S = prompt.shape[1]
        logits = model(prompt, position_ids=torch.arange(S, device=DEV)[None],
                       use_cache=False).logits
        out_tokens = []
        tok = logits[:, -1].argmax(-1, keepdim=True)
        for t in range(steps):
            out_tokens.append(int(tok))
            pos = S + t
            mask = torch.zeros(1, 1, 1, pos + 1, device=DEV)
            logits = model(tok, position_ids=torch.tensor([[pos]], device=DEV),
                           attention_mask=None, use_cache=False,
                           cache_position=torch.tensor([pos], device=DEV)).logits
            tok = logits[:, -1].argmax(-1, keepdim=True)
    mgr.restore()
    assert out_tokens == ref_tokens
    assert KC.get_paging_stats()["pages_evicted"] > 0


@pytest.mark.parametrize("case", ["decode", "mask", "softcap", "chunk", "chunk-mask", "host",
                                  "host-mask", "host-chunk"])
def test_layer_page_list_attention_matches_page_by_page(case, monkeypatch):
    """perform_streaming_attention over the list iterate_layer_pages returns
    runs from the layer's records; a plain copy of the same list runs page by
    page.  The two agree, count the same prefetches, and match the fp64
    oracle: decode with and without a mask or softcap, a query chunk under
    Path 1's top-left causal mask or an additive mask, and pages partly in
    host memory (Path 3: unmasked, no causal)."""
    taken = []
    real = KC._attend_layer_pages

    def spy(*args):
        out = real(*args)
        taken.append(out is not None)
        return out
    monkeypatch.setattr(KC, "_attend_layer_pages", spy)
    Hq, kvh, D, P, T = 8, 2, 128, 16, 300
    host = case.startswith("host")
    S = 5 if "chunk" in case else 1
    page_bytes = 2 * kvh * P * D * 2
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=4 * page_bytes if host else 10 ** 12)
    g = torch.Generator().manual_seed(21)
    k = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    v = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    assert (mgr.layers[0]._n_host > 0) == host
    q = (2 * torch.randn(1, Hq, S, D, generator=g)).bfloat16()
    mask = softcap = None
    ref_mask = None
    if "mask" in case:
        mask = torch.zeros(1, 1, S, T)
        mask[..., 3::5] = float("-inf")
        mask[0, 0, :, T - 9:] = -2.5
        ref_mask = mask[0].double()
    elif case == "softcap":
        softcap = 3.0
    elif S > 1 and not host:
        ref_mask = torch.zeros(1, S, T, dtype=torch.float64)
        ref_mask[0][torch.arange(T)[None, :] > torch.arange(S)[:, None]] = float("-inf")
    outs, stats = [], []
    for linked in (True, False):
        pages = mgr.iterate_layer_pages(0)
        if not linked:
            pages = list(pages)
        KC.reset_paging_stats()
        outs.append(perform_streaming_attention(
            q.to(DEV), pages, attention_mask=mask.to(DEV) if mask is not None else None,
            softcap=softcap).cpu())
        stats.append(KC.get_paging_stats())
    assert taken == [True]
    assert stats[0] == stats[1] and (stats[0]["prefetch_calls"] == 1) == host
    ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(), mask=ref_mask,
                                   softcap=softcap)
    for o in outs:
        assert o.shape == q.shape and o.dtype == q.dtype
        assert (o[0].double() - ref).abs().max().item() <= 1e-2
    assert (outs[0].float() - outs[1].float()).abs().max().item() <= 1e-2
    mgr.clear()


@pytest.mark.parametrize("chunk", ["32", "16"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,B,pps", [(1024, 1, None), (512, 2, 300), (256, 1, None)])
def test_chunk_kernel_long_splits(dtype, S, B, pps, chunk, monkeypatch):
    """Query chunks over 257 pages (last one partial) where a split spans more
    than the 64 page records one lane window holds.  S = 1024: enough
    workgroups that every (KV head, tile block) takes all pages in one split
    and the chunk kernel writes the output itself; S = 512 with a second,
    empty sequence and 300 pages per split: the same, with zeros for the
    empty sequence; S = 256: four splits of 65 pages, merged.  All match the
    fp64 oracle under an additive chunk mask (checked on two KV heads)."""
    monkeypatch.setenv("HELM_AMD_CHUNK", chunk)
    if pps is not None:
        monkeypatch.setenv("HELM_AMD_PPS", str(pps))
    Hq, kvh, D, P, T = 32, 8, 128, 16, 4100
    G = Hq // kvh
    tol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    a = KVAllocator(1, kvh, D, page_size=P, dtype=dtype)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator().manual_seed(23)
    k = torch.randn(1, kvh, T, D, generator=g).to(dtype)
    v = torch.randn(1, kvh, T, D, generator=g).to(dtype)
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    q = torch.randn(B, Hq, S, D, generator=g).to(dtype)
    mask = torch.zeros(1, 1, S, T)
    lim = T - S + torch.arange(S)
    mask[0, 0][torch.arange(T)[None, :] > lim[:, None]] = float("-inf")
    mask[..., 5::11] = -1.75
    rec = mgr.layers[0].records()
    n = len(rec)
    seq_off = np.array([0] + [n] * B, dtype=np.int32)
    out = KC._attend_records(q.to(DEV), rec, seq_off, T, kvh, dtype, 1 / math.sqrt(D),
                             mask.to(DEV), None, False).cpu()
    for hk in (0, kvh - 1):
        hs = slice(hk * G, (hk + 1) * G)
        ref = A.attention_fp64_batched(q[0, hs].float(), k[0, hk:hk + 1].float(),
                                       v[0, hk:hk + 1].float(), mask=mask[0].double())
        assert (out[0, hs].double() - ref).abs().max().item() <= tol
    if B > 1:
        assert torch.count_nonzero(out[1]).item() == 0
    mgr.clear()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_page64_ragged_prefill_chunks_then_decode(dtype):
    """HELM's default page size (64 tokens: four 16-token blocks per page)
    with prefill chunks of odd lengths, so that several pages in the middle
    of the sequence are partly filled (append_prefill starts a new page per
    chunk, kv_cache.py:113-143): a later 300-token chunk under an additive
    mask, and decode steps after it, match the fp64 oracle over the gathered
    tokens, through the records path and HELM's page-list path alike."""
    Hq, kvh, D, P = 16, 4, 128, 64
    tol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    a = KVAllocator(1, kvh, D, page_size=P, dtype=dtype)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator().manual_seed(29)
    chunks = [1000, 777, 515, 300]
    ks, vs = [], []
    for n in chunks:
        k = torch.randn(1, kvh, n, D, generator=g).to(dtype)
        v = torch.randn(1, kvh, n, D, generator=g).to(dtype)
        mgr.append_prefill(0, k.to(DEV), v.to(DEV))
        ks.append(k)
        vs.append(v)
    used = [p.used_tokens for p in mgr.layers[0].pages]
    assert any(u < P for u in used[:-1])              # partly filled pages mid-sequence
    K, V = torch.cat(ks, 2), torch.cat(vs, 2)
    T, S = K.size(2), chunks[-1]
    q = torch.randn(1, Hq, S, D, generator=g).to(dtype)
    mask = torch.zeros(1, 1, S, T)
    mask[0, 0][torch.arange(T)[None, :] > (T - S + torch.arange(S))[:, None]] = float("-inf")
    mask[..., 7::13] = -3.0
    ref = A.attention_fp64_batched(q[0].float(), K[0].float(), V[0].float(),
                                   mask=mask[0].double())
    out = _stream_prefill_batched([mgr], q.to(DEV), 0, 1 / math.sqrt(D),
                                  attention_mask=mask.to(DEV)).cpu()
    assert (out[0].double() - ref).abs().max().item() <= tol
    pl = perform_streaming_attention(q.to(DEV), list(mgr.iterate_layer_pages(0)),
                                     attention_mask=mask.to(DEV)).cpu()
    assert (pl[0].double() - ref).abs().max().item() <= tol
    for step in range(70):                            # crosses into a new page
        kd = torch.randn(1, kvh, 1, D, generator=g).to(dtype)
        vd = torch.randn(1, kvh, 1, D, generator=g).to(dtype)
        qd = torch.randn(1, Hq, 1, D, generator=g).to(dtype)
        od = _decode_batched([mgr], qd.to(DEV), kd.to(DEV), vd.to(DEV), 0, 1 / math.sqrt(D))
        K, V = torch.cat([K, kd], 2), torch.cat([V, vd], 2)
        if step in (0, 69):
            r = A.attention_fp64_batched(qd[0].float(), K[0].float(), V[0].float())
            assert (od[0].double().cpu() - r).abs().max().item() <= tol
    mgr.clear()


@pytest.mark.parametrize("chunk", ["32", "16"])
@pytest.mark.parametrize("S", [5, 9, 12, 17, 33])
def test_chunk_kernels_row_counts(chunk, S, monkeypatch):
    """Both query-chunk kernels (32-row waves on 32x32 MFMA tiles, the
    default; 16-row waves with HELM_AMD_CHUNK=16) at query-row counts that
    leave a wave with one 16-row tile, a partial tile or both (G = 4:
    20 .. 132 rows), under an additive mask and under HELM's top-left
    causal, against the fp64 oracle."""
    monkeypatch.setenv("HELM_AMD_CHUNK", chunk)
    Hq, kvh, D, P, T = 16, 4, 128, 16, 301
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator().manual_seed(31 + S)
    k = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    v = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    q = torch.randn(1, Hq, S, D, generator=g).bfloat16()
    mask = torch.zeros(1, 1, S, T)
    mask[0, 0][torch.arange(T)[None, :] > (T - S + torch.arange(S))[:, None]] = float("-inf")
    mask[..., 2::9] = -1.5
    out = _stream_prefill_batched([mgr], q.to(DEV), 0, 1 / math.sqrt(D),
                                  attention_mask=mask.to(DEV)).cpu()
    ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(), mask=mask[0].double())
    assert (out[0].double() - ref).abs().max().item() <= 1e-2
    causal = _stream_prefill_batched([mgr], q.to(DEV), 0, 1 / math.sqrt(D)).cpu()
    cm = torch.zeros(1, S, T, dtype=torch.float64)
    cm[0][torch.arange(T)[None, :] > torch.arange(S)[:, None]] = float("-inf")
    ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(), mask=cm)
    assert (causal[0].double() - ref).abs().max().item() <= 1e-2
    mgr.clear()


@pytest.mark.parametrize("chunk", ["32", "16"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunk_kernels_softcap_and_window_mask(chunk, dtype, monkeypatch):
    """Gemma-2's prefill over cached pages on the matrix-core chunk kernels:
    a logit soft-cap together with a sliding-window additive mask (every
    feature at once), 40 query rows per KV head, host pages included (the
    watermark keeps four pages on the device), against the fp64 oracle."""
    monkeypatch.setenv("HELM_AMD_CHUNK", chunk)
    Hq, kvh, D, P, T, S, cap = 8, 2, 128, 16, 420, 10, 5.0
    tol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    a = KVAllocator(1, kvh, D, page_size=P, dtype=dtype)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=4 * (2 * kvh * P * D * 2))
    g = torch.Generator().manual_seed(37)
    k = torch.randn(1, kvh, T, D, generator=g).to(dtype)
    v = torch.randn(1, kvh, T, D, generator=g).to(dtype)
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    assert mgr.layers[0]._n_host > 0
    q = (2 * torch.randn(1, Hq, S, D, generator=g)).to(dtype)
    pos = T - S + torch.arange(S)
    key = torch.arange(T)
    mask = torch.zeros(1, 1, S, T)
    mask[0, 0][(key[None, :] > pos[:, None]) | (key[None, :] <= pos[:, None] - 64)] = \
        torch.finfo(torch.float32).min
    out = _stream_prefill_batched([mgr], q.to(DEV), 0, 0.1, attention_mask=mask.to(DEV),
                                  softcap=cap).cpu()
    ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(), scale=0.1,
                                   mask=mask[0].double(), softcap=cap)
    assert (out[0].double() - ref).abs().max().item() <= tol
    mgr.clear()


@pytest.mark.parametrize("masked", [True, False])
def test_chunk32_skips_only_steps_that_add_nothing(masked):
    """A first prompt chunk over its own 600 tokens (S = T) under HF's
    causal mask (finfo.min, as the pipeline's masks are) or HELM's top-left
    causal: the 32x32 kernel skips the steps past each wave's last query
    position, and the result still equals the fp64 oracle; a second case puts
    finite mask values among finfo.min ones so that only all-masked steps
    can be skipped."""
    Hq, kvh, D, P, T = 16, 4, 128, 16, 600
    S = T
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator().manual_seed(41)
    k = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    v = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    q = torch.randn(1, Hq, S, D, generator=g).bfloat16()
    fut = torch.arange(T)[None, :] > torch.arange(S)[:, None]
    for variant in (0, 1):
        mask = None
        ref_mask = torch.zeros(1, S, T, dtype=torch.float64)
        if masked:
            mask = torch.zeros(1, 1, S, T)
            mask[0, 0][fut] = torch.finfo(torch.float32).min
            if variant == 1:
                mask[0, 0, :, 500:520] = -2.0          # visible again, with a bias
            ref_mask = mask[0].double()
        else:
            ref_mask[0][fut] = float("-inf")
            if variant == 1:
                break
        out = _stream_prefill_batched([mgr], q.to(DEV), 0, 1 / math.sqrt(D),
                                      attention_mask=mask.to(DEV) if masked else None).cpu()
        ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(), mask=ref_mask)
        assert (out[0].double() - ref).abs().max().item() <= 1e-2
    mgr.clear()


@pytest.mark.parametrize("mdtype", [torch.float32, torch.bfloat16, torch.float16])
def test_first_chunk_causal_mask_shortcut_is_exact(mdtype, monkeypatch):
    """The first prompt chunk under HF's causal mask (finfo.min of the mask's
    dtype above the diagonal) runs as causal masking, with exactly the output
    of the masked call; a mask that differs anywhere (a padded first key) is
    not taken for causal, and an in-place change of a mask is noticed."""
    from helm_amd.runtime import kv_offload as KO
    B, Hq, kvh, D, S = 2, 8, 2, 128, 300
    g = torch.Generator().manual_seed(43)
    q = torch.randn(B, Hq, S, D, generator=g).bfloat16().to(DEV)
    k = torch.randn(B, kvh, S, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(B, kvh, S, D, generator=g).bfloat16().to(DEV)
    mask = torch.zeros(B, 1, S, S, dtype=mdtype)
    mask[:, 0][:, torch.ones(S, S, dtype=torch.bool).triu(1)] = torch.finfo(mdtype).min
    mask = mask.to(DEV)
    fast = KO._local_attention(q, k, v, 1 / math.sqrt(D), mask)
    assert KO._causal_mask_offset(mask, S) == 0
    monkeypatch.setattr(KO, "_causal_mask_offset", lambda *a: None)
    slow = KO._local_attention(q, k, v, 1 / math.sqrt(D), mask)
    monkeypatch.undo()
    assert torch.equal(fast, slow)
    ref = A.attention_fp64_batched(q[1].float().cpu(), k[1].float().cpu(), v[1].float().cpu(),
                                   mask=mask[1].double().cpu())
    assert (fast[1].double().cpu() - ref).abs().max().item() <= 1e-2
    mask[1, 0, 5:, 0] = torch.finfo(mdtype).min       # item 1: key 0 padded away
    assert KO._causal_mask_offset(mask, S) is None
    out = KO._local_attention(q, k, v, 1 / math.sqrt(D), mask)
    ref = A.attention_fp64_batched(q[1].float().cpu(), k[1].float().cpu(), v[1].float().cpu(),
                                   mask=mask[1].double().cpu())
    assert (out[1].double().cpu()[:, 5:] - ref[:, 5:]).abs().max().item() <= 1e-2


def _chunk_mask(past, S, dtype, B=1):
    """HELM's prefill chunk mask (helm/runtime/pipeline_runtime.py:94-113):
    queries at past .. past + S - 1 see keys 0 .. their own position; finfo.min
    of the mask's dtype elsewhere."""
    T = past + S
    allowed = torch.arange(T)[None, :] <= past + torch.arange(S)[:, None]
    m = torch.where(allowed, torch.zeros((), dtype=dtype),
                    torch.full((), torch.finfo(dtype).min, dtype=dtype))
    return m[None, None].expand(B, 1, S, T).contiguous()


@pytest.mark.parametrize("mdtype,cap,evict", [(torch.float32, None, False),
                                              (torch.bfloat16, None, True),
                                              (torch.float16, 30.0, False)])
def test_later_chunk_causal_mask_shortcut_is_exact(mdtype, cap, evict, monkeypatch):
    """A later prompt chunk (300 queries after 1,037 cached tokens, pages of
    16, two sequences) under HELM's chunk mask runs as causal masking at
    offset `past`, with exactly the output of the masked call (soft-cap and
    host pages too), within tolerance of the fp64 oracle; a mask with one
    entry changed is not taken for causal."""
    from helm_amd.runtime import kv_offload as KO
    B, Hq, kvh, D, P, past, S = 2, 8, 2, 128, 16, 1037, 300
    T = past + S
    g = torch.Generator().manual_seed(47)
    k = torch.randn(B, kvh, T, D, generator=g).bfloat16()
    v = torch.randn(B, kvh, T, D, generator=g).bfloat16()
    q = torch.randn(B, Hq, S, D, generator=g).bfloat16()
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    budget = 8 * (2 * kvh * P * D * 2) if evict else 10 ** 12
    mgrs = [KVCacheManager(a, gpu_high_watermark_bytes=budget) for _ in range(B)]
    for b in range(B):
        mgrs[b].append_prefill(0, k[b:b + 1].to(DEV), v[b:b + 1].to(DEV))
        assert (mgrs[b].layers[0]._n_host > 0) == evict
    mask = _chunk_mask(past, S, mdtype, B).to(DEV)
    assert KO._causal_mask_offset(mask, S) == past
    fast = _stream_prefill_batched(mgrs, q.to(DEV), 0, 1 / math.sqrt(D), attention_mask=mask,
                                   softcap=cap)
    monkeypatch.setattr(KO, "_causal_mask_offset", lambda *a: None)
    slow = _stream_prefill_batched(mgrs, q.to(DEV), 0, 1 / math.sqrt(D), attention_mask=mask,
                                   softcap=cap)
    monkeypatch.undo()
    assert torch.equal(fast, slow)
    for b in range(B):
        ref = A.attention_fp64_batched(q[b].float(), k[b].float(), v[b].float(),
                                       mask=mask[b].double().cpu(), softcap=cap)
        assert (fast[b].double().cpu() - ref).abs().max().item() <= 1e-2
    mask[1, 0, 7, past + 8] = 0.0                   # row 7 sees one future key
    assert KO._causal_mask_offset(mask, S) is None
    out = _stream_prefill_batched(mgrs, q.to(DEV), 0, 1 / math.sqrt(D), attention_mask=mask,
                                  softcap=cap)
    ref = A.attention_fp64_batched(q[1].float(), k[1].float(), v[1].float(),
                                   mask=mask[1].double().cpu(), softcap=cap)
    assert (out[1].double().cpu() - ref).abs().max().item() <= 1e-2
    for m in mgrs:
        m.clear()


@pytest.mark.parametrize("kernel,chunk,S", [("mfma", "32", 4), ("mfma", "32", 40),
                                            ("mfma", "16", 40), ("valu", "32", 40),
                                            ("generic", "32", 9)])
def test_causal_offset_through_the_abi_matches_oracle(kernel, chunk, S, monkeypatch):
    """helm_stream_attn with causal = 1 + past over a contiguous K/V (query
    position s sees keys 0 .. s + past) equals the fp64 oracle under the
    matching additive mask, for an offset that ends inside a page, on every
    kernel that takes the flag (decode tile: G * S <= 16 rows; the 32- and
    16-row chunk kernels; the vector-ALU kernels)."""
    from helm_amd.runtime.kv_cache import _attend, _contiguous_segments
    monkeypatch.setenv("HELM_AMD_KERNEL", kernel)
    monkeypatch.setenv("HELM_AMD_CHUNK", chunk)
    Hq, kvh, D, past = 12, 4, 128, 77
    T = past + S + 5                                  # 5 keys past every row's limit
    g = torch.Generator().manual_seed(53)
    q = torch.randn(1, Hq, S, D, generator=g).half()
    k = torch.randn(1, kvh, T, D, generator=g).half()
    v = torch.randn(1, kvh, T, D, generator=g).half()
    kd, vd = k.to(DEV), v.to(DEV)
    out = _attend(q.to(DEV), [_contiguous_segments(kd, vd, 0)], kvh, torch.float16, 0.125,
                  None, None, 1 + past).cpu()
    allowed = torch.arange(T)[None, :] <= past + torch.arange(S)[:, None]
    mask = torch.zeros(1, S, T, dtype=torch.float64).masked_fill(~allowed, float("-inf"))
    ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(), scale=0.125,
                                   mask=mask)
    assert (out[0].double() - ref).abs().max().item() <= 2e-3


def test_chunk32_rows_that_start_fully_masked_follow_helms_loop():
    """A 40-row chunk (32-row waves) over 300 cached tokens under a mask whose
    rows 0-4 are finfo.min everywhere (HELM's loop weighs such a row's keys
    uniformly: the mean of V) and rows 5-9 finfo.min over their first 100
    keys (weights of those keys are wiped by the first refresh), the rest
    chunk-causal: every row matches HELM's loop restated by the oracle."""
    Hq, kvh, D, P, T, S = 8, 2, 128, 16, 300, 40
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator().manual_seed(59)
    k = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    v = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    mgr.append_prefill(0, k.to(DEV), v.to(DEV))
    q = torch.randn(1, Hq, S, D, generator=g).bfloat16()
    mn = torch.finfo(torch.float32).min
    pos = T - S + torch.arange(S)
    mask = torch.where(torch.arange(T)[None, :] <= pos[:, None], torch.zeros(()),
                       torch.full((), mn))
    mask[0:5] = mn
    mask[5:10, :100] = mn
    mask = mask[None, None]
    out = _stream_prefill_batched([mgr], q.to(DEV), 0, 1 / math.sqrt(D),
                                  attention_mask=mask.to(DEV)).cpu()
    pages = [(k[:, :, t:t + P], v[:, :, t:t + P]) for t in range(0, T, P)]
    helm = A.online_softmax_pages(q.float(), [(kp.float(), vp.float()) for kp, vp in pages],
                                  scale=1 / math.sqrt(D), attention_mask=mask)
    assert (out.float() - helm.float()).abs().max().item() <= 1e-2
    vmean = v[0].float().mean(1).repeat_interleave(Hq // kvh, 0)       # [Hq, D]
    assert (out[0, :, 0:5].float() - vmean[:, None]).abs().max().item() <= 1e-2
    ref = A.attention_fp64_batched(q[0, :, 5:].float(), k[0].float(), v[0].float(),
                                   mask=mask[0, :, 5:].double(), scale=1 / math.sqrt(D))
    assert (out[0, :, 5:].double() - ref).abs().max().item() <= 1e-2
    mgr.clear()


@pytest.mark.parametrize("host_mode", ["copy", "direct"])
def test_causal_chunk_over_host_pages_out_of_token_order(host_mode, monkeypatch):
    """One sequence whose pages, the prompt chunk's own included, are almost
    all evicted (watermark 0).  Host slots come LIFO from reserves of 16, so
    host addresses run against token order inside each reserve, and staged
    pages are copied in address order.  A 100-row prompt chunk under HELM's
    chunk mask (run as causal masking at its offset) and the masked call
    both match the fp64 oracle, whether the host pages are staged or read
    in place.  (They are not compared bit for bit: the causal call attends
    the pages in token order, the masked call in descriptor order — staged
    pages by address, pages read in place ahead of the device pages, among
    them the prompt's partly filled last page — so their fp32 sums run in
    different orders.)"""
    from helm_amd.runtime import kv_offload as KO
    monkeypatch.setenv("HELM_AMD_HOST_READ", host_mode)
    Hq, kvh, D, P, past, S = 8, 2, 128, 16, 500, 100
    T = past + S
    g = torch.Generator().manual_seed(61)
    k = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    v = torch.randn(1, kvh, T, D, generator=g).bfloat16()
    q = torch.randn(1, Hq, S, D, generator=g).bfloat16()
    a = KVAllocator(1, kvh, D, page_size=P, dtype=torch.bfloat16)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=0)
    mgr.append_prefill(0, k[:, :, :past].to(DEV), v[:, :, :past].to(DEV))
    mgr.append_prefill(0, k[:, :, past:].to(DEV), v[:, :, past:].to(DEV))
    rec = mgr.layers[0].records()
    host = rec[(rec["flags"] & _native.HELM_PAGE_HOST) != 0]
    assert len(host) > 16 and np.any(np.diff(host["k"].astype(np.int64)) < 0)
    mask = _chunk_mask(past, S, torch.float32).to(DEV)
    assert KO._causal_mask_offset(mask, S) == past
    scale = 1 / math.sqrt(D)
    fast = _stream_prefill_batched([mgr], q.to(DEV), 0, scale, attention_mask=mask)
    monkeypatch.setattr(KO, "_causal_mask_offset", lambda *a: None)
    slow = _stream_prefill_batched([mgr], q.to(DEV), 0, scale, attention_mask=mask)
    monkeypatch.undo()
    ref = A.attention_fp64_batched(q[0].float(), k[0].float(), v[0].float(),
                                   mask=mask[0].double().cpu())
    assert (fast[0].double().cpu() - ref).abs().max().item() <= 1e-2
    assert (slow[0].double().cpu() - ref).abs().max().item() <= 1e-2
    mgr.clear()


def test_raw_stream_pointer_is_torchs_current_stream():
    """The launch stream the runtime passes is torch's current stream, also
    inside a `with torch.cuda.stream(...)` block."""
    from helm_amd.runtime import engine
    assert engine.stream_ptr(DEV) == torch.cuda.current_stream(DEV).cuda_stream
    s = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(s):
        assert engine.stream_ptr(DEV) == s.cuda_stream
    assert engine.stream_ptr(torch.device("cuda")) == torch.cuda.current_stream().cuda_stream


def test_record_validation_mode_checks_the_device_copy(monkeypatch):
    """HELM_AMD_CHECK_RECORDS=1 on the device-records path: decode steps
    through _decode_batched validate every layer's records and read back
    their device copy (results unchanged, against fp64); a device record
    that drifted from its page (here a smaller used count: a harmless
    change, should the check miss it) makes the next call raise before any
    launch."""
    monkeypatch.setenv("HELM_AMD_CHECK_RECORDS", "1")
    Hq, Hkv, D, T, dtype = 8, 2, 128, 200, torch.bfloat16
    a = KVAllocator(1, Hkv, D, page_size=16, dtype=dtype)
    mgr = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12)
    g = torch.Generator(device=DEV).manual_seed(61)
    k = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    v = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    mgr.append_prefill(0, k, v)
    K, V = k[0].cpu(), v[0].cpu()
    for step in range(3):
        q = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=dtype)
        kn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
        vn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
        out = _decode_batched([mgr], q, kn, vn, 0, 1 / math.sqrt(D), None)
        K, V = torch.cat([K, kn[0].cpu()], 1), torch.cat([V, vn[0].cpu()], 1)
        ref = A.attention_fp64_batched(q[0].float().cpu(), K.float(), V.float())
        assert (out[0].double().cpu() - ref).abs().max().item() <= 1e-2
    layer = mgr.layers[0]
    torch.cuda.synchronize()
    rb = _native.PAGE_DTYPE.itemsize
    dev = layer._dev[:rb].cpu().numpy().view(_native.PAGE_DTYPE).copy()
    dev["used"][0] -= 1
    layer._dev[:rb].copy_(torch.from_numpy(dev.view(np.uint8)).to(DEV))
    q = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=dtype)
    with pytest.raises(RuntimeError, match="device record 0 differs"):
        perform_streaming_attention(q, mgr.iterate_layer_pages(0))
    mgr.clear()


@pytest.mark.parametrize("Hq,Hkv,dtype", [(32, 8, torch.bfloat16), (40, 2, torch.float16),
                                          (16, 8, torch.float32)])
def test_decode_batched_writes_tokens_inside_the_attention_call(Hq, Hkv, dtype, monkeypatch):
    """_decode_batched over device-resident records writes each item's new
    token inside the attention launch (helm_paged_attn_seqs_append) where the
    matrix-core decode kernel runs (16-bit KV, D = 128; with 20 query rows per
    KV head two query tiles write the same token) and with the separate
    append launch otherwise (fp32).  Against the same steps with the separate
    launch forced (HELM_AMD_FUSED_APPEND=0): outputs and every page equal bit
    for bit, over ragged items whose tokens fill partial pages and open new
    ones; the last step against fp64."""
    D, P, L, B = 128, 16, 2, 3
    g = torch.Generator(device=DEV).manual_seed(71)
    lens = [45, 16, 31]
    prompt = [[(torch.randn(1, Hkv, n, D, generator=g, device=DEV).to(dtype),
                torch.randn(1, Hkv, n, D, generator=g, device=DEV).to(dtype)) for n in lens]
              for _ in range(L)]
    steps = [(torch.randn(B, Hq, 1, D, generator=g, device=DEV).to(dtype),
              torch.randn(B, Hkv, 1, D, generator=g, device=DEV).to(dtype),
              torch.randn(B, Hkv, 1, D, generator=g, device=DEV).to(dtype)) for _ in range(5)]

    def run(fused):
        monkeypatch.setenv("HELM_AMD_FUSED_APPEND", "1" if fused else "0")
        a = KVAllocator(L, Hkv, D, page_size=P, dtype=dtype)
        kvcms = [KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12) for _ in range(B)]
        for lid in range(L):
            for i, m in enumerate(kvcms):
                m.append_prefill(lid, *prompt[lid][i])
        outs = []
        for q, kn, vn in steps:
            for lid in range(L):
                outs.append(_decode_batched(kvcms, q, kn, vn, lid, 1 / math.sqrt(D)).cpu())
        torch.cuda.synchronize()
        pages = [_gather(m, lid) for lid in range(L) for m in kvcms]
        for m in kvcms:
            m.clear()
        return outs, pages

    fused_out, fused_pages = run(True)
    sep_out, sep_pages = run(False)
    for x, y in zip(fused_out, sep_out):
        assert torch.equal(x, y)
    for (k1, v1), (k2, v2) in zip(fused_pages, sep_pages):
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
    # the pages hold prompt + every step's token; the last step against fp64
    q = steps[-1][0]
    for i in range(B):
        K = torch.cat([prompt[L - 1][i][0].cpu()] + [s[1][i:i + 1].cpu() for s in steps], 2)
        V = torch.cat([prompt[L - 1][i][1].cpu()] + [s[2][i:i + 1].cpu() for s in steps], 2)
        k_pages, v_pages = fused_pages[(L - 1) * B + i]
        assert torch.equal(k_pages, K) and torch.equal(v_pages, V)
        ref = A.attention_fp64_batched(q[i].float().cpu(), K[0].float(), V[0].float())
        tol = 1e-2 if dtype == torch.bfloat16 else 2e-3
        assert (fused_out[-1][i].double() - ref).abs().max().item() <= tol
