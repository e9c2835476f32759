"""Paged KV cache + streaming attention — drop-in for helm/runtime/kv_cache.py.

Same public surface as HELM (helm/runtime/kv_cache.py:15-662): paging
counters, ``KVPage``, ``LayerKVCache``, ``KVCacheManager`` (append, residency
watermark, oldest-first eviction, contiguous fast path) and
``perform_streaming_attention``.  What changes is where the work happens:

* token appends are one ``helm_page_append`` kernel per call instead of two
  ``copy_`` per page (kv_cache.py:135-136, :164-165);
* eviction moves all selected pages with one batched, coalesced
  ``helm_evict_pages`` copy into pinned host slots (kv_cache.py:179-222);
* attention is ``helm_stream_attn``: split-K HIP kernels over the page list,
  with host pages prefetched through a device staging ring by hipMemcpyAsync
  on the caller's stream, each staged chunk attended right behind its copy
  (kv_cache.py:405-662);
* a query on the CPU (the attention of HELM's CPU-stage layers) runs
  ``helm_cpu_stream_attn`` of libhelm_cpu.so, a native host-CPU kernel over
  the same page records (HELM's masked loop and Path 2 on the CPU,
  kv_cache.py:531-555, :573-577).  Neither library has a torch fallback.
"""
from __future__ import annotations

import heapq
import math
import os
import struct
import threading
import weakref
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from helm_amd import _cpu_native, _native
from helm_amd.runtime import engine as _engine
from helm_amd.runtime.page import KVPage

__all__ = [
    "KVPagingStats", "reset_paging_stats", "get_paging_stats", "KVPage", "LayerKVCache",
    "KVCacheManager", "perform_streaming_attention",
]


# ── paging counters (kv_cache.py:15-62) ─────────────────────────────────────────
@dataclass
class KVPagingStats:
    evict_calls: int = 0
    pages_evicted: int = 0
    bytes_evicted: int = 0
    prefetch_calls: int = 0
    pages_prefetched: int = 0
    bytes_prefetched: int = 0


_PAGING_STATS = KVPagingStats()


def reset_paging_stats() -> None:
    """Zero the process-global paging counters."""
    global _PAGING_STATS
    _PAGING_STATS = KVPagingStats()


def get_paging_stats() -> dict:
    """The paging counters as a plain dict."""
    s = _PAGING_STATS
    return {
        "evict_calls": s.evict_calls,
        "pages_evicted": s.pages_evicted,
        "bytes_evicted": s.bytes_evicted,
        "prefetch_calls": s.prefetch_calls,
        "pages_prefetched": s.pages_prefetched,
        "bytes_prefetched": s.bytes_prefetched,
    }


def _record_eviction(n_pages: int, n_bytes: int) -> None:
    """One eviction call that moved n_pages (n_bytes) GPU->CPU."""
    if n_pages <= 0:
        return
    _PAGING_STATS.evict_calls += 1
    _PAGING_STATS.pages_evicted += n_pages
    _PAGING_STATS.bytes_evicted += n_bytes


def _record_prefetch(n_pages: int, n_bytes: int) -> None:
    """One attention call that streamed n_pages (n_bytes) CPU->GPU."""
    if n_pages <= 0:
        return
    _PAGING_STATS.prefetch_calls += 1
    _PAGING_STATS.pages_prefetched += n_pages
    _PAGING_STATS.bytes_prefetched += n_bytes


def _page_bytes(page: KVPage) -> int:
    """K+V bytes of a whole page tensor (kv_cache.py:218, :232)."""
    return page.k_tensor.numel() * page.k_tensor.element_size() * 2


def _page_record_fields(page: KVPage):
    """(k address, v address, head stride, on host) of a [1, Hkv, P, D] page
    whose rows are dense, or None when the kernel cannot read it in place."""
    k, v = page.k_tensor, page.v_tensor
    if (k.dim() != 4 or v.shape != k.shape or k.size(0) != 1 or k.dtype != v.dtype
            or k.stride(3) != 1 or v.stride(3) != 1 or k.stride(2) != k.size(3)
            or v.stride(2) != v.size(3) or v.stride(1) != k.stride(1)):
        return None
    return k.data_ptr(), v.data_ptr(), k.stride(1), k.device.type != "cuda"


# ── layer cache (kv_cache.py:77-86) ───────────────────────────────────────────
class LayerKVCache:
    """A layer's pages in token order, plus the kernel's view of them.

    Besides HELM's fields the layer keeps one ``helm_page`` record per page
    (address, used tokens, token offset, host flag), updated as pages are
    appended, filled and evicted through the cache manager, so that an
    attention call hands the kernel this array instead of rebuilding a
    descriptor per page.  Pages are expected to change only through
    ``append_page`` and the manager; ``records()`` returns None when a page
    was appended that the kernel cannot read in place.
    """

    def __init__(self, layer_id: int):
        self.layer_id = layer_id
        self.pages: List[KVPage] = []
        self.tail_page: Optional[KVPage] = None
        self.total_tokens: int = 0
        self._rec = np.zeros(16, dtype=_native.PAGE_DTYPE)
        self._rec_ok = True
        self._rec_sig = None            # (dtype, Hkv, D) of the first page
        self._tier: List[tuple] = []    # per page: (tier, host bytes) as counted
        self._n_host = 0                # pages held in host memory
        self._host_bytes = 0            # their used K+V bytes
        self._n_other = 0               # pages neither GPU- nor CPU-resident
        self._page_tokens = 0           # largest page capacity
        self._aligned16 = True          # every K/V base and head stride 16-byte aligned
        self._dev = None                # device copy of the records (uint8 tensor)
        self._dev_dirty: List[int] = []  # records changed since the last upload
        self._dev_all = False           # every record needs an upload
        self._gen = 0                   # bumped whenever the page list changes
        self._tail_tok_off = 0          # the tail record's token offset

    def _reset(self) -> None:
        """Drops every page (the list is emptied in place)."""
        self.pages.clear()
        self._gen += 1
        self.tail_page = None
        self.total_tokens = 0
        self._rec_ok, self._rec_sig = True, None
        self._tier.clear()
        self._n_host = self._host_bytes = self._n_other = 0
        self._page_tokens, self._aligned16 = 0, True
        self._dev_dirty.clear()
        self._dev_all = True
        self._tail_tok_off = 0

    def append_page(self, page: KVPage):
        self.pages.append(page)
        self._gen += 1
        self.tail_page = page
        n = len(self.pages)
        if n > self._rec.shape[0]:
            grown = np.zeros(max(n, 2 * self._rec.shape[0]), dtype=_native.PAGE_DTYPE)
            grown[:n - 1] = self._rec[:n - 1]
            self._rec = grown
        r = self._rec[n - 1:n]
        r["tok_off"] = (int(self._rec["tok_off"][n - 2]) + int(self._rec["used"][n - 2])
                        if n > 1 else 0)
        self._tail_tok_off = int(r["tok_off"][0])
        self._tier.append((0, 0))
        self._set_record(n - 1, page)
        # the old tail's device record takes its final token count
        self._mark_dirty(n - 2)
        self._mark_dirty(n - 1)

    def _set_record(self, idx: int, page: KVPage) -> None:
        """Writes page `idx`'s record and counts its residency tier."""
        tier, hb = self._tier[idx]
        if tier == 1:
            self._n_host -= 1
            self._host_bytes -= hb
        elif tier == 2:
            self._n_other -= 1
        host = page.device.type != "cuda"
        if host and page.state == 'CPU':
            tier, hb = 1, _used_bytes(page)
            self._n_host += 1
            self._host_bytes += hb
        elif not host and page.state == 'GPU':
            tier, hb = 0, 0
        else:
            tier, hb = 2, 0
            self._n_other += 1
        self._tier[idx] = (tier, hb)
        fields = _page_record_fields(page)
        sig = (page.k_tensor.dtype, page.k_tensor.size(1) if page.k_tensor.dim() == 4 else -1,
               page.k_tensor.size(-1) if page.k_tensor.dim() else -1)
        if self._rec_sig is None:
            self._rec_sig = sig
        if fields is None or sig != self._rec_sig:
            self._rec_ok = False
            return
        r = self._rec[idx:idx + 1]
        r["k"], r["v"], r["head_stride"] = fields[0], fields[1], fields[2]
        r["used"] = page.used_tokens
        r["flags"] = _native.HELM_PAGE_HOST if fields[3] else 0
        self._page_tokens = max(self._page_tokens, page.capacity_tokens, page.used_tokens)
        es = page.k_tensor.element_size()
        self._aligned16 = self._aligned16 and (fields[0] % 16 == 0 and fields[1] % 16 == 0
                                               and (fields[2] * es) % 16 == 0)

    def _tail_filled(self) -> None:
        """The tail page gained tokens (its record's used count follows)."""
        self._rec["used"][len(self.pages) - 1] = self.tail_page.used_tokens

    def _replace_page(self, idx: int, page: KVPage) -> None:
        """Page `idx` moved tiers: `page` takes its place and record."""
        old = self.pages[idx]
        self.pages[idx] = page
        self._gen += 1
        if self.tail_page is old:
            self.tail_page = page
        self._set_record(idx, page)
        self._mark_dirty(idx)

    def _mark_dirty(self, idx: int) -> None:
        if idx < 0 or self._dev_all:
            return
        self._dev_dirty.append(idx)
        if len(self._dev_dirty) > 4096:
            self._dev_all = True
            self._dev_dirty.clear()

    def _device_records(self, device: torch.device, eng, stream: int) -> torch.Tensor:
        """The records in device memory, brought up to date on `stream`.

        The device copy differs from the host records in one field: the tail
        page's record keeps the page's capacity as its used count, so tokens
        appended to the tail need no upload (the kernel caps each page at the
        tokens its sequence holds); only new pages and pages that moved tier
        are uploaded."""
        n = len(self.pages)
        rb = _native.PAGE_DTYPE.itemsize
        if self._dev is None or self._dev.device != device or self._dev.numel() < n * rb:
            old = self._dev
            cap = max(n, 64, 2 * (old.numel() // rb if old is not None else 0))
            self._dev = torch.empty(cap * rb, dtype=torch.uint8, device=device)
            if old is not None and old.device == device:
                self._dev[:old.numel()].copy_(old)
            else:
                self._dev_all = True
        if self._dev_all:
            self._dev_all = False
            self._dev_dirty.clear()
            runs = [(0, n)] if n else []
        elif self._dev_dirty:
            idx = np.unique(np.asarray(self._dev_dirty, dtype=np.int64))
            self._dev_dirty.clear()
            idx = idx[(idx >= 0) & (idx < n)]
            cut = np.flatnonzero(np.diff(idx) != 1) + 1
            runs = [(int(r[0]), int(r[-1]) + 1) for r in np.split(idx, cut) if len(r)]
        else:
            return self._dev
        base = self._dev.data_ptr()
        for lo, hi in runs:
            chunk = self._rec[lo:hi].copy()
            if hi == n:
                chunk["used"][-1] = max(int(chunk["used"][-1]), self.tail_page.capacity_tokens)
            _native.call("helm_upload", eng, base + lo * rb, _native.ptr(chunk),
                         (hi - lo) * rb, stream)
        return self._dev

    def total_tokens_recorded(self) -> int:
        """Tokens in the layer's records (its active pages)."""
        n = len(self.pages)
        if n == 0:
            return 0
        last = self._rec[n - 1]
        return int(last["tok_off"]) + int(last["used"])

    def records(self):
        """The pages' ``helm_page`` records in token order (a view), or None
        (validated first in the validation mode: ``check_records``)."""
        if not self._rec_ok:
            return None
        if check_records_enabled():
            self.check_records()
        return self._rec[:len(self.pages)]

    def check_records(self, device: Optional[torch.device] = None) -> None:
        """Validation mode (``HELM_AMD_CHECK_RECORDS=1`` runs it before every
        launch that reads this layer's records): every record must describe
        its page as the page is now — K/V addresses and head stride of the
        page's tensors, its used tokens, the running token offset, the host
        flag of its device — and every byte the kernel may read through it
        (Hkv heads x the page's capacity x D) must lie inside the page
        tensors' own storage.  With `device`, the device-resident copy is
        read back and must equal the host records (the tail record carrying
        the tail page's capacity).  Raises RuntimeError naming the layer,
        page and field; launches nothing."""
        n = len(self.pages)
        if not self._rec_ok:
            raise RuntimeError(f"layer {self.layer_id}: records disabled (a page the kernel "
                               "cannot read in place)")
        rec = self._rec[:n]
        off = 0
        for i, page in enumerate(self.pages):
            where = f"layer {self.layer_id} page {i} (id {page.page_id})"
            fields = _page_record_fields(page)
            if fields is None:
                raise RuntimeError(f"{where}: not readable in place")
            r = rec[i]
            want = {"k": fields[0], "v": fields[1], "head_stride": fields[2],
                    "used": page.used_tokens, "tok_off": off,
                    "flags": _native.HELM_PAGE_HOST if fields[3] else 0}
            for name, value in want.items():
                if int(r[name]) != int(value):
                    raise RuntimeError(f"{where}: record {name} = {int(r[name])}, "
                                       f"page has {int(value)}")
            off += page.used_tokens
            k, v = page.k_tensor, page.v_tensor
            es = k.element_size()
            span = ((k.size(1) - 1) * k.stride(1) + max(page.capacity_tokens, page.used_tokens)
                    * k.size(3)) * es
            for name, t, addr in (("k", k, fields[0]), ("v", v, fields[1])):
                st = t.untyped_storage()
                lo, hi = st.data_ptr(), st.data_ptr() + st.nbytes()
                if not (lo <= addr and addr + span <= hi):
                    raise RuntimeError(f"{where}: {name} reads [{addr:#x}, {addr + span:#x}) "
                                       f"outside its storage [{lo:#x}, {hi:#x})")
        if off != self.total_tokens_recorded():
            raise RuntimeError(f"layer {self.layer_id}: token offsets end at "
                               f"{self.total_tokens_recorded()}, pages hold {off}")
        if device is not None and n:
            if self._dev is None or self._dev_all or self._dev_dirty:
                raise RuntimeError(f"layer {self.layer_id}: device records not uploaded")
            rb = _native.PAGE_DTYPE.itemsize
            dev = self._dev[:n * rb].cpu().numpy().view(_native.PAGE_DTYPE)
            host = rec.copy()
            host["used"][-1] = max(int(host["used"][-1]), self.tail_page.capacity_tokens)
            bad = np.flatnonzero(dev != host)
            if len(bad):
                raise RuntimeError(f"layer {self.layer_id}: device record {int(bad[0])} differs "
                                   f"from the host record ({dev[bad[0]]} vs {host[bad[0]]})")


_ENV_DATA = getattr(os.environ, "_data", None)
_ENV_KEYS: dict = {}


def _env_get(name: str) -> Optional[str]:
    """``os.environ.get(name)`` for the switches read on every decode call,
    without its per-call key encoding: CPython's ``os.environ`` keeps its
    entries (every set and delete goes through it) in the ``_data`` dict
    under encoded keys, so a miss, the common case, is one dict lookup."""
    if _ENV_DATA is None:
        return os.environ.get(name)
    key = _ENV_KEYS.get(name)
    if key is None:
        key = _ENV_KEYS[name] = os.environ.encodekey(name)
    v = _ENV_DATA.get(key)
    return None if v is None else os.environ.decodevalue(v)


def check_records_enabled() -> bool:
    """``HELM_AMD_CHECK_RECORDS`` set (to anything but 0): every launch that
    reads layer records validates them first (``LayerKVCache.check_records``)."""
    v = _env_get("HELM_AMD_CHECK_RECORDS")
    return bool(v) and v != "0"


def _used_bytes(page: KVPage) -> int:
    """K+V bytes of the used tokens of a [1, Hkv, P, D] page."""
    k = page.k_tensor
    if k.dim() != 4:
        return 0
    return page.used_tokens * k.size(0) * k.size(1) * k.size(3) * k.element_size() * 2


class _LayerPages(list):
    """What ``iterate_layer_pages`` returns: a shallow copy of a layer's page
    list (kv_cache.py:173-177) that also remembers the layer and the layer's
    page generation.  While the layer's pages are unchanged and the list has
    not been modified, ``perform_streaming_attention`` attends through the
    layer's records instead of reading every page in Python; any in-place
    change to the list drops that link (the list is then an ordinary list)."""

    __slots__ = ("_layer", "_gen")

    def __init__(self, layer: LayerKVCache):
        super().__init__(layer.pages)
        self._layer = layer
        self._gen = layer._gen

    def _live_layer(self) -> Optional[LayerKVCache]:
        layer = self._layer
        if layer is None or layer._gen != self._gen or len(layer.pages) != len(self):
            return None
        return layer


def _detaching(name):
    base = getattr(list, name)

    def method(self, *args, **kwargs):
        self._layer = None
        return base(self, *args, **kwargs)
    method.__name__ = name
    return method


for _name in ("append", "extend", "insert", "pop", "remove", "clear", "sort", "reverse",
              "__setitem__", "__delitem__", "__iadd__", "__imul__"):
    setattr(_LayerPages, _name, _detaching(_name))
del _name


# ── token writes ───────────────────────────────────────────────────────────────
class _AppendQueue:
    """Token writes into device pages, flushed as one helm_page_append launch."""

    def __init__(self):
        self.rows = []
        self.keep = []          # source tensors alive until the launch is queued
        self.device = None
        self.dtype = None
        self.hkv = 0
        self.d = 0
        self._segs = np.zeros(8, dtype=_native.APPEND_DTYPE)   # reused between flushes
        self._segs_addr = self._segs.ctypes.data

    def add(self, dst_k: torch.Tensor, dst_v: torch.Tensor, dst_tok: int, K: torch.Tensor,
            V: torch.Tensor) -> None:
        n = K.size(2)
        if n == 0:
            return
        if K.dtype != dst_k.dtype:
            K = K.to(dst_k.dtype)
        if V.dtype != dst_v.dtype:
            V = V.to(dst_v.dtype)
        if K.stride(3) != 1 or V.stride(3) != 1 or K.stride()[1:] != V.stride()[1:]:
            K, V = K.contiguous(), V.contiguous()
        if dst_k.stride(1) != dst_v.stride(1) or dst_k.stride(2) != dst_k.size(3):
            raise ValueError("destination page tensors must be [1, Hkv, P, D] with dense rows")
        key = (K.device, dst_k.dtype, dst_k.size(1), dst_k.size(3))
        if self.rows and key != (self.device, self.dtype, self.hkv, self.d):
            self.flush()
        self.device, self.dtype, self.hkv, self.d = key
        self.rows.append((dst_k.data_ptr(), dst_v.data_ptr(), K.data_ptr(), V.data_ptr(),
                          K.stride(1), K.stride(2), dst_k.stride(1), dst_tok, n, 0))
        self.keep.append((K, V))

    def flush(self) -> None:
        n = len(self.rows)
        if not n:
            return
        if n > len(self._segs):
            self._segs = np.zeros(max(n, 2 * len(self._segs)), dtype=_native.APPEND_DTYPE)
            self._segs_addr = self._segs.ctypes.data
        segs = self._segs
        for i, row in enumerate(self.rows):
            segs[i] = row
        rc = _native.entry("helm_page_append")(self._segs_addr, n, self.hkv, self.d,
                                               _native.dtype_code(self.dtype),
                                               _engine.stream_ptr(self.device))
        if rc:
            _native.check("helm_page_append", rc)
        self.rows.clear()
        self.keep.clear()


def _write_tokens(queue: _AppendQueue, page: KVPage, dst_tok: int, K: torch.Tensor,
                  V: torch.Tensor) -> None:
    n = K.size(2)
    if page.device.type == "cuda" and K.device.type == "cuda" and V.device.type == "cuda":
        queue.add(page.k_tensor, page.v_tensor, dst_tok, K, V)
    else:
        queue.flush()
        page.k_tensor[:, :, dst_tok:dst_tok + n, :].copy_(K)
        page.v_tensor[:, :, dst_tok:dst_tok + n, :].copy_(V)


def _evict_sync() -> bool:
    return not bool(os.environ.get("HELM_AMD_ASYNC_EVICT"))


# ── cache manager (kv_cache.py:88-376) ─────────────────────────────────────────
class KVCacheManager:
    """Owns every layer's pages: appends, residency watermark, eviction.

    HELM totals the evictable GPU bytes by scanning every layer's pages after
    each appended page, and sorts them to pick victims (kv_cache.py:179-235).
    Here the evictable pages (GPU-resident, full, not a tail) are kept in a
    heap ordered as HELM's stable sort orders them (start token, then layer
    order, then page order) with their bytes as a running total, so the policy
    check is O(1) and an eviction costs O(log n) per page moved.  The heap
    follows the pages as this manager changes them; when ``layers`` itself is
    changed from outside (a layer deleted or replaced) it is rebuilt from a
    full scan.
    """

    def __init__(self, allocator, gpu_high_watermark_bytes: int = 512 * 1024 * 1024):
        self.allocator = allocator
        self.layers = {}
        self.gpu_high_watermark_bytes = gpu_high_watermark_bytes
        self.cont_K: dict = {}
        self.cont_V: dict = {}
        self._cont: Optional[ContiguousKV] = None
        self.cont_capacity: int = 0
        self.cont_num_layers: int = 0
        self.cont_seq_len: int = 0
        self.cont_prefill_len: int = 0
        self.use_contiguous: bool = False
        self._appends = _AppendQueue()
        # evictable pages: (start_token, layer order, page index, seq, layer, page, bytes)
        self._evq: list = []
        self._ev_bytes = 0
        self._ev_seq = 0
        self._seen: dict = {}        # the `layers` mapping the heap was built for
        self._order: dict = {}       # id(layer) -> the layer's place in `layers`
        self._next_order = 0

    def initialize_layer_caches(self, num_layers: int):
        for i in range(num_layers):
            self.layers[i] = LayerKVCache(layer_id=i)
        self._resync()

    # ── evictable-page bookkeeping ──────────────────────────────────────────
    @staticmethod
    def _is_evictable(page: KVPage, tail: Optional[KVPage]) -> bool:
        return (page.state == 'GPU' and page.device.type == 'cuda' and page is not tail
                and page.used_tokens == page.capacity_tokens)

    def _push_evictable(self, layer: LayerKVCache, idx: int, page: KVPage) -> None:
        nb = _page_bytes(page)
        heapq.heappush(self._evq, (page.start_token, self._order[id(layer)], idx, self._ev_seq,
                                   layer, page, nb))
        self._ev_seq += 1
        self._ev_bytes += nb

    def _resync(self) -> None:
        """Rebuilds the evictable-page heap from a scan of every layer."""
        self._evq, self._ev_bytes, self._ev_seq = [], 0, 0
        self._order, self._next_order = {}, 0
        for layer in self.layers.values():
            self._order[id(layer)] = self._next_order
            self._next_order += 1
            tail = layer.tail_page
            for idx, page in enumerate(layer.pages):
                if self._is_evictable(page, tail):
                    self._push_evictable(layer, idx, page)
        self._seen = dict(self.layers)

    def _sync_layers(self) -> None:
        if self.layers != self._seen:
            self._resync()

    def _layer(self, layer_id: int) -> LayerKVCache:
        self._sync_layers()
        layer = self.layers.get(layer_id)
        if layer is None:
            layer = self.layers[layer_id] = LayerKVCache(layer_id)
            self._seen[layer_id] = layer
            self._order[id(layer)] = self._next_order
            self._next_order += 1
        return layer

    def _add_page(self, layer: LayerKVCache, page: KVPage) -> None:
        """Appends `page` as the new tail; the old tail may become evictable."""
        old = layer.tail_page
        layer.append_page(page)
        idx = len(layer.pages) - 2
        if old is not None and idx >= 0 and layer.pages[idx] is old and \
                self._is_evictable(old, page):
            self._push_evictable(layer, idx, old)

    # ── appends ──────────────────────────────────────────────────────────────
    def append_prefill(self, layer_id: int, K_prefill: torch.Tensor, V_prefill: torch.Tensor):
        """Split a [1,Hkv,S,D] chunk into page-sized blocks, each a new page
        starting at the layer's running token count; the residency policy runs
        after every page (kv_cache.py:113-143)."""
        layer = self._layer(layer_id)
        seq_len = K_prefill.size(2)
        page_size = self.allocator.page_size
        device = K_prefill.device
        try:
            for start_idx in range(0, seq_len, page_size):
                chunk_len = min(page_size, seq_len - start_idx)
                end_idx = start_idx + chunk_len
                page = self.allocator.allocate(device)
                page.layer_id = layer_id
                page.start_token = layer.total_tokens
                page.used_tokens = chunk_len
                _write_tokens(self._appends, page, 0, K_prefill[:, :, start_idx:end_idx, :],
                              V_prefill[:, :, start_idx:end_idx, :])
                self._add_page(layer, page)
                layer.total_tokens += chunk_len
                self._enforce_residency_policy()
        finally:
            self._appends.flush()

    def append_decode(self, layer_id: int, K_new: torch.Tensor, V_new: torch.Tensor,
                      skip_residency: bool = False):
        """Append one token; a new page when the tail is missing or full
        (kv_cache.py:145-171)."""
        self._append_decode_deferred(layer_id, K_new, V_new)
        self._appends.flush()
        if not skip_residency:
            self._enforce_residency_policy()

    def _append_decode_deferred(self, layer_id: int, K_new: torch.Tensor, V_new: torch.Tensor):
        page, tok = self._decode_slot(layer_id, K_new.device)
        _write_tokens(self._appends, page, tok, K_new, V_new)

    def _decode_slot(self, layer_id: int, device: torch.device):
        """The page and token index of one decoded token, with append_decode's
        bookkeeping (a new page when the tail is missing or full, used and
        total counts, kv_cache.py:145-171); the caller writes the token."""
        layer = self._layer(layer_id)
        if layer.tail_page is None or layer.tail_page.used_tokens == layer.tail_page.capacity_tokens:
            page = self.allocator.allocate(device)
            page.layer_id = layer_id
            page.start_token = layer.total_tokens
            page.used_tokens = 0
            self._add_page(layer, page)
        page = layer.tail_page
        tok = page.used_tokens
        page.used_tokens += 1
        layer.total_tokens += 1
        layer._tail_filled()
        return page, tok

    def iterate_layer_pages(self, layer_id: int):
        if layer_id not in self.layers:
            return []
        return _LayerPages(self.layers[layer_id])

    def _evictable(self):
        """(layer, page) pairs HELM may evict: GPU-resident, full, not a tail
        (kv_cache.py:184-192), in layer then page order."""
        out = []
        for layer in self.layers.values():
            tail = layer.tail_page
            for page in layer.pages:
                if self._is_evictable(page, tail):
                    out.append((layer, page))
        return out

    def evict_pages(self, bytes_to_evict: int):
        """Oldest-first (by start_token) eviction of at least `bytes_to_evict`
        bytes of full, non-tail GPU pages to host (kv_cache.py:179-222)."""
        if bytes_to_evict <= 0:
            return
        self._appends.flush()
        self._sync_layers()
        chosen, evicted_bytes = [], 0
        while self._evq and evicted_bytes < bytes_to_evict:
            _, _, idx, _, layer, page, nb = heapq.heappop(self._evq)
            self._ev_bytes -= nb
            if not (idx < len(layer.pages) and layer.pages[idx] is page
                    and self._is_evictable(page, layer.tail_page)):
                continue            # changed since it was queued
            chosen.append((layer, idx, page))
            evicted_bytes += nb
        if not chosen:
            _record_eviction(0, 0)
            return
        new_pages = self.allocator.move_pages([p for _, _, p in chosen], torch.device('cpu'),
                                              sync=_evict_sync())
        moved_bytes = 0
        for (layer, idx, page), new_page in zip(chosen, new_pages):
            assert new_page.start_token == page.start_token, "Page invariant broken during migration"
            layer._replace_page(idx, new_page)
            moved_bytes += _page_bytes(new_page)
        _record_eviction(len(new_pages), moved_bytes)

    def _enforce_residency_policy(self):
        """Evict the excess of evictable GPU bytes over the watermark
        (kv_cache.py:224-235)."""
        self._sync_layers()
        if self._ev_bytes > self.gpu_high_watermark_bytes:
            self.evict_pages(self._ev_bytes - self.gpu_high_watermark_bytes)

    def seq_len(self):
        if 0 in self.layers:
            return self.layers[0].total_tokens
        return 0

    def num_layers(self):
        return len(self.layers)

    def clear(self):
        self._appends.flush()
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state != 'DEAD':
                    self.allocator.free(page)
            layer._reset()
        self.layers.clear()
        self._resync()

    def all_gpu_resident(self, layer_id: int) -> bool:
        if layer_id not in self.layers:
            return True
        for page in self.layers[layer_id].pages:
            if page.used_tokens > 0 and page.state != 'GPU':
                return False
        return True

    # ── contiguous fast path (kv_cache.py:267-354) ──────────────────────────
    # The buffers live in one ContiguousKV arena per manager; cont_K / cont_V
    # are HELM's per-layer [1, Hkv, capacity, D] views into it.
    def build_contiguous(self, num_layers: int, num_kv_heads: int, head_dim: int,
                         capacity: int, device: torch.device, dtype: torch.dtype) -> bool:
        """Reserves the contiguous buffers of every layer; on an allocation
        failure the capacity halves down to min(capacity, 1024) tokens
        (kv_cache.py:269-299).  True with the capacity reached, else False
        with the fast path off."""
        self._cont = None
        self.cont_K, self.cont_V = {}, {}
        cont = ContiguousKV.allocate(num_layers, num_kv_heads, head_dim, capacity, device, dtype)
        self.use_contiguous = cont is not None
        if cont is None:
            return False
        self._cont = cont
        self.cont_capacity = cont.capacity
        self.cont_num_layers = num_layers
        self.cont_K = {lid: cont.k_view(lid) for lid in range(num_layers)}
        self.cont_V = {lid: cont.v_view(lid) for lid in range(num_layers)}
        return True

    def prefill_contiguous(self, layer_id: int, K: torch.Tensor, V: torch.Tensor):
        """The prompt's K/V also go to the buffers; layer 0 sets the lengths."""
        self._write_contiguous(layer_id, 0, K, V)
        if layer_id == 0:
            self.cont_prefill_len = self.cont_seq_len = K.shape[2]

    def write_decode_contiguous(self, layer_id: int, K_new: torch.Tensor, V_new: torch.Tensor):
        """One decoded token at position cont_seq_len of the layer's buffers."""
        self._write_contiguous(layer_id, self.cont_seq_len, K_new, V_new)

    def _write_contiguous(self, layer_id: int, at: int, K: torch.Tensor, V: torch.Tensor):
        self._queue_contiguous(layer_id, at, K, V)
        self._appends.flush()

    def _queue_contiguous(self, layer_id: int, at: int, K: torch.Tensor, V: torch.Tensor):
        dk, dv = self.cont_K[layer_id], self.cont_V[layer_id]
        if dk.device.type == "cuda" and K.device.type == "cuda":
            self._appends.add(dk, dv, at, K, V)
        else:
            self._appends.flush()
            dk[:, :, at:at + K.shape[2], :].copy_(K)
            dv[:, :, at:at + V.shape[2], :].copy_(V)

    def get_kv_contiguous(self, layer_id: int):
        """Views of the layer's tokens including the one being decoded."""
        n = self.cont_seq_len + 1
        return self.cont_K[layer_id][:, :, :n, :], self.cont_V[layer_id][:, :, :n, :]

    def advance_contiguous(self):
        """Commits the decoded token (once per step, after the last layer)."""
        self.cont_seq_len += 1

    def migrate_contiguous_to_pages(self):
        """The decoded tokens that only the buffers hold (cont_prefill_len ..
        cont_seq_len; the prompt went to pages at prefill) become pages of
        every layer, with the residency policy applied as append_prefill
        applies it; then the buffers are released (kv_cache.py:325-342)."""
        cont = self._cont
        if cont is None:
            return
        lo, hi = self.cont_prefill_len, self.cont_seq_len
        for lid in range(self.cont_num_layers if hi > lo else 0):
            self.append_prefill(lid, cont.k_view(lid)[:, :, lo:hi], cont.v_view(lid)[:, :, lo:hi])
        self.drop_contiguous()

    def drop_contiguous(self):
        """Releases the buffers; attention goes back to the pages."""
        self._appends.flush()
        self._cont = None
        self.cont_K, self.cont_V = {}, {}
        self.use_contiguous = False

    def reset_contiguous(self):
        """Re-arms kept buffers for the next request (kv_cache.py:351-354)."""
        if self._cont is not None:
            self.use_contiguous = True
            self.cont_seq_len = self.cont_prefill_len = 0

    def contiguous_records(self, layer_id: int):
        """(device address of the layer's contiguous-buffer records, whether
        every record is 16-byte aligned) — see ContiguousKV."""
        return self._cont.records_ptr(layer_id), self._cont.aligned16

    def layers_keys(self):
        return sorted(self.layers.keys())

    def report_bytes_per_tier(self) -> dict:
        """Whole-page K+V bytes of the GPU- and CPU-resident pages
        (kv_cache.py:356-375); DEAD placeholders count nowhere."""
        tally = {"GPU": 0, "CPU": 0}
        for layer in self.layers.values():
            for page in layer.pages:
                if page.state in tally:
                    tally[page.state] += _page_bytes(page)
        return {"gpu_active_bytes": tally["GPU"], "cpu_active_bytes": tally["CPU"]}


class ContiguousKV:
    """The contiguous cache of one sequence, HELM's Accelerate-style fast path
    (kv_cache.py:267-354), as one arena [layers, 2, Hkv, capacity, D]: layer
    l's K is arena[l, 0], its V arena[l, 1].

    The attention kernels read it as pages: each layer's buffer is cut into
    16-token virtual pages whose ``helm_page`` records are written to device
    memory once, when the arena is made.  A decode step passes those records
    and its token count to ``helm_paged_attn_seqs`` (the kernel stops at the
    token count), so nothing is built or uploaded per call."""

    BLOCK = 16

    def __init__(self, arena: torch.Tensor):
        self.arena = arena
        L, _, hkv, cap, d = arena.shape
        self.capacity = cap
        self.blocks = -(-cap // self.BLOCK)
        es = arena.element_size()
        self.aligned16 = (arena.data_ptr() % 16 == 0 and (arena.stride(1) * es) % 16 == 0
                          and (cap * d * es) % 16 == 0 and (self.BLOCK * d * es) % 16 == 0)
        self._rec = None
        if arena.device.type == "cuda":
            es = arena.element_size()
            t = np.arange(self.blocks, dtype=np.int64) * self.BLOCK
            rec = np.zeros((L, self.blocks), dtype=_native.PAGE_DTYPE)
            for lid in range(L):
                kb = arena[lid, 0].data_ptr()
                vb = arena[lid, 1].data_ptr()
                rec["k"][lid] = kb + t * d * es
                rec["v"][lid] = vb + t * d * es
            rec["used"] = np.minimum(self.BLOCK, cap - t)[None, :]
            rec["tok_off"] = t[None, :]
            rec["head_stride"] = cap * d
            self._rec = torch.from_numpy(rec.view(np.uint8).reshape(-1)).to(arena.device)

    @staticmethod
    def _new_arena(shape, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
        if shape[3] * shape[4] >= 1 << 31:
            raise ValueError("contiguous capacity x head_dim must stay below 2^31 elements")
        return torch.empty(shape, device=device, dtype=dtype)

    @classmethod
    def allocate(cls, num_layers: int, num_kv_heads: int, head_dim: int, capacity: int,
                 device: torch.device, dtype: torch.dtype) -> Optional["ContiguousKV"]:
        """An arena of `capacity` tokens or, where that allocation fails, of
        the first of capacity / 2, / 4, ... (not below min(capacity, 1024))
        that succeeds; None when none does."""
        floor = max(1, min(capacity, 1024))
        sizes = []
        while capacity >= floor:
            sizes.append(capacity)
            capacity //= 2
        for cap in sizes:
            try:
                return cls(cls._new_arena((num_layers, 2, num_kv_heads, cap, head_dim),
                                          device, dtype))
            except (torch.cuda.OutOfMemoryError, RuntimeError):
                if device.type == "cuda":
                    torch.cuda.empty_cache()
        return None

    def k_view(self, lid: int) -> torch.Tensor:
        return self.arena[lid, 0].unsqueeze(0)

    def v_view(self, lid: int) -> torch.Tensor:
        return self.arena[lid, 1].unsqueeze(0)

    def records_ptr(self, lid: int) -> int:
        return self._rec.data_ptr() + lid * self.blocks * _native.PAGE_DTYPE.itemsize


# ── copy stream (kv_cache.py:383-396) ──────────────────────────────────────────
def _get_kv_copy_stream(device: torch.device) -> torch.cuda.Stream:
    """The per-device side stream of the native engine (memoized per device)."""
    return _engine.copy_stream(device)


def _async_kv_prefetch_enabled() -> bool:
    """HELM_DISABLE_ASYNC_KV gates the overlapped prefetch (ablations)."""
    return not bool(_env_get("HELM_DISABLE_ASYNC_KV"))


# ── native attention ────────────────────────────────────────────────────────────
class _Segment:
    """A run of tokens of one sequence as the kernel sees it."""
    __slots__ = ("k", "v", "used", "head_stride", "host", "keep")

    def __init__(self, k, v, used, head_stride, host, keep=None):
        self.k, self.v, self.used, self.head_stride, self.host, self.keep = (
            k, v, used, head_stride, host, keep)


def _page_segments(page: KVPage, b: int, B: int, Hkv: int, D: int, dtype) -> _Segment:
    k, v = page.k_tensor, page.v_tensor
    if k.dim() != 4 or v.shape != k.shape:
        raise ValueError("page tensors must be [batch, Hkv, P, D] and K/V alike")
    if k.size(1) != Hkv or k.size(3) != D:
        raise ValueError(f"page shape {tuple(k.shape)} does not match Hkv={Hkv}, D={D}")
    if k.dtype != dtype or v.dtype != dtype:
        raise TypeError("all pages of one attention call must share one dtype")
    if k.size(0) not in (1, B):
        raise ValueError(f"page batch {k.size(0)} does not match query batch {B}")
    if (k.stride(3) != 1 or k.stride(2) != D or v.stride(3) != 1 or v.stride(2) != D
            or v.stride(1) != k.stride(1)):
        k, v = k.contiguous(), v.contiguous()
    bb = b if k.size(0) > 1 else 0
    es = k.element_size()
    return _Segment(k.data_ptr() + bb * k.stride(0) * es, v.data_ptr() + bb * v.stride(0) * es,
                    page.used_tokens, k.stride(1), k.device.type != "cuda", (k, v))


def _contiguous_segments(K: torch.Tensor, V: torch.Tensor, b: int, block: int = 16):
    """[B,Hkv,n,D] contiguous-cache views as 16-token virtual pages."""
    n = K.size(2)
    es = K.element_size()
    bb = b if K.size(0) > 1 else 0
    kb = K.data_ptr() + bb * K.stride(0) * es
    vb = V.data_ptr() + bb * V.stride(0) * es
    segs = []
    for t in range(0, n, block):
        segs.append(_Segment(kb + t * K.stride(2) * es, vb + t * V.stride(2) * es,
                             min(block, n - t), K.stride(1), False, None))
    return segs


def _attend(query: torch.Tensor, seqs: Sequence[Sequence[_Segment]], Hkv: int, kv_dtype,
            scale: float, attention_mask: Optional[torch.Tensor], softcap: Optional[float],
            causal: int) -> torch.Tensor:
    """One helm_stream_attn call: query [B,Hq,S,D], seqs[b] = ordered segments.
    causal = c > 0: query position s sees keys 0 .. s + c - 1 (c = 1: top-left)."""
    B = query.size(0)
    n = sum(len(s) for s in seqs)
    arr = np.zeros(n, dtype=_native.PAGE_DTYPE)
    seq_off = np.zeros(B + 1, dtype=np.int32)
    i = 0
    t_max = 0
    # causal: keys from q_len + c - 1 on are masked for every row and their
    # pages need not be read
    limit = query.size(2) + int(causal) - 1 if causal else None
    for b, segs in enumerate(seqs):
        tok = 0
        for sg in segs:
            if limit is not None and tok >= limit:
                break
            used = sg.used if limit is None else min(sg.used, limit - tok)
            arr[i] = (sg.k, sg.v, used, tok, sg.head_stride,
                      _native.HELM_PAGE_HOST if sg.host else 0)
            tok += used
            i += 1
        seq_off[b + 1] = i
        t_max = max(t_max, tok)
    return _attend_records(query, arr, seq_off, t_max, Hkv, kv_dtype, scale, attention_mask,
                           softcap, causal)


# fp32 copies of additive masks that a kernel cannot read as given (a mask on
# another device, or a CPU query's 16-bit mask: the host-CPU kernel reads
# fp32), one per mask object: HELM's pipeline builds one decode mask per step
# in the model's dtype (pipeline_runtime.py:79-92) and hands that object to
# every layer, so it is converted once per step, not once per layer.  An entry
# is dropped when its mask is freed; it is used only while the mask's address,
# shape, strides, dtype, version counter and the target device are unchanged.
# A tensor made under torch.inference_mode() has no version counter (HELM's
# generate runs there, inference.py:747): an in-place change to it cannot be
# seen, so such a mask is converted on every call.  The copies kept at once
# are bounded; past the bound a mask converts per call.
_F32_MASKS: dict = {}
_F32_MASK_MAX_ELEMS = 1 << 26      # one mask
_F32_MASK_MAX_TOTAL = 1 << 28      # all copies kept (elements, 1 GiB of fp32)


def _mask_fp32(m: torch.Tensor, device: torch.device) -> torch.Tensor:
    if m.numel() > _F32_MASK_MAX_ELEMS or m.is_inference():
        return m.to(device=device, dtype=torch.float32)
    key = id(m)
    sig = (m.data_ptr(), tuple(m.shape), tuple(m.stride()), m.dtype, m._version, device)
    ent = _F32_MASKS.get(key)
    if ent is not None and ent[0]() is m and ent[1] == sig:
        return ent[2]
    f = m.to(device=device, dtype=torch.float32)
    if ent is not None:
        del _F32_MASKS[key]
    if sum(e[2].numel() for e in _F32_MASKS.values()) + f.numel() <= _F32_MASK_MAX_TOTAL:
        _F32_MASKS[key] = (weakref.ref(m, lambda _r, k=key: _F32_MASKS.pop(k, None)), sig, f)
    return f


# mask element types the GPU kernels read as given (HELM_F32 / BF16 / F16)
_MASK_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


def _query_and_mask(query: torch.Tensor, Hkv: int, kv_dtype, t_max: int,
                    attention_mask: Optional[torch.Tensor], gpu: bool = True):
    """The query in a kernel dtype, its output buffer and the mask arguments
    (pointer, batch / head / row strides, and for a GPU call the element type)
    of one attention call.  A GPU call reads a mask on the query's device in
    fp32, bf16 or fp16 as given; the host-CPU kernel reads fp32."""
    device = query.device
    B, Hq, S, D = query.shape
    if Hq % Hkv != 0:
        raise ValueError(f"num_q_heads {Hq} is not a multiple of num_kv_heads {Hkv}")
    q = query
    if q.dtype != kv_dtype and q.dtype != torch.float32:
        q = q.float()
    if not q.is_contiguous():
        q = q.contiguous()
    out = torch.empty_like(q)
    mask_ptr, mbs, mhs, mqs = None, 0, 0, 0
    mdt = _native.HELM_F32
    m = None
    if attention_mask is not None:
        m = attention_mask
        if m.device != device or (m.dtype != torch.float32 and
                                  (not gpu or m.dtype not in _MASK_NATIVE)):
            m = _mask_fp32(m, device)
        if m.dim() != 4:
            raise ValueError("attention_mask must be 4-D [B, H, q_len, kv_len]")
        Bm, Hm, Sm, Tm = m.shape
        if Bm not in (1, B) or Hm not in (1, Hq) or Sm not in (1, S):
            raise ValueError(f"attention_mask shape {tuple(m.shape)} does not broadcast to "
                             f"[{B}, {Hq}, {S}, kv_len]")
        if Tm < t_max:
            if Tm != 1:
                raise ValueError(f"attention_mask covers {Tm} keys, the pages hold {t_max}")
            m = m.expand(Bm, Hm, Sm, t_max)
        if m.stride(3) != 1:
            m = m.contiguous()
        mask_ptr = m.data_ptr()
        mbs = m.stride(0) if Bm > 1 else 0
        mhs = m.stride(1) if Hm > 1 else 0
        mqs = m.stride(2) if Sm > 1 else 0
        mdt = _native.dtype_code(m.dtype)
    margs = (mask_ptr, mbs, mhs, mqs, mdt) if gpu else (mask_ptr, mbs, mhs, mqs)
    return q, out, margs, m


def _attend_records(query: torch.Tensor, arr: np.ndarray, seq_off: np.ndarray, t_max: int,
                    Hkv: int, kv_dtype, scale: float, attention_mask: Optional[torch.Tensor],
                    softcap: Optional[float], causal: int) -> torch.Tensor:
    """One helm_stream_attn call over prepared ``helm_page`` records: sequence
    b owns records seq_off[b]:seq_off[b+1] (token offsets per sequence), the
    longest sequence holds t_max tokens."""
    device = query.device
    if device.type != "cuda":
        return _attend_records_cpu(query, arr, seq_off, t_max, Hkv, kv_dtype, scale,
                                   attention_mask, softcap, causal)
    B, Hq, S, D = query.shape
    q, out, margs, _keep = _query_and_mask(query, Hkv, kv_dtype, t_max, attention_mask)
    n = int(seq_off[B])
    _native.call("helm_stream_attn", _engine.get_engine(device), q.data_ptr(), out.data_ptr(),
                 B, Hq, Hkv, S, D, _native.ptr(arr) if n else None, _native.ptr(seq_off),
                 float(scale), float(softcap) if softcap is not None else 0.0, *margs,
                 int(causal), _native.dtype_code(kv_dtype), _native.dtype_code(q.dtype),
                 _engine.stream_ptr(device))
    return out if out.dtype == query.dtype else out.to(query.dtype)


def _attend_records_cpu(query: torch.Tensor, arr: np.ndarray, seq_off: np.ndarray, t_max: int,
                        Hkv: int, kv_dtype, scale: float, attention_mask: Optional[torch.Tensor],
                        softcap: Optional[float], causal: int) -> torch.Tensor:
    """``_attend_records`` for a query on the CPU: one helm_cpu_stream_attn
    call (libhelm_cpu.so) over records whose pages are in host memory, on
    torch's intra-op thread count."""
    B, Hq, S, D = query.shape
    q, out, margs, _keep = _query_and_mask(query, Hkv, kv_dtype, t_max, attention_mask,
                                           gpu=False)
    n = int(seq_off[B])
    _cpu_native.call("helm_cpu_stream_attn", q.data_ptr(), out.data_ptr(), B, Hq, Hkv, S, D,
                     _native.ptr(arr) if n else None, _native.ptr(seq_off), float(scale),
                     float(softcap) if softcap is not None else 0.0, *margs, int(causal),
                     _native.dtype_code(kv_dtype), _native.dtype_code(q.dtype),
                     torch.get_num_threads())
    return out if out.dtype == query.dtype else out.to(query.dtype)


_tls = threading.local()


def _seq_args(B: int):
    """This thread's (record pointers, page counts, token counts) argument
    arrays for a call over B sequences — views of arrays kept between calls
    (the native call reads them before it returns) — and their addresses."""
    a = getattr(_tls, "seq_args", None)
    if a is None or len(a[0]) < B:
        n = max(16, B)
        arrs = (np.zeros(n, np.uint64), np.zeros(n, np.int32), np.zeros(n, np.int32))
        a = _tls.seq_args = arrs + (tuple(x.ctypes.data for x in arrs),)
    return a[0][:B], a[1][:B], a[2][:B], a[3]


def _attend_layers(query: torch.Tensor, layers: Sequence[LayerKVCache], lens: Sequence[int],
                   Hkv: int, kv_dtype, scale: float, attention_mask: Optional[torch.Tensor],
                   softcap: Optional[float], causal: int, tokens_app: Optional[int] = None):
    """One helm_paged_attn_seqs call: sequence b is layers[b]'s pages, read
    through the layer's device-resident records (uploaded only where they
    changed); lens[b] tokens.  Every page must be device-resident.

    tokens_app: host address of B helm_append_seg rows, each sequence's new
    decode token, which the call then also writes into the last page
    (helm_paged_attn_seqs_append); returns None, with nothing launched, when
    that call cannot take them (the caller writes them and calls again)."""
    device = query.device
    eng = _engine.get_engine(device)
    stream = _engine.stream_ptr(device)
    B = len(layers)
    if tokens_app is not None and (B > _MAX_SEQS or causal or query.size(2) != 1
                                   or query.size(3) != 128 or query.dtype != kv_dtype):
        return None
    ptrs, npages, tokens, addrs = _seq_args(B)
    page_tokens, aligned, t_max = 0, True, 0
    for b, layer in enumerate(layers):
        ptrs[b] = layer._device_records(device, eng, stream).data_ptr()
        npages[b] = len(layer.pages)
        n = lens[b]
        tokens[b] = n
        if n > t_max:
            t_max = n
        if layer._page_tokens > page_tokens:
            page_tokens = layer._page_tokens
        aligned = aligned and layer._aligned16
    if check_records_enabled():
        for layer in layers:
            layer.check_records(device)
    if causal:
        # causal c: keys from S + c - 1 on are masked for every row; the pages
        # holding only such keys are left out (records are in token order)
        limit = query.size(2) + int(causal) - 1
        t_max = min(t_max, limit)
        for b, layer in enumerate(layers):
            if tokens[b] > limit:
                tokens[b] = limit
                npages[b] = int(np.searchsorted(layer._rec["tok_off"][:npages[b]], limit,
                                                "left"))
    if tokens_app is not None:
        return _launch_seqs(query, addrs, int(t_max), page_tokens, aligned, Hkv, kv_dtype,
                            scale, attention_mask, softcap, causal, tokens_app=tokens_app)
    if B <= _MAX_SEQS:
        return _launch_seqs(query, addrs, int(t_max), page_tokens, aligned, Hkv, kv_dtype,
                            scale, attention_mask, softcap, causal)
    return _attend_device_records(query, ptrs, npages, tokens, page_tokens, aligned, Hkv,
                                  kv_dtype, scale, attention_mask, softcap, causal)


def _attend_device_records(query: torch.Tensor, ptrs: np.ndarray, npages: np.ndarray,
                           tokens: np.ndarray, page_tokens: int, aligned: bool, Hkv: int,
                           kv_dtype, scale: float, attention_mask: Optional[torch.Tensor],
                           softcap: Optional[float], causal: int) -> torch.Tensor:
    """helm_paged_attn_seqs over record arrays already in device memory:
    sequence b reads npages[b] records at ptrs[b] (token order), tokens[b]
    tokens; at most 16 sequences per call (more are issued in groups)."""
    B = query.size(0)
    if B > _MAX_SEQS:
        outs = []
        for b0 in range(0, B, _MAX_SEQS):
            m = attention_mask
            if m is not None and m.size(0) > 1:
                m = m[b0:b0 + _MAX_SEQS]
            outs.append(_attend_device_records(
                query[b0:b0 + _MAX_SEQS], ptrs[b0:b0 + _MAX_SEQS], npages[b0:b0 + _MAX_SEQS],
                tokens[b0:b0 + _MAX_SEQS], page_tokens, aligned, Hkv, kv_dtype, scale, m,
                softcap, causal))
        return torch.cat(outs, 0)
    t_max = int(tokens[0]) if B == 1 else int(tokens.max())
    if ptrs.dtype != np.uint64 or not ptrs.flags["C_CONTIGUOUS"]:
        ptrs = np.ascontiguousarray(ptrs, dtype=np.uint64)
    if npages.dtype != np.int32 or not npages.flags["C_CONTIGUOUS"]:
        npages = np.ascontiguousarray(npages, dtype=np.int32)
    if tokens.dtype != np.int32 or not tokens.flags["C_CONTIGUOUS"]:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    return _launch_seqs(query, (_native.ptr(ptrs), _native.ptr(npages), _native.ptr(tokens)),
                        t_max, page_tokens, aligned, Hkv, kv_dtype, scale, attention_mask,
                        softcap, causal, (ptrs, npages, tokens))


_MAX_SEQS = 16     # sequences one helm_paged_attn_seqs call carries


def _launch_seqs(query: torch.Tensor, addrs, t_max: int, page_tokens: int, aligned: bool,
                 Hkv: int, kv_dtype, scale: float, attention_mask: Optional[torch.Tensor],
                 softcap: Optional[float], causal: int, _keep_args=None,
                 tokens_app: Optional[int] = None):
    """The helm_paged_attn_seqs call itself: `addrs` = host addresses of the
    B record pointers, page counts and token counts (B <= 16).  With
    tokens_app (decode, q in the KV dtype) helm_paged_attn_seqs_append, or
    None when it does not take the call (nothing launched)."""
    device = query.device
    B, Hq, S, D = query.shape
    q, out, margs, _keep = _query_and_mask(query, Hkv, kv_dtype, t_max, attention_mask)
    if tokens_app is not None:
        rc = _native.entry("helm_paged_attn_seqs_append")(
            _engine.get_engine(device), q.data_ptr(), out.data_ptr(), B, Hq, Hkv, D, addrs[0],
            addrs[1], addrs[2], page_tokens, 1 if aligned else 0, float(scale),
            float(softcap) if softcap is not None else 0.0, *margs,
            _native.dtype_code(kv_dtype), tokens_app, _engine.stream_ptr(device))
        if rc == _native.HELM_E_UNSUPPORTED:
            return None
        if rc:
            _native.check("helm_paged_attn_seqs_append", rc)
        return out
    rc = _native.entry("helm_paged_attn_seqs")(
        _engine.get_engine(device), q.data_ptr(), out.data_ptr(), B, Hq, Hkv, S, D,
        addrs[0], addrs[1], addrs[2], page_tokens, 1 if aligned else 0, float(scale),
        float(softcap) if softcap is not None else 0.0, *margs, int(causal),
        _native.dtype_code(kv_dtype), _native.dtype_code(q.dtype), _engine.stream_ptr(device))
    if rc:
        _native.check("helm_paged_attn_seqs", rc)
    return out if out.dtype == query.dtype else out.to(query.dtype)


# helm_decode_args (include/helm_amd.h) written with precompiled structs:
# q, out, mask, stream and the mask strides; the per-sequence arrays; B ..
# pad, scale, softcap
_DA_FIELDS = _native.DECODE_ARGS_DTYPE.fields
_DA_HEAD = struct.Struct("<4Q3q")
_DA_TAIL = struct.Struct("<10i2f")
_DA_TAIL_OFF = _DA_FIELDS["B"][1]
_DA_PAGES, _DA_TOKK, _DA_TOKV, _DA_TOKHS, _DA_NPAGES, _DA_TOKENS = (
    _DA_FIELDS[f][1] for f in ("seq_pages", "tok_k", "tok_v", "tok_head_stride", "seq_npages",
                               "seq_tokens"))
_DA_U64, _DA_I64, _DA_I32 = struct.Struct("<Q"), struct.Struct("<q"), struct.Struct("<i")
assert _DA_FIELDS["q"][1] == 0 and _DA_FIELDS["seq_pages"][1] == _DA_HEAD.size
assert _DA_TAIL_OFF + _DA_TAIL.size == _native.DECODE_ARGS_DTYPE.itemsize
_MASK_CODES = {torch.float32: _native.HELM_F32, torch.bfloat16: _native.HELM_BF16,
               torch.float16: _native.HELM_F16}
_KV16 = {torch.bfloat16: _native.HELM_BF16, torch.float16: _native.HELM_F16}


def _decode_args():
    """This thread's helm_decode_args block: (the struct array, its bytes,
    its address)."""
    a = getattr(_tls, "decode_args", None)
    if a is None:
        arr = np.zeros(1, dtype=_native.DECODE_ARGS_DTYPE)
        a = _tls.decode_args = (arr, arr.view(np.uint8), arr.ctypes.data)
    return a


def _decode_step_fast(kvcms, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      layer_idx: int, scale: float,
                      attention_mask: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """The common decode step of ``_decode_batched`` in one native call
    (helm_decode_step): every item a KVCacheManager whose layer holds only
    device pages with device-resident records that need no upload, the tail
    page with room for the token, nothing over the watermark, 16-bit KV,
    D = 128, q in the KV dtype.  Then HELM's append_decode bookkeeping for the
    token is a tail count, the residency policy (kv_cache.py:224-235) cannot
    evict anything (the evictable pages and their bytes do not change), and
    the attention kernel writes each token itself.  Returns None, having
    changed nothing, when any of that does not hold (the general path runs;
    HELM_AMD_FAST_DECODE=0 always takes it)."""
    B, Hq, S, D = q.shape
    kv_code = _KV16.get(q.dtype)
    if (kv_code is None or S != 1 or D != 128 or B > _native.DECODE_MAX_SEQS
            or not q.is_cuda or k.dtype is not q.dtype or v.dtype is not q.dtype
            or not q.is_contiguous()):
        return None
    kB, Hkv, kS, _ = k.shape
    ks, vs = k.stride(), v.stride()
    kp, vp = k.data_ptr(), v.data_ptr()
    qp = q.data_ptr()
    if (Hq > 16 * Hkv                           # more than one 16-row tile per KV head
            or kB < B or kS != 1 or ks[3] != 1 or vs[3] != 1 or ks[1] != vs[1]
            or (ks[1] * 2) % 16 or (kp | vp | qp | (ks[0] * 2) | (vs[0] * 2)) % 16):
        return None
    if (check_records_enabled() or not _async_kv_prefetch_enabled()
            or _env_get("HELM_AMD_FAST_DECODE") == "0"
            or _env_get("HELM_AMD_FUSED_APPEND") == "0"
            or _env_get("HELM_AMD_KERNEL") not in (None, "", "auto", "mfma")):
        return None
    device = q.device
    sig = (q.dtype, Hkv, D)
    layers = []
    for kvcm in kvcms[:B]:
        if (type(kvcm) is not KVCacheManager or "append_decode" in kvcm.__dict__
                or kvcm.use_contiguous):
            return None
        layer = kvcm.layers.get(layer_idx)
        if layer is None or layer._n_host or layer._n_other or not layer._rec_ok:
            return None
        tail = layer.tail_page
        if (tail is None or tail.used_tokens >= tail.capacity_tokens or tail.state != "GPU"
                or layer._rec_sig != sig or not layer._aligned16 or layer._dev is None
                or layer._dev_dirty or layer._dev_all or layer._dev.device != device):
            return None
        kvcm._sync_layers()
        if kvcm._ev_bytes > kvcm.gpu_high_watermark_bytes:
            return None
        layers.append(layer)
    if B > 1 and len({id(layer) for layer in layers}) != B:
        return None
    mask_code, mbs, mhs, mptr = _native.HELM_F32, 0, 0, 0
    m = attention_mask
    if m is not None:
        mask_code = _MASK_CODES.get(m.dtype)
        t_max = max(l._tail_tok_off + l.tail_page.used_tokens for l in layers) + 1
        mshape = m.shape
        if (mask_code is None or m.device != device or len(mshape) != 4
                or mshape[0] not in (1, B) or mshape[1] not in (1, Hq) or mshape[2] != 1
                or mshape[3] < t_max):
            return None
        mst = m.stride()
        if mst[3] != 1:
            return None
        mptr = m.data_ptr()
        mbs = mst[0] if mshape[0] > 1 else 0
        mhs = mst[1] if mshape[1] > 1 else 0
    # HELM's append_decode bookkeeping (kv_cache.py:145-171): the tail gains
    # the token
    _, buf, addr = _decode_args()
    ks0, vs0, hs = ks[0] * 2, vs[0] * 2, ks[1]
    page_tokens = 0
    u64, i64, i32 = _DA_U64.pack_into, _DA_I64.pack_into, _DA_I32.pack_into
    for b, layer in enumerate(layers):
        tail = layer.tail_page
        used = tail.used_tokens + 1
        tail.used_tokens = used
        layer.total_tokens += 1
        n = len(layer.pages)
        layer._rec["used"][n - 1] = used
        u64(buf, _DA_PAGES + 8 * b, layer._dev.data_ptr())
        u64(buf, _DA_TOKK + 8 * b, kp + b * ks0)
        u64(buf, _DA_TOKV + 8 * b, vp + b * vs0)
        i64(buf, _DA_TOKHS + 8 * b, hs)
        i32(buf, _DA_NPAGES + 4 * b, n)
        i32(buf, _DA_TOKENS + 4 * b, layer._tail_tok_off + used)
        if layer._page_tokens > page_tokens:
            page_tokens = layer._page_tokens
    out = torch.empty_like(q)
    _DA_HEAD.pack_into(buf, 0, qp, out.data_ptr(), mptr, _engine.stream_ptr(device),
                       mbs, mhs, 0)
    _DA_TAIL.pack_into(buf, _DA_TAIL_OFF, B, Hq, Hkv, D, page_tokens, 1, mask_code, kv_code,
                       1, 0, scale, 0.0)
    rc = _native.entry("helm_decode_step")(_engine.get_engine(device), addr)
    if rc:
        _native.check("helm_decode_step", rc)
    return out


def _stage_host_pages_sync(segs: List[_Segment], device: torch.device) -> List[_Segment]:
    """HELM_DISABLE_ASYNC_KV: copy host pages to device synchronously first."""
    out = []
    for sg in segs:
        if not sg.host:
            out.append(sg)
            continue
        k, v = sg.keep
        kd = k.to(device)
        vd = v.to(device)
        torch.cuda.current_stream(device).synchronize()
        out.append(_Segment(kd.data_ptr() + (sg.k - k.data_ptr()),
                            vd.data_ptr() + (sg.v - v.data_ptr()),
                            sg.used, sg.head_stride, False, (kd, vd)))
    return out


def perform_streaming_attention(
    query: torch.Tensor,
    pages: List[KVPage],
    scale: float = None,
    attention_mask: Optional[torch.Tensor] = None,
    softcap: Optional[float] = None,
):
    """Attention of `query` [B,Hq,q_len,D] over `pages`, HELM's helper
    (kv_cache.py:405-662) with HIP kernels.

    Path selection follows HELM: a mask or softcap attends every active page
    in token order (online-softmax branch, :468-555); otherwise GPU-only pages
    use top-left causal masking when q_len > 1 (Path 1, :562-568) and mixed
    residency attends all pages unmasked (Path 3, :584-662).  Host pages are
    prefetched through the engine's staging ring, overlapped with the device
    pages.  A query on the CPU runs the host-CPU kernel (Path 2 and the CPU
    branch of the loop, :531-555, :573-577).  The output has the query's
    shape and dtype.
    """
    device = query.device
    if scale is None:
        scale = 1.0 / math.sqrt(query.size(-1))
    if type(pages) is _LayerPages:
        out = _attend_layer_pages(query, pages, scale, attention_mask, softcap)
        if out is not None:
            return out
    active_pages = [p for p in pages if p.used_tokens > 0 and p.state != 'DEAD']
    if not active_pages:
        return torch.zeros_like(query)

    gpu_pages = [p for p in active_pages if p.state == 'GPU' and p.device.type == "cuda"]
    cpu_pages = [p for p in active_pages if p.state == 'CPU' and p.device.type != "cuda"]

    if device.type == "cuda" and cpu_pages:
        _cpu_bytes = sum(p.k_tensor[:, :, :p.used_tokens, :].numel() * p.k_tensor.element_size() * 2
                         for p in cpu_pages)
        _record_prefetch(len(cpu_pages), _cpu_bytes)

    if device.type != "cuda":
        return _cpu_query_attention(query, active_pages, gpu_pages, cpu_pages, scale,
                                    attention_mask, softcap)

    masked = attention_mask is not None or softcap is not None
    if masked:
        seq_pages, causal = active_pages, False
    elif not cpu_pages:
        seq_pages, causal = gpu_pages, query.size(2) > 1
    else:
        seq_pages, causal = gpu_pages + cpu_pages, False
    if not seq_pages:
        return torch.zeros_like(query)

    first = seq_pages[0].k_tensor
    Hkv, D, kv_dtype = first.size(1), query.size(-1), first.dtype
    B = query.size(0)
    seqs = []
    for b in range(B):
        segs = [_page_segments(p, b, B, Hkv, D, kv_dtype) for p in seq_pages]
        if not _async_kv_prefetch_enabled():
            segs = _stage_host_pages_sync(segs, device)
        if B > 1 and any(sg.host for sg in segs):
            # host pages are streamed per sequence
            return torch.cat([
                perform_streaming_attention(
                    query[i:i + 1], [_batch_view(p, i) for p in pages], scale,
                    attention_mask[i:i + 1] if attention_mask is not None and
                    attention_mask.size(0) > 1 else attention_mask, softcap)
                for i in range(B)], dim=0)
        seqs.append(segs)
    return _attend(query, seqs, Hkv, kv_dtype, scale, attention_mask, softcap, causal)


def _on_host(page: KVPage) -> KVPage:
    """`page` itself when its tensors are in host memory, else a host copy of
    its used tokens (HELM's loop moves such a page with .to(device))."""
    if page.k_tensor.device.type != "cuda":
        return page
    u = page.used_tokens
    return KVPage(page.page_id, page.layer_id, page.start_token, u, page.capacity_tokens,
                  page.k_tensor[:, :, :u, :].cpu(), page.v_tensor[:, :, :u, :].cpu(),
                  torch.device("cpu"), page.state)


def _cpu_query_attention(query: torch.Tensor, active_pages, gpu_pages, cpu_pages, scale: float,
                         attention_mask: Optional[torch.Tensor], softcap: Optional[float]):
    """perform_streaming_attention for a query on the CPU (HELM's CPU-stage
    layers) on the host-CPU kernel.  With a mask or soft-cap: every active
    page in token order, HELM's loop (kv_cache.py:468-555; a page held on a
    GPU is first copied to the host, as the loop's .to(device) does).
    Otherwise HELM's Path 2 over the CPU pages (:573-577: unmasked and not
    causal, whatever q_len).  Without a mask, a CPU query over GPU-resident
    pages is HELM's Path 1 or 3, whose torch ops fail across devices: it
    raises RuntimeError here too."""
    if attention_mask is not None or softcap is not None:
        seq_pages = active_pages
    elif gpu_pages:
        raise RuntimeError("perform_streaming_attention: a query on the CPU over GPU-resident "
                           "pages needs a mask or soft-cap (HELM's unmasked paths for it run "
                           "torch ops across devices)")
    else:
        seq_pages = cpu_pages
    if not seq_pages:
        return torch.zeros_like(query)
    seq_pages = [_on_host(p) for p in seq_pages]
    first = seq_pages[0].k_tensor
    Hkv, D, kv_dtype = first.size(1), query.size(-1), first.dtype
    B = query.size(0)
    seqs = [[_page_segments(p, b, B, Hkv, D, kv_dtype) for p in seq_pages] for b in range(B)]
    return _attend(query, seqs, Hkv, kv_dtype, scale, attention_mask, softcap, 0)


def _attend_layer_pages(query: torch.Tensor, pages: _LayerPages, scale: float,
                        attention_mask: Optional[torch.Tensor], softcap: Optional[float]):
    """perform_streaming_attention over a layer's unchanged page list from
    the layer's records: the same path choice, token order, masking and
    prefetch counting as the page-by-page branch below, without reading each
    page in Python.  None when the records cannot serve."""
    layer = pages._live_layer()
    cpu = query.device.type != "cuda"
    if layer is None or query.size(0) != 1 or (not cpu and not _async_kv_prefetch_enabled()):
        return None
    rec = layer.records()
    n = len(pages)
    sig = layer._rec_sig
    if rec is None or n == 0 or layer._n_other or sig is None or sig[2] != query.size(-1):
        return None
    kv_dtype, Hkv = sig[0], sig[1]
    t = int(rec["tok_off"][n - 1]) + int(rec["used"][n - 1])
    if t == 0:
        return torch.zeros_like(query)
    if cpu:
        # every page in host memory: the loop and Path 2 attend all of them
        if layer._n_host != n:
            return None
        return _attend_records(query, rec, np.array([0, n], dtype=np.int32), t, Hkv, kv_dtype,
                               scale, attention_mask, softcap, 0)
    host = layer._n_host > 0
    if host:
        _record_prefetch(layer._n_host, layer._host_bytes)
    masked = attention_mask is not None or softcap is not None
    # Path 1's top-left causal applies to all-device pages only (Path 3 is unmasked)
    causal = (not masked) and (not host) and query.size(2) > 1
    if not host:
        return _attend_layers(query, [layer], [t], Hkv, kv_dtype, scale, attention_mask, softcap,
                              causal)
    return _attend_records(query, rec, np.array([0, n], dtype=np.int32), t, Hkv, kv_dtype, scale,
                           attention_mask, softcap, causal)


def _batch_view(page: KVPage, i: int) -> KVPage:
    if page.k_tensor.dim() == 4 and page.k_tensor.size(0) > 1:
        return KVPage(page.page_id, page.layer_id, page.start_token, page.used_tokens,
                      page.capacity_tokens, page.k_tensor[i:i + 1], page.v_tensor[i:i + 1],
                      page.device, page.state)
    return page
