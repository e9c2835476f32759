"""CPU model of HELM's page management — TEST INFRASTRUCTURE ONLY.

Only tests/ (and __graft_entry__.smoke()) may import this module, as the
reference for helm_amd.runtime's page bookkeeping.  It restates, over plain
Python objects and numpy payloads, the semantics of:

* KVAllocator pools (helm/runtime/kv_allocator.py:6-163): LIFO free pools,
  GPU reserve 8 / CPU reserve 16, unique page ids, move_page with the GPU
  page left DEAD, report_usage;
* KVCacheManager appends and residency (helm/runtime/kv_cache.py:113-260):
  prefill split into new pages starting at the running token count, decode
  into the tail page, residency policy after every page / token, eviction of
  full non-tail GPU pages oldest-first by start_token until the excess is
  covered, paging counters.

Each page's payload is a numpy array holding, for every stored token, the
token's position in the layer, so a model run states exactly which bytes
every page of the product must hold (bit-exact gather/append checks).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np


@dataclass
class ModelPage:
    page_id: int
    layer_id: int
    start_token: int
    used_tokens: int
    capacity_tokens: int
    device: str          # 'cuda' | 'cpu'
    state: str           # 'FREE' | 'GPU' | 'CPU' | 'DEAD'
    payload: np.ndarray = field(repr=False)  # token positions, -1 = never written


class AllocatorModel:
    """kv_allocator.py:6-163 over metadata."""

    def __init__(self, page_size: int, page_bytes: int):
        self.page_size = page_size
        self.page_bytes = page_bytes
        self.gpu_free: List[ModelPage] = []
        self.cpu_free: List[ModelPage] = []
        self.gpu_total = 0
        self.cpu_total = 0
        self.next_id = 0

    def _create(self, device: str) -> ModelPage:                 # :22-48
        p = ModelPage(self.next_id, -1, 0, 0, self.page_size, device, "FREE",
                      np.full(self.page_size, -1, dtype=np.int64))
        self.next_id += 1
        if device == "cuda":
            self.gpu_total += 1
        else:
            self.cpu_total += 1
        return p

    def reserve_batch(self, n: int, device: str) -> None:       # :50-57
        for _ in range(n):
            (self.gpu_free if device == "cuda" else self.cpu_free).append(self._create(device))

    def allocate(self, device: str) -> ModelPage:               # :59-78
        pool = self.gpu_free if device == "cuda" else self.cpu_free
        if not pool:
            self.reserve_batch(8 if device == "cuda" else 16, device)
        p = pool.pop()
        p.state = "GPU" if device == "cuda" else "CPU"
        p.layer_id, p.start_token, p.used_tokens, p.device = -1, 0, 0, device
        return p

    def free(self, p: ModelPage) -> None:                       # :80-93
        p.state, p.layer_id, p.start_token, p.used_tokens = "FREE", -1, 0, 0
        (self.gpu_free if p.device == "cuda" else self.cpu_free).append(p)

    def move_page(self, p: ModelPage, target: str) -> ModelPage:  # :95-144
        if p.device == target:
            return p
        q = self.allocate(target)
        if p.used_tokens > 0:
            q.payload[:p.used_tokens] = p.payload[:p.used_tokens]
        q.layer_id, q.start_token, q.used_tokens, q.device = (p.layer_id, p.start_token,
                                                              p.used_tokens, target)
        if p.device == "cuda" and target != "cuda":
            p.state = "DEAD"
            self.gpu_total -= 1
        else:
            self.free(p)
        return q

    def report_usage(self) -> dict:                             # :146-163
        gu = self.gpu_total - len(self.gpu_free)
        cu = self.cpu_total - len(self.cpu_free)
        bpp = self.page_bytes
        return {
            "gpu_pool_size": self.gpu_total, "cpu_pool_size": self.cpu_total,
            "active_gpu_pages": gu, "active_cpu_pages": cu,
            "gpu_free_pages": len(self.gpu_free), "cpu_free_pages": len(self.cpu_free),
            "gpu_reserved_bytes": self.gpu_total * bpp, "cpu_reserved_bytes": self.cpu_total * bpp,
            "gpu_used_bytes": gu * bpp, "cpu_used_bytes": cu * bpp,
        }


@dataclass
class LayerModel:
    pages: List[ModelPage] = field(default_factory=list)
    tail: Optional[ModelPage] = None
    total: int = 0


class CacheModel:
    """KVCacheManager (kv_cache.py:88-260) over metadata; payloads hold token
    positions."""

    def __init__(self, alloc: AllocatorModel, watermark: int):
        self.alloc = alloc
        self.watermark = watermark
        self.layers: Dict[int, LayerModel] = {}
        self.stats = dict(evict_calls=0, pages_evicted=0, bytes_evicted=0)

    def _layer(self, lid: int) -> LayerModel:
        return self.layers.setdefault(lid, LayerModel())

    def append_prefill(self, lid: int, n: int, device: str = "cuda") -> None:  # :113-143
        layer = self._layer(lid)
        ps = self.alloc.page_size
        for s in range(0, n, ps):
            c = min(ps, n - s)
            p = self.alloc.allocate(device)
            p.layer_id, p.start_token, p.used_tokens = lid, layer.total, c
            p.payload[:c] = np.arange(layer.total, layer.total + c)
            layer.pages.append(p)
            layer.tail = p
            layer.total += c
            self.enforce()

    def append_decode(self, lid: int, device: str = "cuda", skip_residency: bool = False):  # :145-171
        layer = self._layer(lid)
        if layer.tail is None or layer.tail.used_tokens == layer.tail.capacity_tokens:
            p = self.alloc.allocate(device)
            p.layer_id, p.start_token, p.used_tokens = lid, layer.total, 0
            layer.pages.append(p)
            layer.tail = p
        p = layer.tail
        p.payload[p.used_tokens] = layer.total
        p.used_tokens += 1
        layer.total += 1
        if not skip_residency:
            self.enforce()

    def _evictable(self):
        return [(layer, p) for layer in self.layers.values() for p in layer.pages
                if p.state == "GPU" and p.device == "cuda" and p is not layer.tail
                and p.used_tokens == p.capacity_tokens]

    def evict_pages(self, nbytes: int) -> None:                 # :179-222
        if nbytes <= 0:
            return
        cands = sorted(self._evictable(), key=lambda t: t[1].start_token)
        moved, done = 0, 0
        for layer, p in cands:
            if done >= nbytes:
                break
            q = self.alloc.move_page(p, "cpu")
            idx = next(i for i, x in enumerate(layer.pages) if x is p)
            layer.pages[idx] = q
            done += self.alloc.page_bytes
            moved += 1
        if moved:
            self.stats["evict_calls"] += 1
            self.stats["pages_evicted"] += moved
            self.stats["bytes_evicted"] += done

    def enforce(self) -> None:                                  # :224-235
        gpu = self.alloc.page_bytes * len(self._evictable())
        if gpu > self.watermark:
            self.evict_pages(gpu - self.watermark)

    def gathered(self, lid: int) -> np.ndarray:
        """Token positions of the layer's active pages in page order."""
        return np.concatenate([p.payload[:p.used_tokens] for p in self.layers[lid].pages
                               if p.used_tokens > 0 and p.state != "DEAD"] or [np.zeros(0, int)])
