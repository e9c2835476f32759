"""Page allocator over slot arenas — drop-in for helm/runtime/kv_allocator.py.

HELM (helm/runtime/kv_allocator.py:6-163) gives every page two separate
``torch.empty([1, Hkv, page, D])`` tensors.  Here a page is a *slot* of an
arena tensor ``[n_slots, 2, Hkv, page, D]`` that holds K at ``[slot, 0]`` and
V at ``[slot, 1]``:

* on the GPU the arena is one HBM allocation, so the attention kernel walks
  pages through a page table (slot ids) into a single pool, and a page's K/V
  head tiles are 4 KiB-contiguous at the headline shapes;
* on the host the arena is pinned memory (hipHostMalloc through torch's pinned
  allocator), so evict/prefetch copies are real DMA, and pages evicted in
  address order coalesce into one large copy.

``KVPage.k_tensor`` / ``v_tensor`` are the same ``[1, Hkv, page, D]`` shapes
as HELM's (views into the arena), pool and page-id accounting follow HELM
exactly (LIFO reuse, GPU reserve 8, CPU reserve 16, DEAD on eviction).
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from helm_amd.runtime.page import KVPage


def _pin_host() -> bool:
    return torch.cuda.is_available()


class _SlotPool:
    """Arenas of page slots on one device; free slots are reused LIFO."""

    def __init__(self, device: torch.device, slot_shape: Tuple[int, ...], dtype: torch.dtype):
        self.device = device
        self.slot_shape = slot_shape
        self.dtype = dtype
        self.arenas: List[torch.Tensor] = []
        self.bump = 0                      # next never-used slot of the last arena
        self.free: List[Tuple[int, int]] = []
        self.min_arena = int(os.environ.get("HELM_AMD_ARENA_PAGES", "64"))
        self.max_arena = 16384

    @property
    def capacity(self) -> int:
        return sum(a.shape[0] for a in self.arenas)

    def available(self) -> int:
        last = self.arenas[-1].shape[0] - self.bump if self.arenas else 0
        return len(self.free) + last

    def grow(self, n: int) -> None:
        """Adds an arena of at least `n` slots (geometric growth, capped)."""
        if self.arenas:
            # the never-used tail of the current arena stays available; pushed
            # highest-first so that the LIFO pops hand it out lowest-first
            last = len(self.arenas) - 1
            tail = [(last, s) for s in range(self.bump, self.arenas[-1].shape[0])]
            self.free.extend(reversed(tail))
            self.bump = self.arenas[-1].shape[0]
        size = max(n, min(max(self.capacity, self.min_arena), self.max_arena))
        pin = self.device.type == "cpu" and _pin_host()
        arena = torch.empty((size, *self.slot_shape), dtype=self.dtype, device=self.device,
                            pin_memory=pin)
        self.arenas.append(arena)
        self.bump = 0

    def take(self) -> Tuple[int, int]:
        if self.free:
            return self.free.pop()
        if not self.arenas or self.bump >= self.arenas[-1].shape[0]:
            self.grow(1)
        slot = (len(self.arenas) - 1, self.bump)
        self.bump += 1
        return slot

    def release(self, arena: int, slot: int) -> None:
        self.free.append((arena, slot))

    def view(self, arena: int, slot: int) -> Tuple[torch.Tensor, torch.Tensor]:
        a = self.arenas[arena]
        return a[slot, 0].unsqueeze(0), a[slot, 1].unsqueeze(0)

    def slot_ptr(self, arena: int, slot: int) -> int:
        a = self.arenas[arena]
        return a.data_ptr() + slot * a.stride(0) * a.element_size()

    def slot_bytes(self) -> int:
        return int(np.prod(self.slot_shape)) * torch.tensor([], dtype=self.dtype).element_size()


def _pool_key(device: torch.device):
    if device.type == "cuda":
        return ("cuda", device.index if device.index is not None else torch.cuda.current_device())
    return (device.type, None)


class KVAllocator:
    """Same constructor, fields and methods as HELM's KVAllocator."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, page_size: int = 64,
                 dtype=torch.bfloat16):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.dtype = dtype

        self.gpu_free_pool: List[KVPage] = []
        self.cpu_free_pool: List[KVPage] = []

        self.gpu_total_pages = 0
        self.cpu_total_pages = 0

        self._next_page_id = 0
        self._pools: Dict[tuple, _SlotPool] = {}

    # ── slots ────────────────────────────────────────────────────────────────
    def _slot_pool(self, device: torch.device) -> _SlotPool:
        key = _pool_key(device)
        pool = self._pools.get(key)
        if pool is None:
            dev = torch.device("cuda", key[1]) if key[0] == "cuda" else torch.device(device.type)
            shape = (2, self.num_kv_heads, self.page_size, self.head_dim)
            pool = self._pools[key] = _SlotPool(dev, shape, self.dtype)
        return pool

    def page_slot_pool(self, page: KVPage) -> Optional[_SlotPool]:
        """The slot pool backing `page`, or None for a foreign page."""
        if page.arena is None:
            return None
        return self._pools.get(_pool_key(page.device))

    def _create_page(self, device: torch.device) -> KVPage:
        pool = self._slot_pool(device)
        arena, slot = pool.take()
        k_tensor, v_tensor = pool.view(arena, slot)
        page = KVPage(
            page_id=self._next_page_id,
            layer_id=-1,
            start_token=0,
            used_tokens=0,
            capacity_tokens=self.page_size,
            k_tensor=k_tensor,
            v_tensor=v_tensor,
            device=device,
            state='FREE',
            arena=arena,
            slot=slot,
        )
        self._next_page_id += 1
        if device.type == 'cuda':
            self.gpu_total_pages += 1
        else:
            self.cpu_total_pages += 1
        return page

    # ── HELM API ─────────────────────────────────────────────────────────────
    def reserve_batch(self, batch_size: int, device: torch.device):
        """Create `batch_size` free pages on `device` (kv_allocator.py:50-57)."""
        pool = self._slot_pool(device)
        short = batch_size - pool.available()
        if short > 0:
            pool.grow(short)
        for _ in range(batch_size):
            page = self._create_page(device)
            if device.type == 'cuda':
                self.gpu_free_pool.append(page)
            else:
                self.cpu_free_pool.append(page)

    def allocate(self, device: torch.device) -> KVPage:
        """Pop a free page (LIFO), reserving 8 GPU / 16 CPU pages when empty
        (kv_allocator.py:59-78)."""
        if device.type == 'cuda':
            if not self.gpu_free_pool:
                self.reserve_batch(8, device)
            page = self.gpu_free_pool.pop()
            page.state = 'GPU'
        else:
            if not self.cpu_free_pool:
                self.reserve_batch(16, device)
            page = self.cpu_free_pool.pop()
            page.state = 'CPU'
        page.layer_id = -1
        page.start_token = 0
        page.used_tokens = 0
        page.device = device
        return page

    def free(self, page: KVPage):
        """Return a page to its pool without touching its data
        (kv_allocator.py:80-93)."""
        page.state = 'FREE'
        page.layer_id = -1
        page.start_token = 0
        page.used_tokens = 0
        if page.device.type == 'cuda':
            self.gpu_free_pool.append(page)
        else:
            self.cpu_free_pool.append(page)

    def move_page(self, page: KVPage, target_device: torch.device) -> KVPage:
        """Copy a page's tokens to a page on `target_device`
        (kv_allocator.py:95-144).  GPU->CPU leaves the old page DEAD and its
        HBM slot free for reuse."""
        if page.device == target_device:
            return page
        return self.move_pages([page], target_device)[0]

    def move_pages(self, pages: List[KVPage], target_device: torch.device,
                   sync: bool = True) -> List[KVPage]:
        """move_page for several pages with one batched copy call.

        Pages are moved in list order (new pages are allocated in that order,
        as HELM's per-page loop does); the data moves with one
        helm_evict_pages / helm_prefetch_pages call that coalesces adjacent
        slots.  ``sync`` keeps HELM's synchronous-copy contract
        (kv_allocator.py:108-116)."""
        moves = []
        for page in pages:
            if page.device == target_device:
                moves.append((page, page))
                continue
            new_page = self.allocate(target_device)
            moves.append((page, new_page))
        self._copy_data([(o, n) for o, n in moves if o is not n], sync)
        out = []
        for page, new_page in moves:
            if page is new_page:
                out.append(page)
                continue
            new_page.layer_id = page.layer_id
            new_page.start_token = page.start_token
            new_page.used_tokens = page.used_tokens
            new_page.device = target_device
            if page.device.type == 'cuda' and target_device.type != 'cuda':
                pool = self.page_slot_pool(page)
                if pool is not None:
                    pool.release(page.arena, page.slot)
                placeholder_dtype = page.k_tensor.dtype
                page.k_tensor = torch.empty(0, dtype=placeholder_dtype)
                page.v_tensor = torch.empty(0, dtype=placeholder_dtype)
                page.arena = None
                page.slot = -1
                page.state = 'DEAD'
                self.gpu_total_pages -= 1
            else:
                self.free(page)
            out.append(new_page)
        return out

    def _copy_data(self, moves: List[Tuple[KVPage, KVPage]], sync: bool) -> None:
        from helm_amd import _native
        from helm_amd.runtime import engine

        regions = {"d2h": [], "h2d": []}
        for src, dst in moves:
            used = src.used_tokens
            if used <= 0:
                continue
            sp, dp = self.page_slot_pool(src), self.page_slot_pool(dst)
            direction = None
            if src.device.type == "cuda" and dst.device.type == "cpu":
                direction = "d2h"
            elif src.device.type == "cpu" and dst.device.type == "cuda":
                direction = "h2d"
            if (direction is not None and sp is not None and dp is not None
                    and sp.slot_shape == dp.slot_shape
                    and (direction == "h2d" or dp.arenas[dst.arena].is_pinned())
                    and (direction == "d2h" or sp.arenas[src.arena].is_pinned())):
                # whole slot (K and V adjacent) in one region
                regions[direction].append((sp.slot_ptr(src.arena, src.slot),
                                           dp.slot_ptr(dst.arena, dst.slot), sp.slot_bytes()))
            else:
                dst.k_tensor[:, :, :used, :].copy_(src.k_tensor[:, :, :used, :])
                dst.v_tensor[:, :, :used, :].copy_(src.v_tensor[:, :, :used, :])
        for direction, regs in regions.items():
            if not regs:
                continue
            dev = next(p.device for pair in moves for p in pair if p.device.type == "cuda")
            arr = np.array(regs, dtype=np.uint64)
            src = np.ascontiguousarray(arr[:, 0])
            dst = np.ascontiguousarray(arr[:, 1])
            nb = np.ascontiguousarray(arr[:, 2])
            fn = "helm_evict_pages" if direction == "d2h" else "helm_prefetch_pages"
            _native.call(fn, engine.get_engine(dev), len(regs), _native.ptr(src),
                         _native.ptr(dst), _native.ptr(nb), 1 if sync else 0,
                         engine.stream_ptr(dev))

    def report_usage(self) -> dict:
        """Pool statistics (kv_allocator.py:146-163)."""
        bytes_per_page = 2 * (1 * self.num_kv_heads * self.page_size * self.head_dim
                              * torch.finfo(self.dtype).bits // 8)
        gpu_used_pages = self.gpu_total_pages - len(self.gpu_free_pool)
        cpu_used_pages = self.cpu_total_pages - len(self.cpu_free_pool)
        return {
            "gpu_pool_size": self.gpu_total_pages,
            "cpu_pool_size": self.cpu_total_pages,
            "active_gpu_pages": gpu_used_pages,
            "active_cpu_pages": cpu_used_pages,
            "gpu_free_pages": len(self.gpu_free_pool),
            "cpu_free_pages": len(self.cpu_free_pool),
            "gpu_reserved_bytes": self.gpu_total_pages * bytes_per_page,
            "cpu_reserved_bytes": self.cpu_total_pages * bytes_per_page,
            "gpu_used_bytes": gpu_used_pages * bytes_per_page,
            "cpu_used_bytes": cpu_used_pages * bytes_per_page,
        }
