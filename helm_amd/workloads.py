"""Synthetic decode-attention workloads at the benchmark shapes.

Every workload is a slot pool in the allocator's arena layout
``[n_slots, 2, Hkv, page, D]`` (K at ``[:, 0]``, V at ``[:, 1]``), an int32
page table drawn as a seeded random permutation of the slots (sequences take
consecutive runs of one shuffled free list), per-sequence context lengths, and
q ~ N(0, 1).  K/V are N(0, 1) in the storage dtype.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    B: int
    Hq: int
    Hkv: int
    D: int
    dtype: torch.dtype
    T: Optional[int] = None                       # fixed context per sequence
    T_range: Optional[Tuple[int, int]] = None     # ragged contexts ~ U[lo, hi]
    page_size: int = 16
    offload_frac: float = 0.0                     # oldest fraction of pages in host RAM
    layers: int = 1
    model: str = ""

    @property
    def G(self) -> int:
        return self.Hq // self.Hkv

    def token_bytes(self) -> int:
        """K+V bytes of one token of one layer."""
        return 2 * self.Hkv * self.D * torch.tensor([], dtype=self.dtype).element_size()


WORKLOADS = {
    w.name: w for w in [
        Workload("qwen3-0.6b-2k", 1, 16, 8, 128, torch.float16, T=2048, model="Qwen3-0.6B"),
        Workload("qwen3-8b-32k", 1, 32, 8, 128, torch.bfloat16, T=32768, model="Qwen3-8B"),
        Workload("qwen3-8b-32k-offload50", 1, 32, 8, 128, torch.bfloat16, T=32768,
                 offload_frac=0.5, model="Qwen3-8B"),
        Workload("qwen3-14b-ragged-b8", 8, 40, 8, 128, torch.bfloat16, T_range=(4096, 32768),
                 model="Qwen3-14B"),
        Workload("llama2-13b-128k-offload75", 1, 40, 40, 128, torch.float16, T=131072,
                 offload_frac=0.75, model="Llama-2-13B"),
        Workload("qwen3-14b-40l-b4-64k", 4, 40, 8, 128, torch.bfloat16, T=65536, layers=40,
                 model="Qwen3-14B"),
    ]
}


def context_lengths(w: Workload, seed: int) -> list:
    if w.T is not None:
        return [w.T] * w.B
    lo, hi = w.T_range
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (w.B,), generator=g).tolist()


def make_pool_case(w: Workload, seed: int, device, lens: Optional[list] = None,
                   extra_slots: int = 0) -> dict:
    """Pool, page table, lengths and q for one layer of workload `w`."""
    device = torch.device(device)
    lens = context_lengths(w, seed) if lens is None else list(lens)
    P = w.page_size
    n_pages = [max(0, math.ceil(t / P)) for t in lens]
    n_slots = sum(n_pages) + extra_slots
    gen_dev = device if device.type == "cuda" else torch.device("cpu")
    g = torch.Generator(device=gen_dev).manual_seed(seed)
    pool = torch.randn((max(n_slots, 1), 2, w.Hkv, P, w.D), generator=g, device=gen_dev,
                       dtype=torch.float32 if gen_dev.type == "cpu" else w.dtype)
    pool = pool.to(device=device, dtype=w.dtype)
    q = torch.randn((w.B, w.Hq, 1, w.D), generator=g, device=gen_dev,
                    dtype=torch.float32 if gen_dev.type == "cpu" else w.dtype)
    q = q.to(device=device, dtype=w.dtype)
    gc = torch.Generator().manual_seed(seed + 7919)
    perm = torch.randperm(max(n_slots, 1), generator=gc)
    max_pages = max(n_pages + [1])
    table = torch.zeros((w.B, max_pages), dtype=torch.int32)
    off = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    return {
        "q": q,
        "pool": pool,
        "k_pool": pool[:, 0],
        "v_pool": pool[:, 1],
        "table": table.to(device),
        "table_cpu": table,
        "lens": torch.tensor(lens, dtype=torch.int32, device=device),
        "lens_list": lens,
        "n_pages": n_pages,
        "max_pages": max_pages,
        "scale": 1.0 / math.sqrt(w.D),
    }


def kv_bytes(w: Workload, lens: list) -> int:
    """Algorithmic K+V bytes one attention call over `lens` reads."""
    return sum(lens) * w.token_bytes()


def algorithmic_bytes(w: Workload, lens: list) -> int:
    """K+V + q + out + page-table bytes of one decode-attention call."""
    es = torch.tensor([], dtype=w.dtype).element_size()
    pages = sum(math.ceil(t / w.page_size) for t in lens)
    return kv_bytes(w, lens) + 2 * w.B * w.Hq * w.D * es + 4 * pages


def pool_records(case: dict, w: Workload):
    """``helm_page`` records of a pool case in page-table order (sequence b
    owns seq_off[b]:seq_off[b+1]; token offsets from 0 per sequence), for the
    entry points that take page records (helm_stream_attn,
    helm_cpu_stream_attn).  Returns (records, seq_off) numpy arrays."""
    import numpy as np
    from helm_amd import _native
    pool, table, P = case["pool"], case["table_cpu"], w.page_size
    es = pool.element_size()
    recs, seq_off = [], [0]
    for b, n in enumerate(case["n_pages"]):
        t = case["lens_list"][b]
        for i in range(n):
            base = pool.data_ptr() + int(table[b, i]) * pool.stride(0) * es
            recs.append((base, base + pool.stride(1) * es, min(P, t - i * P), i * P,
                         pool.stride(2), 0))
        seq_off.append(len(recs))
    arr = np.array(recs, dtype=_native.PAGE_DTYPE) if recs else np.zeros(0, _native.PAGE_DTYPE)
    return arr, np.array(seq_off, dtype=np.int32)
