"""Direct binding of the batched pool-layout decode attention
(``helm_paged_decode_attn``): the vLLM-style entry point that the
benchmark and any caller with its own page table use.

The pool is the allocator's arena ``[n_slots, 2, Hkv, page, D]``;
``k_pool = arena[:, 0]`` and ``v_pool = arena[:, 1]`` are passed as views, so
the slot stride is ``2*Hkv*page*D`` elements and one page's head tile is
``page*D`` contiguous elements.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence

import numpy as np
import torch

from helm_amd import _native
from helm_amd.runtime import engine as _engine

_workspaces: Dict[int, torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A zero-initialised byte workspace of at least `nbytes` on `device`
    (reused; the kernels leave its ticket region zero)."""
    idx = _engine.device_index(device)
    ws = _workspaces.get(idx)
    if ws is None or ws.numel() < nbytes:
        torch.cuda.current_stream(device).synchronize()
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[idx] = ws
    return ws


class PreparedDecode:
    """helm_paged_decode_attn with its argument list built once, for callers
    that issue the same shape every step (serving loops, benchmarks): one
    ctypes call per ``run``.  ``run(k_pool, v_pool)`` may pass another pool of
    identical shape and strides (rotated pools); q, page table, lengths and
    out stay the ones given to ``prepare_paged_decode``."""

    def __init__(self, args: list, pool_index: int, fn):
        self._args = args
        self._pool_index = pool_index
        self._fn = fn
        self.out = None

    def run(self, k_pool: Optional[torch.Tensor] = None,
            v_pool: Optional[torch.Tensor] = None) -> torch.Tensor:
        a = self._args
        if k_pool is not None:
            a = list(a)
            a[self._pool_index] = k_pool.data_ptr()
            a[self._pool_index + 1] = v_pool.data_ptr()
        rc = self._fn(*a)
        if rc:
            _native.check("helm_paged_decode_attn", rc)
        return self.out


def prepare_paged_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                         page_table: torch.Tensor, seq_lens: torch.Tensor,
                         max_pages: Optional[int] = None, total_pages: int = 0,
                         scale: Optional[float] = None, softcap: Optional[float] = None,
                         out: Optional[torch.Tensor] = None,
                         pages_per_split: int = 0,
                         attention_mask: Optional[torch.Tensor] = None,
                         host_lens: Optional[Sequence[int]] = None) -> PreparedDecode:
    """Validates the shapes once and returns a PreparedDecode bound to torch's
    current stream on q's device (same arguments as paged_decode_attention;
    the mask, if any, is read at every run)."""
    args, keep = _decode_args(q, k_pool, v_pool, page_table, seq_lens, max_pages, total_pages,
                              scale, softcap, attention_mask, out, pages_per_split, host_lens)
    prep = PreparedDecode(args, 2, _native.load().helm_paged_decode_attn)
    prep.out = keep["out"]
    prep._keep = keep
    return prep


def paged_decode_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           page_table: torch.Tensor, seq_lens: torch.Tensor,
                           max_pages: Optional[int] = None, total_pages: int = 0,
                           scale: Optional[float] = None, softcap: Optional[float] = None,
                           attention_mask: Optional[torch.Tensor] = None,
                           out: Optional[torch.Tensor] = None,
                           pages_per_split: int = 0,
                           host_lens: Optional[Sequence[int]] = None) -> torch.Tensor:
    """Decode attention of q [B,Hq,q_len,D] over pooled pages.

    k_pool / v_pool: [n_slots, Hkv, page, D] (any slot stride, dense rows);
    page_table: int32 [B, >=max_pages] slot ids; seq_lens: int32 [B] tokens
    (device).  attention_mask: additive fp32-convertible [B|1, 1|Hq, q_len|1,
    >=max tokens].  host_lens: the same lengths as a host sequence (optional:
    a batch then gets a grid of exactly its splits).  Returns out
    [B,Hq,q_len,D] in q's dtype."""
    args, keep = _decode_args(q, k_pool, v_pool, page_table, seq_lens, max_pages, total_pages,
                              scale, softcap, attention_mask, out, pages_per_split, host_lens)
    _native.call("helm_paged_decode_attn", *args)
    return keep["out"]


def _decode_args(q, k_pool, v_pool, page_table, seq_lens, max_pages, total_pages, scale, softcap,
                 attention_mask, out, pages_per_split, host_lens=None):
    """Checks the operands and returns (C-ABI argument list, tensors to keep alive)."""
    if q.device.type != "cuda":
        raise RuntimeError("paged_decode_attention needs HIP tensors")
    B, Hq, S, D = q.shape
    n_slots, Hkv, P, Dk = k_pool.shape
    if Dk != D or v_pool.shape != k_pool.shape:
        raise ValueError("pool shapes do not match q")
    if k_pool.stride()[1:] != v_pool.stride()[1:] or k_pool.stride(0) != v_pool.stride(0):
        raise ValueError("k_pool and v_pool must share strides")
    if k_pool.stride(3) != 1 or k_pool.stride(2) != D:
        raise ValueError("pool pages need dense [page, D] rows")
    if page_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("page_table and seq_lens must be int32")
    if page_table.dim() != 2 or page_table.size(0) != B or seq_lens.numel() != B:
        raise ValueError("page_table must be [B, >=max_pages] and seq_lens [B]")
    if max_pages is None:
        max_pages = page_table.size(1)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    mask_ptr, mbs, mhs, mqs = None, 0, 0, 0
    m = None
    if attention_mask is not None:
        # fp32, bf16 and fp16 masks are read as given; others are widened
        m = attention_mask.to(device=q.device)
        if m.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            m = m.float()
        if m.stride(3) != 1:
            m = m.contiguous()
        mask_ptr = m.data_ptr()
        mbs = m.stride(0) if m.size(0) > 1 else 0
        mhs = m.stride(1) if m.size(1) > 1 else 0
        mqs = m.stride(2) if m.size(2) > 1 else 0
    hl = None
    if host_lens is not None:
        hl = np.ascontiguousarray(np.asarray(host_lens, dtype=np.int32))
        if hl.shape != (B,):
            raise ValueError("host_lens must hold B lengths")
    kcode = _native.dtype_code(k_pool.dtype)
    qcode = _native.dtype_code(q.dtype)
    lib = _native.load()
    need = lib.helm_query_workspace_bytes(B, Hq, Hkv, S, D, max_pages, P, pages_per_split)
    ws = workspace(q.device, need)
    args = [q.data_ptr(), out.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0),
            k_pool.stride(1), page_table.data_ptr(), page_table.stride(0), seq_lens.data_ptr(), B,
            Hq, Hkv, S, D, P, max_pages, total_pages,
            _native.ptr(hl) if hl is not None else None, float(scale),
            float(softcap) if softcap else 0.0, mask_ptr, mbs, mhs, mqs,
            _native.dtype_code(m.dtype) if m is not None else _native.HELM_F32, kcode, qcode,
            pages_per_split, ws.data_ptr(), ws.numel(), _engine.stream_ptr(q.device)]
    keep = {"q": q, "out": out, "mask": m, "ws": ws, "table": page_table, "lens": seq_lens,
            "host_lens": hl}
    return args, keep
