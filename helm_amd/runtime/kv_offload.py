"""KV offload integration — drop-in for helm/runtime/kv_offload.py.

Installs paged-KV attention forwards on a Hugging Face model's attention
modules and routes every attention through the HIP paged-attention library:

* decode (q_len == 1) appends the token to each batch item's paged cache and
  runs one batched native attention call when every item is GPU-resident,
  otherwise per-item streaming attention with host-page prefetch
  (``_decode_batched``, kv_offload.py:86-186);
* prefill appends the chunk to the pages; the first chunk attends over its
  own K/V, later chunks stream over every cached page (kv_offload.py:197-227);
* layers whose tensors are on the CPU (CPU stages of a hybrid plan) keep
  their pages in host memory and attend on the host-CPU kernel of
  libhelm_cpu.so, as HELM's patched forwards do on the CPU for every module
  (kv_offload.py:736-762).

The per-architecture differences of HELM's forwards (kv_offload.py:291-651) —
where q/k norms apply, Gemma-2's scaling, soft-cap and sliding window — are
captured by one traits table and a single forward builder.
"""
from __future__ import annotations

import importlib
import math
import os
import threading
import weakref
from dataclasses import dataclass
from types import MethodType
from typing import Optional

import numpy as np
import torch

from helm_amd import _native
from helm_amd.runtime import engine as _engine
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import (ContiguousKV, KVCacheManager, _async_kv_prefetch_enabled,
                                       _decode_step_fast,
                                       _attend, _attend_device_records, _attend_layers,
                                       _attend_records, _contiguous_segments, _page_segments,
                                       _record_prefetch, perform_streaming_attention)


# ── config (kv_offload.py:33-79) ───────────────────────────────────────────────
@dataclass
class KVOffloadConfig:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    page_size: int = 64
    dtype: torch.dtype = torch.float16
    # GPU KV bytes kept hot before older pages go to host; default ~512 tokens
    # per layer.
    gpu_watermark_bytes: Optional[int] = None
    # tokens of the optional pre-allocated contiguous all-GPU cache (0 = off)
    cont_capacity: int = 0

    def __post_init__(self):
        if self.gpu_watermark_bytes is None:
            elem = torch.tensor([], dtype=self.dtype).element_size()
            per_token_bytes = 2 * self.num_kv_heads * self.head_dim * elem
            self.gpu_watermark_bytes = 512 * per_token_bytes * self.num_layers

    @staticmethod
    def from_model(model, page_size: int = 64, gpu_watermark_bytes: Optional[int] = None,
                   cont_capacity: Optional[int] = None) -> "KVOffloadConfig":
        cfg = model.config
        num_kv_heads = getattr(cfg, "num_key_value_heads", cfg.num_attention_heads)
        head_dim = getattr(cfg, "head_dim", None) or (cfg.hidden_size // cfg.num_attention_heads)
        return KVOffloadConfig(
            num_layers=cfg.num_hidden_layers,
            num_kv_heads=num_kv_heads,
            head_dim=head_dim,
            page_size=page_size,
            dtype=next(model.parameters()).dtype,
            gpu_watermark_bytes=gpu_watermark_bytes,
            cont_capacity=0 if cont_capacity is None else cont_capacity,
        )


def _require_hip(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what}: tensors must be on a HIP device (no CPU attention path)")


def _own_append(kvcm) -> bool:
    """True when `kvcm` is a KVCacheManager whose append_decode is the class's
    own: its token writes can then be queued and issued as one launch for the
    batch, and its layers' page records serve attention.  Any other cache
    object HELM's forwards accept (one that only has append_decode /
    iterate_layer_pages / all_gpu_resident, or a manager whose append_decode
    a caller replaced on the instance, e.g. to count calls) gets its public
    append_decode called per item, as kv_offload.py:147 and :617 do."""
    return (isinstance(kvcm, KVCacheManager) and "append_decode" not in kvcm.__dict__
            and type(kvcm).append_decode is KVCacheManager.append_decode)


def _append_decode_items(kvcms, k, v, layer_idx: int, bsz: int, residency_kwarg: bool,
                         flush: bool = True) -> list:
    """Each item's token into its pages, then its residency policy (HELM's
    append_decode(..., skip_residency=False) per item); the writes of the
    managers that allow it go out as one append launch.  `residency_kwarg`:
    pass skip_residency=False to a foreign append_decode (kv_offload.py:147)
    or call it with the token only (the Gemma-2 forward, :617).  flush=False
    leaves those writes queued and returns the queues, one per such manager
    in item order: the caller issues them (or has the attention call write
    the tokens) before anything reads the pages."""
    queued = []
    for i in range(bsz):
        c = kvcms[i]
        if _own_append(c):
            c._append_decode_deferred(layer_idx, k[i:i + 1], v[i:i + 1])
            c._enforce_residency_policy()
            queued.append(c._appends)
        elif residency_kwarg:
            c.append_decode(layer_idx, k[i:i + 1], v[i:i + 1], skip_residency=False)
        else:
            c.append_decode(layer_idx, k[i:i + 1], v[i:i + 1])
    if flush:
        _flush_appends(queued)
    return queued


# ── decode (kv_offload.py:86-186) ──────────────────────────────────────────────
def _decode_batched(kvcms, q, k, v, layer_idx: int, scale: float,
                    attention_mask: Optional[torch.Tensor] = None):
    """One decode step of attention for a batch; returns [bsz, Hq, 1, D].

    Contiguous-cache path when enabled and within capacity; otherwise the
    token goes into every item's pages (residency enforced), then a single
    batched kernel call if all items are GPU-resident (ragged lengths are
    fine), else per-item streaming attention with host prefetch.
    `attention_mask` is the caller's additive key mask, [bsz, *, 1, kv_len].
    """
    bsz = q.shape[0]
    Hkv, D = k.shape[1], q.shape[-1]

    if getattr(kvcms[0], "use_contiguous", False):
        if kvcms[0].cont_seq_len < kvcms[0].cont_capacity:
            _require_hip(q, "_decode_batched")
            out = _decode_contiguous(kvcms[:bsz], q, k, v, layer_idx, Hkv, scale,
                                     attention_mask)
            # the step's token is committed after the last layer
            if layer_idx == kvcms[0].cont_num_layers - 1:
                for kvcm in kvcms:
                    kvcm.advance_contiguous()
            return out
        for kvcm in kvcms:
            kvcm.migrate_contiguous_to_pages()

    out = _decode_step_fast(kvcms, q, k, v, layer_idx, scale, attention_mask)
    if out is not None:
        return out
    queued = _append_decode_items(kvcms, k, v, layer_idx, bsz, True, flush=False)
    if len(queued) != bsz:
        _flush_appends(queued)
        queued = None
    return _decode_attend(kvcms, q, layer_idx, Hkv, scale, attention_mask, queued)


def _decode_contiguous(kvcms, q, k, v, layer_idx: int, Hkv: int, scale: float,
                       attention_mask: Optional[torch.Tensor]):
    """The contiguous fast path of a decode step (kv_offload.py:116-138):
    every item's token written into its buffers at its position (one append
    launch), then one attention call over the buffers' device-resident
    virtual-page records (ContiguousKV), each item over its tokens so far
    including this one."""
    for i, kvcm in enumerate(kvcms):
        kvcm._queue_contiguous(layer_idx, kvcm.cont_seq_len, k[i:i + 1], v[i:i + 1])
    _flush_appends([kvcm._appends for kvcm in kvcms])
    recs = [kvcm.contiguous_records(layer_idx) for kvcm in kvcms]
    ptrs = np.array([r[0] for r in recs], dtype=np.uint64)
    tokens = np.array([kvcm.cont_seq_len + 1 for kvcm in kvcms], dtype=np.int32)
    npages = (tokens + ContiguousKV.BLOCK - 1) // ContiguousKV.BLOCK
    kv_dtype = kvcms[0].cont_K[layer_idx].dtype
    return _attend_device_records(q, ptrs, npages.astype(np.int32), tokens, ContiguousKV.BLOCK,
                                  all(r[1] for r in recs), Hkv, kv_dtype, scale, attention_mask,
                                  None, 0)


def _decode_attend(kvcms, q, layer_idx: int, Hkv: int, scale: float,
                   attention_mask: Optional[torch.Tensor], pending=None):
    """The attention of a decode step once every item's token is in its pages:
    from the layers' records, else HELM's batched or per-item page-list path
    (kv_offload.py:116-186).  pending: the items' queued token writes, one
    queue per item, not yet issued (the records call may write them itself)."""
    bsz, D = q.shape[0], q.shape[-1]
    out = _decode_from_records(kvcms, q, layer_idx, Hkv, D, scale, attention_mask,
                               pending=pending)
    if out is not None:
        return out
    if pending:
        _flush_appends(pending)

    all_pages = [kvcms[i].iterate_layer_pages(layer_idx) for i in range(bsz)]

    if all(kvcms[i].all_gpu_resident(layer_idx) for i in range(bsz)):
        lists = [[p for p in pages if p.used_tokens > 0] for pages in all_pages]
        if all(lists):
            dtype = lists[0][0].k_tensor.dtype
            seqs = [[_page_segments(p, 0, 1, Hkv, D, dtype) for p in lst] for lst in lists]
            return _attend(q, seqs, Hkv, dtype, scale, attention_mask, None, False)

    outs = [
        perform_streaming_attention(
            q[i:i + 1], all_pages[i], scale=scale,
            attention_mask=attention_mask[i:i + 1] if attention_mask is not None else None)
        for i in range(bsz)
    ]
    return torch.cat(outs, dim=0)


def _flush_appends(queues) -> None:
    """Flushes several managers' queued token writes, as few launches as the
    (device, dtype, shape) of their rows allow."""
    head = None
    for q in queues:
        if not q.rows:
            continue
        if head is None:
            head = q
        elif (q.device, q.dtype, q.hkv, q.d) == (head.device, head.dtype, head.hkv, head.d):
            head.rows.extend(q.rows)
            head.keep.extend(q.keep)
            q.rows.clear()
            q.keep.clear()
        else:
            head.flush()
            head = q
    if head is not None:
        head.flush()


_MAX_SEQ_ARGS = 16     # sequences one helm_paged_attn_seqs call carries
_tls = threading.local()


def _fused_tokens(pending, kv_dtype, device) -> Optional[int]:
    """Host address of the items' token rows (helm_append_seg, item order) for
    helm_paged_attn_seqs_append, or None unless every queue holds exactly one
    one-token write of the KV dtype on `device`.  HELM_AMD_FUSED_APPEND=0
    keeps the separate append launch."""
    if os.environ.get("HELM_AMD_FUSED_APPEND") == "0":
        return None
    n = len(pending)
    # this thread's row array (kept between calls) as 8-byte words: the call
    # reads src_k, src_v, src_head_stride and n_tok of each 64-byte row,
    # words 2, 3, 4 and the low half of 7
    kept = getattr(_tls, "token_rows", None)
    if kept is None or len(kept[0]) < n:
        rows = np.zeros(max(n, _MAX_SEQ_ARGS), dtype=_native.APPEND_DTYPE)
        kept = _tls.token_rows = (rows, rows.view(np.uint64), rows.ctypes.data)
    rows, words, addr = kept
    for b, queue in enumerate(pending):
        if (len(queue.rows) != 1 or queue.dtype != kv_dtype or queue.device != device
                or queue.rows[0][8] != 1):
            return None
        row = queue.rows[0]
        w = 8 * b
        words[w + 2] = row[2]
        words[w + 3] = row[3]
        words[w + 4] = row[4]
        words[w + 7] = 1
    return addr


def _decode_from_records(kvcms, q, layer_idx: int, Hkv: int, D: int, scale: float,
                         attention_mask: Optional[torch.Tensor],
                         softcap: Optional[float] = None, pending=None):
    """The decode attention of `_decode_batched` from the layers' page records.

    Same outcome as the page-list path below (one batched call when every
    item is GPU-resident, else per-item streaming attention that counts the
    prefetched host pages), without touching each page in Python.  Returns
    None when a layer's records are unusable, so the page-list path runs
    (its caller then issues `pending`).  pending: one queue per item holding
    that item's new token, not yet written; every page on the device, the
    attention call writes the tokens itself, else they are issued first.
    """
    cpu = q.device.type != "cuda"
    if not cpu and not _async_kv_prefetch_enabled():
        return None
    # one pass over the items: each a KVCacheManager whose layer has usable
    # records of this call's shape and one KV dtype
    layers, recs, lens = [], [], []
    kv_dtype, host = None, False
    for kvcm in kvcms:
        if not isinstance(kvcm, KVCacheManager):
            return None
        layer = kvcm.layers.get(layer_idx)
        if layer is None:
            return None
        r = layer.records()
        sig = layer._rec_sig
        if r is None or len(r) == 0 or layer._n_other or sig is None or sig[1] != Hkv \
                or sig[2] != D or (kv_dtype is not None and sig[0] != kv_dtype):
            return None
        kv_dtype = sig[0]
        layers.append(layer)
        recs.append(r)
        lens.append(layer.total_tokens_recorded())
        host = host or layer._n_host > 0
    bsz = len(layers)
    if not cpu:
        # HELM streams the items that hold host pages one by one and counts
        # each as a prefetch (kv_offload.py:176-186, kv_cache.py:441-447)
        if host:
            for layer in layers:
                _record_prefetch(layer._n_host, layer._host_bytes)
        elif bsz <= _MAX_SEQ_ARGS:
            # every page on the device: the layers' device-resident records,
            # each item's new token written by the same launch where it can
            if pending:
                app = _fused_tokens(pending, kv_dtype, q.device)
                if app is not None:
                    out = _attend_layers(q, layers, lens, Hkv, kv_dtype, scale, attention_mask,
                                         softcap, False, tokens_app=app)
                    if out is not None:
                        for queue in pending:
                            queue.rows.clear()
                            queue.keep.clear()
                        return out
                _flush_appends(pending)
            return _attend_layers(q, layers, lens, Hkv, kv_dtype, scale, attention_mask,
                                  softcap, False)
    if pending:
        _flush_appends(pending)
    # (concatenated as raw 8-byte words: numpy's structured-dtype
    # concatenate is ~15x slower)
    arr = recs[0] if bsz == 1 else np.concatenate(
        [r.view(np.uint64) for r in recs]).view(recs[0].dtype)
    seq_off = np.zeros(bsz + 1, dtype=np.int32)
    np.cumsum([len(r) for r in recs], out=seq_off[1:])
    if cpu:
        # a CPU-stage layer: every page in host memory, one host-CPU call for
        # the batch (HELM's per-item loop or Path 2, kv_offload.py:176-186)
        if any(layer._n_host != len(layer.pages) for layer in layers):
            return None
        return _attend_records(q, arr, seq_off, max(lens), Hkv, kv_dtype, scale,
                               attention_mask, softcap, False)
    if bsz == 1 or not host:
        return _attend_records(q, arr, seq_off, max(lens), Hkv, kv_dtype, scale,
                               attention_mask, softcap, False)
    try:
        # host pages in mapped pinned memory are read in place: one call
        return _attend_records(q, arr, seq_off, max(lens), Hkv, kv_dtype, scale,
                               attention_mask, softcap, False)
    except NotImplementedError:
        pass        # some host pages must be staged: one call per item
    outs = []
    for i, r in enumerate(recs):
        m = attention_mask[i:i + 1] if attention_mask is not None else None
        outs.append(_attend_records(q[i:i + 1], r, np.array([0, len(r)], dtype=np.int32),
                                    lens[i], Hkv, kv_dtype, scale, m, softcap, False))
    return torch.cat(outs, dim=0)


def _cached_tokens(kvcm, layer_idx: int) -> int:
    """Tokens in the layer's active pages (from its records when they serve)."""
    layer = kvcm.layers.get(layer_idx) if isinstance(kvcm, KVCacheManager) else None
    if layer is not None and layer.records() is not None and not layer._n_other:
        n = len(layer.pages)
        return int(layer._rec["tok_off"][n - 1]) + int(layer._rec["used"][n - 1]) if n else 0
    return sum(page.used_tokens for page in kvcm.iterate_layer_pages(layer_idx)
               if page.used_tokens > 0 and getattr(page, "state", None) != "DEAD")


def _append_prefill_batched(kvcms, k, v, layer_idx: int) -> list:
    """Append a prefill chunk per item; returns each item's past length."""
    past_lengths = []
    for i in range(k.shape[0]):
        past_lengths.append(_cached_tokens(kvcms[i], layer_idx))
        kvcms[i].append_prefill(layer_idx, k[i:i + 1], v[i:i + 1])
        if getattr(kvcms[i], "use_contiguous", False):
            kvcms[i].prefill_contiguous(layer_idx, k[i:i + 1], v[i:i + 1])
    return past_lengths


def _stream_prefill_batched(kvcms, q, layer_idx: int, scale: float,
                            attention_mask: Optional[torch.Tensor] = None,
                            softcap: Optional[float] = None):
    """A later prefill chunk attends over every cached page, per item
    (perform_streaming_attention per item, kv_offload.py:207-227), issued from
    the layers' page records when they serve."""
    out = _prefill_from_records(kvcms, q, layer_idx, scale, attention_mask, softcap)
    if out is not None:
        return out
    outs = []
    for i in range(q.shape[0]):
        item_mask = attention_mask[i:i + 1] if attention_mask is not None else None
        outs.append(perform_streaming_attention(q[i:i + 1], kvcms[i].iterate_layer_pages(layer_idx),
                                                scale=scale, attention_mask=item_mask,
                                                softcap=softcap))
    return torch.cat(outs, dim=0)


def _prefill_from_records(kvcms, q, layer_idx: int, scale: float,
                          attention_mask: Optional[torch.Tensor], softcap: Optional[float]):
    """What per-item perform_streaming_attention gives for a prefill chunk
    (every active page in token order; top-left causal when unmasked and all
    pages are on the device, kv_cache.py:562-568; an exactly causal chunk mask
    as causal masking at its offset), from the layers' records;
    None when they cannot serve (the page-list path then runs)."""
    cpu = q.device.type != "cuda"
    if (not cpu and not _async_kv_prefetch_enabled()) or not all(
            isinstance(kvcm, KVCacheManager) for kvcm in kvcms):
        return None
    B, _, S, D = q.shape
    layers = [kvcm.layers.get(layer_idx) for kvcm in kvcms[:B]]
    if len(layers) != B:
        return None
    recs = []
    for layer in layers:
        r = layer.records() if layer is not None else None
        if r is None or len(r) == 0 or layer._n_other or layer._rec_sig is None:
            return None
        recs.append(r)
    kv_dtype, Hkv = layers[0]._rec_sig[0], layers[0]._rec_sig[1]
    if any(layer._rec_sig != (kv_dtype, Hkv, D) for layer in layers):
        return None
    lens = [int(r["tok_off"][-1]) + int(r["used"][-1]) for r in recs]
    # a chunk mask that is exactly causal after `past` tokens runs as causal
    # masking at that offset (same result, no mask reads; see
    # _causal_mask_offset); it covers every cached token, as the mask must
    causal_mask = 0
    if attention_mask is not None and attention_mask.shape[-1] >= max(lens):
        past = _causal_mask_offset(attention_mask, S)
        if past is not None:
            attention_mask, causal_mask = None, 1 + past
    if cpu:
        # a CPU-stage layer, every page in host memory: HELM's loop under a
        # mask, else its Path 2 (unmasked, not causal), in one host-CPU call
        if any(layer._n_host != len(layer.pages) for layer in layers):
            return None
        arr = recs[0] if B == 1 else np.concatenate(
            [r.view(np.uint64) for r in recs]).view(recs[0].dtype)
        seq_off = np.zeros(B + 1, dtype=np.int32)
        np.cumsum([len(r) for r in recs], out=seq_off[1:])
        return _attend_records(q, arr, seq_off, max(lens), Hkv, kv_dtype, scale, attention_mask,
                               softcap, causal_mask)
    masked = attention_mask is not None or softcap is not None or causal_mask > 0
    host = [layer._n_host > 0 for layer in layers]
    if not masked and any(host) and not all(host):
        return None         # causal differs between items: the page-list path
    # unmasked with every page on the device: Path 1's top-left causal
    causal = causal_mask or int((not masked) and S > 1 and not any(host))
    for layer in layers:
        _record_prefetch(layer._n_host, layer._host_bytes)
    if B <= _MAX_SEQ_ARGS and not any(host):
        return _attend_layers(q, layers, lens, Hkv, kv_dtype, scale, attention_mask, softcap,
                              causal)
    arr = recs[0] if B == 1 else np.concatenate(
        [r.view(np.uint64) for r in recs]).view(recs[0].dtype)
    seq_off = np.zeros(B + 1, dtype=np.int32)
    np.cumsum([len(r) for r in recs], out=seq_off[1:])
    try:
        return _attend_records(q, arr, seq_off, max(lens), Hkv, kv_dtype, scale, attention_mask,
                               softcap, causal)
    except NotImplementedError:
        pass        # host pages that must be staged: one call per item
    outs = []
    for i, r in enumerate(recs):
        m = attention_mask[i:i + 1] if attention_mask is not None and \
            attention_mask.size(0) > 1 else attention_mask
        outs.append(_attend_records(q[i:i + 1], r, np.array([0, len(r)], dtype=np.int32),
                                    lens[i], Hkv, kv_dtype, scale, m, softcap, causal))
    return torch.cat(outs, dim=0)


_CAUSAL_MASKS: dict = {}   # id(mask) -> (weak reference, signature, past or None)


def _causal_mask_offset(mask: Optional[torch.Tensor], S: int) -> Optional[int]:
    """past = T - S when an additive [B, H, S, T] mask is exactly the causal
    pattern of a prompt chunk after `past` cached tokens: 0 where key
    j <= past + i, <= -1e4 elsewhere (HF's and HELM's finfo.min masks in fp32,
    bf16 or fp16, helm/runtime/pipeline_runtime.py:94-113); None otherwise.
    Attending under such a mask equals attending with causal masking at that
    offset: every row sees key 0 .. past + i, which come before its masked
    keys in token order, so each masked weight exp(logit + mask - max)
    underflows to exactly 0, as with -inf.  The answer is remembered per
    tensor object and version (the forward passes one mask object to every
    layer), so the check runs once per forward and chunk.  The entry holds a
    weak reference: a later mask that reuses a freed mask's memory (same
    address, shape and a fresh version counter) is a different object and is
    checked anew.  A mask made under torch.inference_mode() (HELM's generate,
    inference.py:747) has no version counter, so an in-place change to it
    cannot be seen: it is checked on every call."""
    if (mask is None or S < 2 or mask.dim() != 4 or mask.shape[-2] != S
            or mask.shape[-1] < S
            or mask.dtype not in (torch.float32, torch.bfloat16, torch.float16)):
        return None
    T = mask.shape[-1]
    inference = mask.is_inference()
    sig = None if inference else (mask.data_ptr(), tuple(mask.shape), tuple(mask.stride()),
                                  mask.dtype, mask._version)
    ent = None if inference else _CAUSAL_MASKS.get(id(mask))
    if ent is not None and ent[0]() is mask and ent[1] == sig:
        return ent[2]
    upper = torch.ones(S, T, dtype=torch.bool, device=mask.device).triu_(1 + T - S)
    past = T - S if bool(torch.where(upper, mask <= -1e4, mask == 0).all()) else None
    if inference:
        return past
    if len(_CAUSAL_MASKS) > 64:
        _CAUSAL_MASKS.clear()
    _CAUSAL_MASKS[id(mask)] = (weakref.ref(mask), sig, past)
    return past


def _local_attention(q, k, v, scale, attention_mask, softcap=None):
    """First prefill chunk: attention over the chunk's own K/V (no pages yet),
    the SDPA / eager call of kv_offload.py:330-338, :605-613.  A mask that is
    exactly causal runs as causal masking (same result; the kernel then skips
    the keys past each row instead of reading the mask).  A query on the CPU
    (a CPU-stage layer) runs the host-CPU kernel."""
    if attention_mask is not None and attention_mask.dtype == torch.bool:
        attention_mask = torch.zeros(attention_mask.shape, dtype=torch.float32,
                                     device=attention_mask.device).masked_fill_(
            ~attention_mask, torch.finfo(torch.float32).min)
    if k.stride(3) != 1 or k.stride(2) != k.size(3) or v.stride() != k.stride():
        k, v = k.contiguous(), v.contiguous()
    seqs = [_contiguous_segments(k, v, b) for b in range(q.shape[0])]
    if (attention_mask is not None and attention_mask.shape[-1] == k.shape[2]
            and _causal_mask_offset(attention_mask, q.shape[2]) == k.shape[2] - q.shape[2]):
        return _attend(q, seqs, k.shape[1], k.dtype, scale, None, softcap,
                       1 + k.shape[2] - q.shape[2])
    return _attend(q, seqs, k.shape[1], k.dtype, scale, attention_mask, softcap, 0)


def _apply_softcap(attn_weights: torch.Tensor, softcap: Optional[float]) -> torch.Tensor:
    if softcap is None:
        return attn_weights
    return torch.tanh(attn_weights / softcap) * softcap


def _gemma2_sliding_window_mask(attn_self, attention_mask, cache_position, key_length: int, *,
                                device: torch.device, dtype: torch.dtype):
    """Caller mask plus Gemma-2's per-layer sliding window
    (kv_offload.py:240-288): key j is visible to query position i iff
    i - window < j <= i."""
    if attention_mask is not None:
        query_length = attention_mask.shape[-2]
        attention_mask = attention_mask[:, :, :query_length, :key_length]
    elif cache_position is not None:
        query_length = int(cache_position.numel())
    else:
        query_length = key_length

    window = getattr(attn_self, "sliding_window", None)
    if window is None:
        return attention_mask

    if cache_position is None:
        qpos = torch.arange(query_length, device=device, dtype=torch.long)
    else:
        qpos = cache_position.to(device=device, dtype=torch.long).reshape(-1)
        if qpos.numel() != query_length:
            raise ValueError(
                "Gemma2 sliding-window mask requires cache_position to match "
                f"query length ({query_length}), got {qpos.numel()}.")
    kpos = torch.arange(key_length, device=device, dtype=torch.long)
    visible = (kpos[None, :] <= qpos[:, None]) & (kpos[None, :] > qpos[:, None] - window)
    sliding = torch.full((query_length, key_length), torch.finfo(dtype).min, device=device,
                         dtype=dtype).masked_fill_(visible, 0)[None, None]
    return sliding if attention_mask is None else attention_mask + sliding


# ── per-architecture forwards (kv_offload.py:291-651) ─────────────────────────
@dataclass(frozen=True)
class _Arch:
    module: str        # transformers module holding the attention class
    cls: str           # attention class name
    rope_module: str   # module whose apply_rotary_pos_emb the forward uses
    qk_norm: str       # "none" | "head" (norm per head, Qwen3) | "proj" (OLMo-2)
    gemma: bool = False


_TM = "transformers.models."
_ARCHS = {
    "qwen2": _Arch(_TM + "qwen2.modeling_qwen2", "Qwen2Attention", _TM + "qwen2.modeling_qwen2", "none"),
    "qwen3": _Arch(_TM + "qwen3.modeling_qwen3", "Qwen3Attention", _TM + "qwen3.modeling_qwen3", "head"),
    "llama": _Arch(_TM + "llama.modeling_llama", "LlamaAttention", _TM + "llama.modeling_llama", "none"),
    "mistral": _Arch(_TM + "mistral.modeling_mistral", "MistralAttention",
                     _TM + "llama.modeling_llama", "none"),
    "ministral": _Arch(_TM + "ministral.modeling_ministral", "MinistralAttention",
                       _TM + "llama.modeling_llama", "none"),
    "olmo2": _Arch(_TM + "olmo2.modeling_olmo2", "Olmo2Attention", _TM + "olmo2.modeling_olmo2", "proj"),
    "gemma2": _Arch(_TM + "gemma2.modeling_gemma2", "Gemma2Attention",
                    _TM + "gemma2.modeling_gemma2", "none", gemma=True),
}
# name-substring resolution order of kv_offload.py:766-795 ("ministral" is
# checked before "mistral"; "qwen3" before "qwen2")
_RESOLVE_ORDER = ("qwen3", "qwen2", "gemma2", "ministral", "olmo2", "mistral", "llama")


def _gemma2_decode_from_records(attn_self, kvcms, q, layer: int, scale: float, softcap,
                                attention_mask, cache_position):
    """Gemma-2 decode attention with each item's sliding-window mask
    (kv_offload.py:577-613) as one call over the layers' records; None when
    the records cannot serve."""
    bsz = q.shape[0]
    if not all(isinstance(c, KVCacheManager) for c in kvcms[:bsz]):
        return None
    layers = [c.layers.get(layer) for c in kvcms[:bsz]]
    if any(L is None or L.records() is None or len(L.pages) == 0 for L in layers):
        return None
    lens = [int(L._rec["tok_off"][len(L.pages) - 1]) + int(L._rec["used"][len(L.pages) - 1])
            for L in layers]
    t_max = max(lens)
    mask = torch.zeros(bsz, 1, 1, t_max, device=q.device, dtype=torch.float32)
    for i in range(bsz):
        item = _gemma2_sliding_window_mask(
            attn_self, attention_mask[i:i + 1] if attention_mask is not None else None,
            cache_position, lens[i], device=q.device, dtype=q.dtype)
        if item is None:
            continue            # no window, no caller mask: nothing masked
        if item.dim() != 4 or item.size(1) != 1 or item.size(-1) < lens[i]:
            return None         # per-head masks: the per-item page-list path
        mask[i, :, :, :lens[i]] = item[0, :, -1:, :lens[i]]
    return _decode_from_records(kvcms[:bsz], q, layer, layers[0]._rec_sig[1], q.shape[-1],
                                scale, mask, softcap)


_FRONT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_FRONT_NORMS = {"head": ("Qwen3RMSNorm", 1), "proj": ("Olmo2RMSNorm", 2)}


def _front_norm(attn_self, arch: _Arch, dtype, Hq: int, Hkv: int, D: int):
    """(mode, q weight, k weight, eps) of the forward's q / k norm as
    helm_decode_front computes it, or None for a norm it does not reproduce."""
    if arch.qk_norm == "none":
        return 0, None, None, 0.0
    name, mode = _FRONT_NORMS[arch.qk_norm]
    qn, kn = getattr(attn_self, "q_norm", None), getattr(attn_self, "k_norm", None)
    if type(qn).__name__ != name or type(kn).__name__ != name:
        return None
    qw, kw = qn.weight, kn.weight
    want = (D, D) if mode == 1 else (Hq * D, Hkv * D)
    if (qw.dtype != dtype or kw.dtype != dtype or (qw.numel(), kw.numel()) != want
            or not qw.is_contiguous() or not kw.is_contiguous()
            or qn.variance_epsilon != kn.variance_epsilon):
        return None
    return mode, qw, kw, float(qn.variance_epsilon)


def _page_dst_ok(page, device, dtype, Hkv: int, D: int) -> bool:
    k, v = page.k_tensor, page.v_tensor
    return (k.device == device and v.device == device and k.dtype == dtype and v.dtype == dtype
            and k.dim() == 4 and k.shape[:2] == (1, Hkv) and k.size(3) == D
            and v.shape == k.shape and k.stride(3) == 1 and v.stride(3) == 1
            and k.stride(2) == D and v.stride(2) == D and k.stride(1) == v.stride(1))


def _decode_front(kvcms, attn_self, arch: _Arch, qp, kp, vp, cos, sin, layer: int):
    """The decode front end in one helm_decode_front launch: q / k norm,
    rotary embedding, and each item's token written into its pages (then
    the residency policy per item, as append_decode does).  Returns q
    [B, Hq, 1, D], or None when the forward's torch ops must run instead."""
    if os.environ.get("HELM_AMD_FRONT", "1") == "0":
        return None
    bsz = qp.shape[0]
    D = attn_self.head_dim
    dtype, device = qp.dtype, qp.device
    if (device.type != "cuda" or dtype not in _FRONT_DTYPES or len(kvcms) < bsz
            or not all(_own_append(c) for c in kvcms[:bsz])
            or any(c.use_contiguous for c in kvcms[:bsz])
            or (torch.is_grad_enabled() and (qp.requires_grad or kp.requires_grad))):
        return None
    if (qp.dim() != 3 or qp.size(1) != 1 or kp.shape != vp.shape or kp.dtype != dtype
            or vp.dtype != dtype or qp.size(2) % D or kp.size(2) % D or D % 2 or D > 256
            or qp.stride(2) != 1 or kp.stride(2) != 1 or vp.stride(2) != 1
            or kp.stride(0) != vp.stride(0)):
        return None
    Hq, Hkv = qp.size(2) // D, kp.size(2) // D
    if (Hq % Hkv or cos.dim() != 3 or cos.shape != sin.shape or cos.shape[1:] != (1, D)
            or cos.size(0) not in (1, bsz) or cos.dtype != sin.dtype
            or cos.dtype not in (dtype, torch.float32) or cos.stride(2) != 1
            or cos.stride() != sin.stride() or cos.device != device):
        return None
    norm = _front_norm(attn_self, arch, dtype, Hq, Hkv, D)
    if norm is None:
        return None
    for c in kvcms[:bsz]:
        lc = c.layers.get(layer)
        tail = lc.tail_page if lc is not None else None
        if (tail is not None and tail.used_tokens < tail.capacity_tokens
                and not _page_dst_ok(tail, device, dtype, Hkv, D)):
            return None
    # the destination of each item's token (bookkeeping as append_decode's)
    dst = np.zeros(bsz, dtype=_native.APPEND_DTYPE)
    for i in range(bsz):
        page, tok = kvcms[i]._decode_slot(layer, device)
        if not _page_dst_ok(page, device, dtype, Hkv, D):
            raise RuntimeError("decode front end: the tail page of layer %d is not a dense "
                               "[1, Hkv, P, D] device page" % layer)
        dst[i]["dst_k"] = page.k_tensor.data_ptr()
        dst[i]["dst_v"] = page.v_tensor.data_ptr()
        dst[i]["dst_head_stride"] = page.k_tensor.stride(1)
        dst[i]["dst_tok"] = tok
    mode, qw, kw, eps = norm
    q_out = torch.empty(bsz, Hq, 1, D, dtype=dtype, device=device)
    _native.call("helm_decode_front", qp.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                 qp.stride(0), kp.stride(0), qw.data_ptr() if qw is not None else None,
                 kw.data_ptr() if kw is not None else None, mode, eps, cos.data_ptr(),
                 sin.data_ptr(), cos.stride(0) if cos.size(0) > 1 else 0,
                 _native.dtype_code(cos.dtype), q_out.data_ptr(), _native.ptr(dst), bsz, Hq,
                 Hkv, D, _native.dtype_code(dtype), _engine.stream_ptr(device))
    for i in range(bsz):
        kvcms[i]._enforce_residency_policy()
    return q_out


def _gemma2_decode_attend(attn_self, kvcms, q, layer: int, scale: float, softcap,
                          attention_mask, cache_position):
    """Gemma-2 decode attention once every item's token is in its pages:
    one call over the layers' records with per-item sliding-window masks,
    else per-item streaming attention (kv_offload.py:577-613)."""
    out = _gemma2_decode_from_records(attn_self, kvcms, q, layer, scale, softcap,
                                      attention_mask, cache_position)
    if out is not None:
        return out
    outs = []
    for i in range(q.shape[0]):
        pages = kvcms[i].iterate_layer_pages(layer)
        key_length = sum(p.used_tokens for p in pages
                         if p.used_tokens > 0 and getattr(p, "state", None) != "DEAD")
        item_mask = (_gemma2_sliding_window_mask(
            attn_self, attention_mask[i:i + 1] if attention_mask is not None else None,
            cache_position, key_length, device=q.device, dtype=q.dtype)
            if key_length > 0 else None)
        outs.append(perform_streaming_attention(q[i:i + 1], pages, scale=scale,
                                                attention_mask=item_mask, softcap=softcap))
    return torch.cat(outs, dim=0)


def _make_forward(kvcms, arch: _Arch):
    """Attention forward for `arch` bound to the per-item caches `kvcms`."""

    def forward(attn_self, hidden_states, position_embeddings, attention_mask=None,
                past_key_values=None, cache_position=None, **kwargs):
        bsz, q_len, _ = hidden_states.shape
        shape = (bsz, q_len, -1, attn_self.head_dim)
        if arch.gemma:
            scale = getattr(attn_self, "scaling", 1.0 / math.sqrt(attn_self.head_dim))
            softcap = getattr(attn_self, "attn_logit_softcapping", None)
        else:
            scale = 1.0 / math.sqrt(attn_self.head_dim)
            softcap = None
        layer = attn_self.layer_idx
        cos, sin = position_embeddings

        q = attn_self.q_proj(hidden_states)
        k = attn_self.k_proj(hidden_states)
        v = attn_self.v_proj(hidden_states)
        if q_len == 1:
            # norm + rotary + page write in one launch where the kernel can
            qf = _decode_front(kvcms, attn_self, arch, q, k, v, cos, sin, layer)
            if qf is not None:
                if arch.gemma:
                    out = _gemma2_decode_attend(attn_self, kvcms, qf, layer, scale, softcap,
                                                attention_mask, cache_position)
                else:
                    out = _decode_attend(kvcms, qf, layer, k.size(2) // attn_self.head_dim,
                                         scale, attention_mask)
                out = out.transpose(1, 2).contiguous().reshape(bsz, q_len, -1)
                return attn_self.o_proj(out), None

        rope = importlib.import_module(arch.rope_module).apply_rotary_pos_emb
        if arch.qk_norm == "proj":
            q, k = attn_self.q_norm(q), attn_self.k_norm(k)
        q, k, v = q.view(shape), k.view(shape), v.view(shape)
        if arch.qk_norm == "head":
            q, k = attn_self.q_norm(q), attn_self.k_norm(k)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        q, k = rope(q, k, cos, sin)

        if q_len > 1:
            past_lengths = _append_prefill_batched(kvcms, k, v, layer)
            if any(past > 0 for past in past_lengths):
                mask = attention_mask
                if arch.gemma:
                    key_length = max(_cached_tokens(c, layer) for c in kvcms)
                    mask = _gemma2_sliding_window_mask(attn_self, attention_mask, cache_position,
                                                       key_length, device=q.device, dtype=q.dtype)
                out = _stream_prefill_batched(kvcms, q, layer, scale, mask, softcap)
            else:
                mask = attention_mask
                if arch.gemma:
                    mask = _gemma2_sliding_window_mask(attn_self, attention_mask, cache_position,
                                                       k.shape[-2], device=q.device, dtype=q.dtype)
                out = _local_attention(q, k, v, scale, mask, softcap)
        elif arch.gemma:
            _append_decode_items(kvcms, k, v, layer, bsz, False)
            out = _gemma2_decode_attend(attn_self, kvcms, q, layer, scale, softcap,
                                        attention_mask, cache_position)
        else:
            out = _decode_batched(kvcms, q, k, v, layer, scale, attention_mask)

        out = out.transpose(1, 2).contiguous().reshape(bsz, q_len, -1)
        return attn_self.o_proj(out), None

    return forward


def _make_qwen2_forward(kvcms):
    return _make_forward(kvcms, _ARCHS["qwen2"])


def _make_qwen3_forward(kvcms):
    return _make_forward(kvcms, _ARCHS["qwen3"])


def _make_olmo2_forward(kvcms):
    return _make_forward(kvcms, _ARCHS["olmo2"])


def _make_llama_forward(kvcms):
    return _make_forward(kvcms, _ARCHS["llama"])


def _make_gemma2_forward(kvcms):
    return _make_forward(kvcms, _ARCHS["gemma2"])


# ── manager (kv_offload.py:658-831) ────────────────────────────────────────────
class KVOffloadManager:
    """Installs paged-KV attention forwards on one model's attention modules
    and owns one KVCacheManager per batch item over a shared KVAllocator."""

    def __init__(self, model, config: KVOffloadConfig, batch_size: int = 1):
        self.config = config
        self.batch_size = batch_size
        self.allocator = KVAllocator(num_layers=config.num_layers,
                                     num_kv_heads=config.num_kv_heads,
                                     head_dim=config.head_dim, page_size=config.page_size,
                                     dtype=config.dtype)
        watermark_per_item = max(config.gpu_watermark_bytes // batch_size, 1)
        self.kvcms = [KVCacheManager(self.allocator, gpu_high_watermark_bytes=watermark_per_item)
                      for _ in range(batch_size)]
        self._patched: dict = {}
        self._patched_instance_forwards: dict = {}
        self._apply_patches(model)
        self.patch_module_roots(model)

        if config.cont_capacity > 0:
            device = next(model.parameters()).device
            if device.type == "cuda":
                built = [kvcm.build_contiguous(num_layers=config.num_layers,
                                               num_kv_heads=config.num_kv_heads,
                                               head_dim=config.head_dim,
                                               capacity=config.cont_capacity, device=device,
                                               dtype=config.dtype)
                         for kvcm in self.kvcms]
                if not all(built):
                    for kvcm in self.kvcms:
                        kvcm.drop_contiguous()

    def reset(self):
        """Clear every paged cache and re-arm the contiguous path."""
        for kvcm in self.kvcms:
            kvcm.clear()
            kvcm.reset_contiguous()

    def restore(self):
        """Put the original attention forwards back."""
        for module, had_instance_forward, original in self._patched_instance_forwards.values():
            if had_instance_forward:
                module.forward = original
            else:
                module.__dict__.pop("forward", None)
        self._patched_instance_forwards.clear()
        self._patched.clear()

    def report(self) -> dict:
        return self.allocator.report_usage()

    def patch_module_roots(self, *roots):
        """Bind the patched forward on every matching module instance under
        `roots` (instances only: the class and other models stay untouched)."""
        for root in roots:
            if root is None:
                continue
            for cls, patched_forward in self._patched.values():
                for module in root.modules():
                    if not isinstance(module, cls):
                        continue
                    key = id(module)
                    if key in self._patched_instance_forwards:
                        continue
                    had = "forward" in module.__dict__
                    original = module.__dict__.get("forward")
                    module.forward = MethodType(patched_forward, module)
                    self._patched_instance_forwards[key] = (module, had, original)

    def _apply_patches(self, model):
        name = model.__class__.__name__.lower()
        for arch in _RESOLVE_ORDER:
            if arch in name:
                self._patch(arch)
                return
        raise NotImplementedError(
            f"KVOffloadManager: no attention patch for {model.__class__.__name__}")

    def _patch(self, arch: str):
        spec = _ARCHS.get(arch)
        if spec is None:
            raise ValueError(arch)
        cls = getattr(importlib.import_module(spec.module), spec.cls)
        self._patched[arch] = (cls, _make_forward(self.kvcms, spec))
