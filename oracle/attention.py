"""CPU oracle for HELM's streaming attention — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the reference results are compared with (or,
in bench.py, as the timed CPU baseline).  The product (helm_amd) never imports it: its own host-CPU
attention (helm_cpu_stream_attn in libhelm_cpu.so) is checked against it.

Three independent statements of the same arithmetic:

* ``online_softmax_pages`` restates HELM's per-page online-softmax branch of
  perform_streaming_attention on CPU (helm/runtime/kv_cache.py:468-555, the
  branch taken whenever a mask or soft-cap is passed — every production
  decode step, pipeline_runtime.py:217 -> kv_offload.py:176-186);
* ``concat_sdpa`` restates HELM's all-CPU Path 2 (kv_cache.py:573-577):
  concatenate the pages, upcast to fp32, expand GQA, one fp32 SDPA;
* ``attention_fp64`` is the textbook formula in float64 numpy, written
  without any of HELM's structure (no pages, no online rescaling), which
  pins the two restatements (tests/test_oracle.py).

GQA everywhere: query head h reads KV head h // (Hq / Hkv), HELM's
repeat_interleave (kv_cache.py:459-466).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

PageKV = Tuple[torch.Tensor, torch.Tensor]  # k, v: [1, Hkv, used, D]


def expand_kv(k: torch.Tensor, v: torch.Tensor, num_q_heads: int):
    """repeat_interleave KV heads up to the query heads (kv_cache.py:459-466)."""
    num_kv = k.size(1)
    if num_kv != num_q_heads:
        groups = num_q_heads // num_kv
        k = k.repeat_interleave(groups, dim=1)
        v = v.repeat_interleave(groups, dim=1)
    return k, v


def online_softmax_pages(query: torch.Tensor, pages: Sequence[PageKV], scale: float = None,
                         attention_mask: Optional[torch.Tensor] = None,
                         softcap: Optional[float] = None) -> torch.Tensor:
    """HELM's masked / soft-capped streaming branch on CPU
    (kv_cache.py:468-473 setup, :531-552 loop, :554-555 normalise).

    `pages` are the active pages in token order, each already sliced to its
    used tokens.  Returns [B, Hq, q_len, D] in the query's dtype."""
    num_q_heads = query.size(1)
    if scale is None:
        scale = 1.0 / math.sqrt(query.size(-1))
    dtype = query.dtype
    q32 = query.float()
    bsz, _, q_len, _ = query.shape
    out = torch.zeros(bsz, num_q_heads, q_len, query.size(-1), dtype=torch.float32)
    running_max = torch.full((bsz, num_q_heads, q_len, 1), -float("inf"), dtype=torch.float32)
    running_sum = torch.zeros((bsz, num_q_heads, q_len, 1), dtype=torch.float32)
    token_cursor = 0
    for k_page, v_page in pages:
        used = k_page.size(2)
        k, v = expand_kv(k_page.float(), v_page.float(), num_q_heads)
        scores = torch.matmul(q32, k.transpose(-2, -1)) * scale
        if softcap is not None:
            scores = torch.tanh(scores / softcap) * softcap
        if attention_mask is not None:
            scores = scores + attention_mask[:, :, :, token_cursor:token_cursor + used].float()
        block_max = scores.amax(dim=-1, keepdim=True)
        new_max = torch.maximum(running_max, block_max)
        old_scale = torch.nan_to_num(torch.exp(running_max - new_max), nan=0.0)
        block_exp = torch.exp(scores - new_max)
        out = out * old_scale + torch.matmul(block_exp, v)
        running_sum = running_sum * old_scale + block_exp.sum(dim=-1, keepdim=True)
        running_max = new_max
        token_cursor += used
    out = out / torch.clamp(running_sum, min=1e-12)
    return out.to(dtype)


def concat_sdpa(query: torch.Tensor, pages: Sequence[PageKV], scale: float = None) -> torch.Tensor:
    """HELM's all-CPU Path 2 (kv_cache.py:573-577)."""
    if scale is None:
        scale = 1.0 / math.sqrt(query.size(-1))
    K = torch.cat([k for k, _ in pages], dim=2).float()
    V = torch.cat([v for _, v in pages], dim=2).float()
    K, V = expand_kv(K, V, query.size(1))
    return F.scaled_dot_product_attention(query.float(), K, V, scale=scale).to(query.dtype)


def streaming_attention(query: torch.Tensor, pages: Sequence[PageKV], scale: float = None,
                        attention_mask: Optional[torch.Tensor] = None,
                        softcap: Optional[float] = None) -> torch.Tensor:
    """HELM's CPU dispatch: no pages -> zeros (kv_cache.py:441-442); mask or
    soft-cap -> online-softmax loop; otherwise Path 2."""
    pages = [(k, v) for k, v in pages if k.size(2) > 0]
    if not pages:
        return torch.zeros_like(query)
    if attention_mask is not None or softcap is not None:
        return online_softmax_pages(query, pages, scale, attention_mask, softcap)
    return concat_sdpa(query, pages, scale)


def attention_fp64(q, K, V, scale: float = None, mask=None, softcap: Optional[float] = None,
                   causal: bool = False) -> np.ndarray:
    """softmax(q K^T * scale [softcap] [+ mask]) V in float64.

    q [B,Hq,S,D]; K, V [B or 1, Hkv, T, D]; mask broadcastable to
    [B,Hq,S,T] (additive); causal: key t visible to query row s iff t <= s.
    Keys whose logit is -inf get weight 0; a row with every logit -inf
    yields 0."""
    q = np.asarray(q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    B, Hq, S, D = q.shape
    Hkv, T = K.shape[1], K.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    G = Hq // Hkv
    out = np.zeros((B, Hq, S, D))
    m = None
    if mask is not None:
        m = np.broadcast_to(np.asarray(mask, dtype=np.float64)[..., :T], (B, Hq, S, T))
    for b in range(B):
        kb = K[b if K.shape[0] > 1 else 0]
        vb = V[b if V.shape[0] > 1 else 0]
        for h in range(Hq):
            kh, vh = kb[h // G], vb[h // G]
            for s in range(S):
                logits = (kh @ q[b, h, s]) * scale
                if softcap is not None:
                    logits = np.tanh(logits / softcap) * softcap
                if m is not None:
                    logits = logits + m[b, h, s]
                if causal:
                    logits = np.where(np.arange(T) <= s, logits, -np.inf)
                finite = logits > -np.inf
                if not finite.any():
                    continue
                mx = logits[finite].max()
                w = np.where(finite, np.exp(np.where(finite, logits - mx, 0.0)), 0.0)
                out[b, h, s] = (w @ vh) / w.sum()
    return out


def split_pages(k: torch.Tensor, v: torch.Tensor, sizes: List[int]) -> List[PageKV]:
    """[1,Hkv,T,D] -> consecutive pages of the given token counts."""
    out, t = [], 0
    for n in sizes:
        out.append((k[:, :, t:t + n, :], v[:, :, t:t + n, :]))
        t += n
    return out


def attention_fp64_batched(q, K, V, scale: float = None, mask=None,
                           softcap: Optional[float] = None) -> torch.Tensor:
    """The textbook formula of ``attention_fp64`` for decode shapes, vectorised
    with float64 torch matmuls so full-size contexts (10^5 keys) check in
    seconds.  q [Hq, S, D]; K, V [Hkv, T, D]; mask broadcastable to
    [Hq, S, T].  Pinned to ``attention_fp64`` in tests/test_oracle.py."""
    q = torch.as_tensor(q).double()
    K = torch.as_tensor(K).double()
    V = torch.as_tensor(V).double()
    Hq, S, D = q.shape
    Hkv, T, _ = K.shape
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qg = q.reshape(Hkv, G * S, D)
    logits = torch.matmul(qg, K.transpose(1, 2)).reshape(Hq, S, T) * scale
    if softcap is not None:
        logits = torch.tanh(logits / softcap) * softcap
    if mask is not None:
        logits = logits + torch.as_tensor(mask).double()[..., :T]
    finite = logits > -math.inf
    mx = torch.where(finite, logits, torch.full_like(logits, -math.inf)).amax(-1, keepdim=True)
    mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    w = torch.where(finite, torch.exp(logits - mx), torch.zeros_like(logits))
    den = w.sum(-1, keepdim=True)
    out = torch.matmul(w.reshape(Hkv, G * S, T), V).reshape(Hq, S, D)
    return torch.where(den > 0, out / torch.where(den > 0, den, torch.ones_like(den)),
                       torch.zeros_like(out))
