"""HELM's other page sizes on the GPU: 128, 256 and 512 tokens per page (the
page-size sweep of HELM's paper, results/paper/table4_kv_page_size.csv:2-5,
set by HELM_KV_PAGE_SIZE / KVOffloadConfig.page_size, experiments/
paper_bench.py:1142-1158, helm/runtime/kv_offload.py:38), beside the 16 and
64 the other GPU tests use.

A page of P tokens is P / 16 blocks per page for the decode and chunk kernels,
so a split of up to 64 pages walks up to 2,048 blocks.  Per page size and KV
dtype (bf16, fp16; D = 128, Qwen3-8B's 32 / 8 heads), one layer holds a
prompt whose oldest pages the watermark moves to pinned host memory, then:

* a decode step through _decode_batched (the token appended, every page
  attended, host pages read in place or staged) under HELM's decode mask;
* a decode call through perform_streaming_attention over the layer's page
  list, masked (HELM's loop) and unmasked (Path 3);
* a 96-token prompt chunk appended and attended under HELM's chunk-prefill
  mask (pipeline_runtime.py:94-113), which the runtime runs as causal
  masking at the chunk's offset;

each against the float64 oracle (1e-2 bf16, 2e-3 fp16), and the pages'
contents against the source tensors bit for bit.
"""
import math

import pytest
import torch

from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager, perform_streaming_attention
from helm_amd.runtime.kv_offload import _decode_batched
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _layer_kv(mgr):
    pages = [p for p in mgr.layers[0].pages if p.used_tokens > 0 and p.state != "DEAD"]
    K = torch.cat([p.k_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
    V = torch.cat([p.v_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
    return K, V


def _err(out, q, K, V, G, mask=None, causal=False):
    """Max |out - fp64| over every query head ([Hq, S, D] rows)."""
    ref = A.attention_fp64(q[None].float(), K[None].float(), V[None].float(),
                           mask=mask, causal=causal)[0]
    return (out.double().cpu() - torch.from_numpy(ref)).abs().max().item()


def _chunk_mask(past, S, dtype):
    """HELM's _build_chunk_prefill_mask: key j visible to chunk row i iff
    j <= past + i, finfo.min elsewhere, in the model's dtype."""
    lo = torch.finfo(dtype).min
    q_idx = torch.arange(S, device=DEV).view(S, 1)
    k_idx = torch.arange(past + S, device=DEV).view(1, past + S)
    return torch.where(k_idx <= past + q_idx, torch.zeros((), device=DEV, dtype=dtype),
                       torch.full((), lo, device=DEV, dtype=dtype))[None, None]


@pytest.mark.parametrize("page", [128, 256, 512])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_page_sizes_decode_and_chunk_with_host_pages(page, dtype):
    Hq, Hkv, D = 32, 8, 128
    G = Hq // Hkv
    n_pages = 24
    T = n_pages * page - page // 3                  # a partial last page
    host_pages = 9
    es = torch.tensor([], dtype=dtype).element_size()
    page_bytes = 2 * Hkv * page * D * es
    # HELM's watermark bounds the evictable bytes (full, non-tail device
    # pages, kv_cache.py:224-235): 23 of them, so 9 go to the host
    mgr = KVCacheManager(KVAllocator(1, Hkv, D, page_size=page, dtype=dtype),
                         gpu_high_watermark_bytes=(n_pages - 1 - host_pages) * page_bytes)
    g = torch.Generator(device=DEV).manual_seed(page + es)
    k = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    v = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    mgr.append_prefill(0, k, v)
    states = [p.state for p in mgr.layers[0].pages]
    assert states == ["CPU"] * host_pages + ["GPU"] * (n_pages - host_pages), states
    K, V = _layer_kv(mgr)
    assert torch.equal(K, k[0].cpu()) and torch.equal(V, v[0].cpu())

    # perform_streaming_attention over the page list: masked loop and Path 3
    q = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=dtype)
    dmask = torch.zeros(1, 1, 1, T, device=DEV, dtype=dtype)
    out_m = perform_streaming_attention(q, mgr.iterate_layer_pages(0), attention_mask=dmask)
    out_u = perform_streaming_attention(q, mgr.iterate_layer_pages(0))
    assert _err(out_m[0], q[0].cpu(), K, V, G) <= TOL[dtype]
    assert _err(out_u[0], q[0].cpu(), K, V, G) <= TOL[dtype]

    # one decode step through the batched decode of the patched forwards
    kn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
    vn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
    q2 = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=dtype)
    dmask2 = torch.zeros(1, 1, 1, T + 1, device=DEV, dtype=dtype)
    out_d = _decode_batched([mgr], q2, kn, vn, 0, 1 / math.sqrt(D), dmask2)
    K2, V2 = _layer_kv(mgr)
    assert torch.equal(K2, torch.cat([K, kn[0].cpu()], 1))
    assert torch.equal(V2, torch.cat([V, vn[0].cpu()], 1))
    assert _err(out_d[0], q2[0].cpu(), K2, V2, G) <= TOL[dtype]

    # a prompt chunk of 96 tokens after T + 1 cached tokens, HELM's chunk mask
    S = 96
    past = T + 1
    kc = torch.randn((1, Hkv, S, D), generator=g, device=DEV, dtype=dtype)
    vc = torch.randn((1, Hkv, S, D), generator=g, device=DEV, dtype=dtype)
    qc = torch.randn((1, Hq, S, D), generator=g, device=DEV, dtype=dtype)
    mgr.append_prefill(0, kc, vc)
    K3, V3 = _layer_kv(mgr)
    assert torch.equal(K3, torch.cat([K2, kc[0].cpu()], 1))
    cmask = _chunk_mask(past, S, dtype)
    out_c = perform_streaming_attention(qc, mgr.iterate_layer_pages(0), attention_mask=cmask)
    torch.cuda.synchronize()
    assert _err(out_c[0], qc[0].cpu(), K3, V3, G, mask=cmask.float().cpu().numpy()) \
        <= TOL[dtype]
    mgr.clear()


@pytest.mark.parametrize("page", [128, 512])
def test_page_sizes_many_pages_per_split(page):
    """All-resident layers long enough that a split walks many pages of many
    blocks (Qwen3-8B shape, 8k / 32k tokens): decode through
    _decode_batched and a 512-token chunk, against fp64 on sampled heads."""
    Hq, Hkv, D = 32, 8, 128
    G = Hq // Hkv
    T = 64 * page - 5
    dtype = torch.bfloat16
    mgr = KVCacheManager(KVAllocator(1, Hkv, D, page_size=page, dtype=dtype),
                         gpu_high_watermark_bytes=1 << 40)
    g = torch.Generator(device=DEV).manual_seed(page)
    k = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    v = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=dtype)
    mgr.append_prefill(0, k, v)
    kn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
    vn = torch.randn((1, Hkv, 1, D), generator=g, device=DEV, dtype=dtype)
    q = torch.randn((1, Hq, 1, D), generator=g, device=DEV, dtype=dtype)
    out = _decode_batched([mgr], q, kn, vn, 0, 1 / math.sqrt(D))
    K, V = _layer_kv(mgr)
    assert torch.equal(K[:, :T], k[0].cpu()) and torch.equal(K[:, T:], kn[0].cpu())
    assert _err(out[0], q[0].cpu(), K, V, G) <= 1e-2
    S = 512
    kc = torch.randn((1, Hkv, S, D), generator=g, device=DEV, dtype=dtype)
    vc = torch.randn((1, Hkv, S, D), generator=g, device=DEV, dtype=dtype)
    qc = torch.randn((1, Hq, S, D), generator=g, device=DEV, dtype=dtype)
    mgr.append_prefill(0, kc, vc)
    cmask = _chunk_mask(T + 1, S, dtype)
    out_c = perform_streaming_attention(qc, mgr.iterate_layer_pages(0), attention_mask=cmask)
    torch.cuda.synchronize()
    K3, V3 = _layer_kv(mgr)
    rows = [0, 1, 200, 511]                       # sampled chunk rows of two KV heads
    m = cmask[:, :, rows].float().cpu().numpy()
    for kvh in (0, 3):
        hs = slice(kvh * G, (kvh + 1) * G)
        ref = A.attention_fp64(qc[:, hs][:, :, rows].float().cpu(),
                               K3[None, kvh:kvh + 1].float(), V3[None, kvh:kvh + 1].float(),
                               mask=m)
        got = out_c[0, hs][:, rows].double().cpu()
        assert (got - torch.from_numpy(ref[0])).abs().max().item() <= 1e-2
    mgr.clear()
