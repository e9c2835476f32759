"""Additive masks in the model's dtype (GPU).

HELM's pipeline builds its masks in the model's dtype (bf16 / fp16,
helm/runtime/pipeline_runtime.py:79-113) and its loop widens each page's mask
slice to fp32 before adding it (helm/runtime/kv_cache.py:519, :535).  The
kernels read such a mask as given: a 16-bit element widens to fp32 exactly,
so every kernel must give the same bits as with the mask widened first.  The
masks here hold arbitrary values (not only 0 / finfo.min), so a wrongly
decoded element changes the output.  Masks made under torch.inference_mode()
(HELM's generate) go through the production decode call unchanged.
"""
import math

import pytest
import torch

from helm_amd import workloads as W
from helm_amd.paged import paged_decode_attention
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager, KVPage, perform_streaming_attention
from helm_amd.runtime.kv_offload import _decode_batched
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _pages(T, Hkv, D, dtype, seed, page=16):
    g = torch.Generator().manual_seed(seed)
    K = torch.randn(1, Hkv, T, D, generator=g).to(dtype)
    V = torch.randn(1, Hkv, T, D, generator=g).to(dtype)
    pages = []
    for i, t in enumerate(range(0, T, page)):
        n = min(page, T - t)
        pages.append(KVPage(page_id=i, layer_id=0, start_token=t, used_tokens=n,
                            capacity_tokens=n, k_tensor=K[:, :, t:t + n].clone().to(DEV),
                            v_tensor=V[:, :, t:t + n].clone().to(DEV), device=DEV,
                            state="GPU"))
    return K, V, pages


def _mask(shape, mdtype, seed):
    g = torch.Generator().manual_seed(seed)
    m = (torch.randn(*shape, generator=g) * 3).to(mdtype)
    m.view(-1)[::7] = torch.finfo(mdtype).min
    return m


KERNELS = ["mfma", "valu", "generic"]


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("per_head", [False, True])
def test_decode_mask_dtype_bit_equal(kernel, mdtype, per_head, monkeypatch):
    monkeypatch.setenv("HELM_AMD_KERNEL", kernel)
    Hq, Hkv, D, T = 32, 8, 128, 1000
    K, V, pages = _pages(T, Hkv, D, torch.bfloat16, seed=3)
    q = torch.randn(1, Hq, 1, D, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    m = _mask((1, Hq if per_head else 1, 1, T), mdtype, seed=5).to(DEV)
    out16 = perform_streaming_attention(q.to(DEV), pages, attention_mask=m)
    out32 = perform_streaming_attention(q.to(DEV), pages, attention_mask=m.float())
    torch.cuda.synchronize()
    assert torch.equal(out16, out32)
    ref = A.attention_fp64(q.float(), K.float(), V.float(), mask=m.float().cpu().numpy())
    assert (out16.double().cpu() - torch.from_numpy(ref)).abs().max().item() <= 1e-2


@pytest.mark.parametrize("chunk", ["32", "16", "valu"])
@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float16])
def test_chunk_mask_dtype_bit_equal(chunk, mdtype, monkeypatch):
    """A prompt chunk (q_len 40 over 300 cached tokens + its own) under a
    non-causal mask: the 32-row and 16-row matrix-core chunk kernels and the
    vector-ALU kernel."""
    if chunk == "valu":
        monkeypatch.setenv("HELM_AMD_KERNEL", "valu")
    else:
        monkeypatch.setenv("HELM_AMD_CHUNK", chunk)
    Hq, Hkv, D, T, S = 16, 4, 128, 340, 40
    K, V, pages = _pages(T, Hkv, D, torch.float16, seed=6)
    q = torch.randn(1, Hq, S, D, generator=torch.Generator().manual_seed(7)).to(torch.float16)
    m = _mask((1, 1, S, T), mdtype, seed=8).to(DEV)
    out16 = perform_streaming_attention(q.to(DEV), pages, attention_mask=m)
    out32 = perform_streaming_attention(q.to(DEV), pages, attention_mask=m.float())
    torch.cuda.synchronize()
    assert torch.equal(out16, out32)
    ref = A.attention_fp64(q.float(), K.float(), V.float(), mask=m.float().cpu().numpy())
    assert (out16.double().cpu() - torch.from_numpy(ref)).abs().max().item() <= 2e-3


@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float16])
def test_pool_entry_mask_dtype_bit_equal(mdtype):
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=11, device=DEV, lens=[3000])
    m = _mask((1, 1, 1, 3000), mdtype, seed=12).to(DEV)
    outs = [paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                   case["lens"], max_pages=case["max_pages"], attention_mask=mm)
            for mm in (m, m.float())]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_production_decode_under_inference_mode():
    """_decode_batched (HELM's decode step of one layer) under HELM's bf16
    decode mask made inside torch.inference_mode() gives the bits of the same
    mask made outside it (two caches holding the same tokens), and a change
    made to the mask in place before the next step is seen by that step."""
    Hq, Hkv, D, T = 32, 8, 128, 700
    g = torch.Generator().manual_seed(13)
    K = torch.randn(1, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    V = torch.randn(1, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    mgrs = []
    for _ in range(2):
        mgr = KVCacheManager(KVAllocator(1, Hkv, D, page_size=16, dtype=torch.bfloat16),
                             gpu_high_watermark_bytes=1 << 40)
        mgr.append_prefill(0, K, V)
        mgrs.append(mgr)
    steps = [tuple(torch.randn(1, h, 1, D, generator=g).to(torch.bfloat16).to(DEV)
                   for h in (Hq, Hkv, Hkv)) for _ in range(2)]
    lo = torch.finfo(torch.bfloat16).min
    scale = 1 / math.sqrt(D)
    plain = torch.zeros(1, 1, 1, T + 2, dtype=torch.bfloat16, device=DEV)
    plain[..., 100:300] = lo
    q, kn, vn = steps[0]
    out_a = _decode_batched([mgrs[0]], q, kn, vn, 0, scale, plain[..., :T + 1])
    with torch.inference_mode():
        m = torch.zeros(1, 1, 1, T + 2, dtype=torch.bfloat16, device=DEV)
        m[..., 100:300] = lo
        out_b = _decode_batched([mgrs[1]], q, kn, vn, 0, scale, m[..., :T + 1])
        m[..., 100:200] = 0                # in place, before the next step
    plain[..., 100:200] = 0
    q, kn, vn = steps[1]
    out_c = _decode_batched([mgrs[0]], q, kn, vn, 0, scale, plain)
    with torch.inference_mode():
        out_d = _decode_batched([mgrs[1]], q, kn, vn, 0, scale, m)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    assert torch.equal(out_c, out_d)
    Kc = torch.cat([K, steps[0][1], kn], 2)[0].float().cpu()
    Vc = torch.cat([V, steps[0][2], vn], 2)[0].float().cpu()
    ref = A.attention_fp64(q.float().cpu(), Kc[None], Vc[None], mask=plain.float().cpu().numpy())
    assert (out_d.double().cpu() - torch.from_numpy(ref)).abs().max().item() <= 1e-2
