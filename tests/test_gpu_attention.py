"""Parity of the HIP decode-attention kernels with the oracle (GPU).

* the pool entry point (helm_paged_decode_attn) at every benchmark shape —
  the Qwen3-0.6B, Qwen3-8B and Llama-2-13B shapes at full context, the
  ragged Qwen3-14B batch at full context — against the float64 oracle,
  within 2e-3 (fp16) / 1e-2 (bf16);
* perform_streaming_attention over hand-built pages (HELM's test shapes:
  ragged pages, D = 4..256, fp32/fp16/bf16 queries, masks, soft-cap, GQA,
  q_len > 1 with a causal chunk mask) against the oracle's restatement of
  HELM's own CPU path and the float64 formula;
* size-independent properties at full size (page-table permutation
  invariance, split-count invariance).
"""
import math

import numpy as np
import pytest
import torch

from helm_amd import workloads as W
from helm_amd.paged import paged_decode_attention
from helm_amd.runtime.kv_cache import KVPage, perform_streaming_attention
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-5}


@pytest.fixture(params=[("auto", "auto"), ("auto", "fused"), ("auto", "kernel"),
                        ("valu", "auto"), ("valu", "fused")],
                ids=lambda p: f"{p[0]}-{p[1]}")
def kernel(request, monkeypatch):
    """Runs a test on the matrix-core kernel (the automatic choice for 16-bit
    D = 128 pages) and on the vector-ALU kernels, with the split merge chosen
    automatically, in-kernel by the last split (fused) and by
    merge_splits_kernel."""
    monkeypatch.setenv("HELM_AMD_KERNEL", request.param[0])
    monkeypatch.setenv("HELM_AMD_MERGE", request.param[1])
    return request.param


def _pool_reference(case, w, b, mask=None, softcap=None):
    """fp64 oracle for sequence b of a pool case (gathers its pages on CPU)."""
    T = case["lens_list"][b]
    n = case["n_pages"][b]
    slots = case["table_cpu"][b, :n].long()
    pool = case["pool"][slots.to(DEV)].cpu()                 # [n, 2, Hkv, P, D]
    K = pool[:, 0].permute(1, 0, 2, 3).reshape(w.Hkv, n * w.page_size, w.D)[:, :T]
    V = pool[:, 1].permute(1, 0, 2, 3).reshape(w.Hkv, n * w.page_size, w.D)[:, :T]
    q = case["q"][b].cpu()                                    # [Hq, 1, D]
    return A.attention_fp64_batched(q, K, V, scale=case["scale"], mask=mask, softcap=softcap)


def _check_pool(w, case, out, atol=None):
    atol = atol or TOL[w.dtype]
    worst = 0.0
    for b in range(w.B):
        ref = _pool_reference(case, w, b)
        err = (out[b].double().cpu() - ref).abs().max().item()
        worst = max(worst, err)
    assert worst <= atol, f"max abs err {worst} > {atol}"
    return worst


@pytest.mark.parametrize("name,T", [
    ("qwen3-0.6b-2k", None),          # full Qwen3-0.6B shape, fp16
    ("qwen3-8b-32k", 4096),
    ("qwen3-8b-32k", None),           # full 32k Qwen3-8B shape, bf16
    ("llama2-13b-128k-offload75", 8192),
])
def test_pool_decode_matches_fp64(name, T, kernel):
    w = W.WORKLOADS[name]
    lens = [T] * w.B if T else None
    case = W.make_pool_case(w, seed=17, device=DEV, lens=lens)
    out = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                 case["lens"], max_pages=case["max_pages"])
    torch.cuda.synchronize()
    print(name, "max err", _check_pool(w, case, out))


def test_pool_decode_ragged_batch_full_size(kernel):
    w = W.WORKLOADS["qwen3-14b-ragged-b8"]
    case = W.make_pool_case(w, seed=3, device=DEV)
    out = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                 case["lens"], max_pages=case["max_pages"],
                                 total_pages=sum(case["n_pages"]))
    torch.cuda.synchronize()
    _check_pool(w, case, out)


def test_workspace_reused_across_shapes(kernel):
    """One workspace for a long single-sequence call (its split counts and
    partials fill the workspace) and then a batch of short sequences with 20x
    the tiles, merged in-kernel: the tickets sit in their own region, so the
    second call does not see the first call's bytes as tickets."""
    long_w = W.WORKLOADS["qwen3-8b-32k"]
    short_w = W.Workload("short-b20", 20, 32, 8, 128, torch.bfloat16, T_range=(100, 400))
    for w, seed in ((long_w, 1), (short_w, 5), (long_w, 2), (short_w, 6)):
        case = W.make_pool_case(w, seed=seed, device=DEV)
        out = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                     case["lens"], max_pages=case["max_pages"],
                                     total_pages=sum(case["n_pages"]))
        torch.cuda.synchronize()
        _check_pool(w, case, out)


@pytest.mark.parametrize("pps", [1, 3, 8, 64, 256])
def test_pool_decode_split_invariance(pps, kernel):
    """Any split count gives the same attention (merge correctness)."""
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=5, device=DEV, lens=[3000])
    out = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                 case["lens"], max_pages=case["max_pages"], pages_per_split=pps)
    torch.cuda.synchronize()
    _check_pool(w, case, out)


def test_pool_decode_page_table_permutation_invariance(kernel):
    """Full-size property: relocating pages (new table, moved slots) leaves
    the output bit-identical for the same split plan."""
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=9, device=DEV)
    args = dict(max_pages=case["max_pages"], pages_per_split=32)
    out1 = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                  case["lens"], **args)
    perm = torch.randperm(case["pool"].shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    pool2 = case["pool"][perm.to(DEV)]                     # slot s of pool2 = slot perm[s]
    table2 = inv.to(DEV)[case["table"].long()].to(torch.int32)
    out2 = paged_decode_attention(case["q"], pool2[:, 0], pool2[:, 1], table2, case["lens"], **args)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_pool_decode_mask_and_softcap(kernel):
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=21, device=DEV, lens=[1000])
    g = torch.Generator().manual_seed(0)
    mask = torch.zeros(1, 1, 1, 1000)
    mask[..., torch.randperm(1000, generator=g)[:300]] = torch.finfo(torch.float32).min
    out = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                 case["lens"], max_pages=case["max_pages"], softcap=30.0,
                                 attention_mask=mask.to(DEV))
    torch.cuda.synchronize()
    ref = _pool_reference(case, w, 0, mask=mask[0], softcap=30.0)
    assert (out[0].double().cpu() - ref).abs().max().item() <= TOL[w.dtype]


# ── perform_streaming_attention on hand-built pages (HELM's test shapes) ──────
def _page(k, v, i=0, start=0, state="GPU"):
    return KVPage(page_id=i, layer_id=0, start_token=start, used_tokens=k.size(2),
                  capacity_tokens=k.size(2), k_tensor=k.clone(), v_tensor=v.clone(),
                  device=k.device, state=state)


def _paged(sizes, H, D, kvh, dtype, seed, device=DEV):
    g = torch.Generator().manual_seed(seed)
    ks = [torch.randn(1, kvh, n, D, generator=g).to(dtype) for n in sizes]
    vs = [torch.randn(1, kvh, n, D, generator=g).to(dtype) for n in sizes]
    q = torch.randn(1, H, 1, D, generator=g).to(dtype)
    pages, start = [], 0
    for i, (k, v) in enumerate(zip(ks, vs)):
        pages.append(_page(k.to(device), v.to(device), i, start))
        start += k.size(2)
    return q, pages, ks, vs


@pytest.mark.parametrize("sizes,H,kvh,D,dtype", [
    ([4], 2, 2, 8, torch.float32), ([4, 3], 2, 2, 8, torch.float32),
    ([3, 5, 2], 1, 1, 16, torch.float32), ([6], 4, 2, 8, torch.float32),
    ([4, 3], 4, 2, 8, torch.float32), ([3], 1, 1, 4, torch.float32),
    ([16] * 5 + [3], 16, 8, 128, torch.float16), ([16] * 9, 32, 8, 128, torch.bfloat16),
    ([64, 64, 17], 8, 8, 64, torch.bfloat16), ([16, 16], 8, 4, 256, torch.float16),
    ([5, 16, 16], 40, 8, 128, torch.bfloat16), ([7, 9], 6, 2, 96, torch.float32),
])
@pytest.mark.parametrize("masked", [False, True])
def test_streaming_matches_oracle(sizes, H, kvh, D, dtype, masked, kernel):
    q, pages, ks, vs = _paged(sizes, H, D, kvh, dtype, seed=sum(sizes) * 7 + H)
    T = sum(sizes)
    mask = None
    if masked:
        mask = torch.zeros(1, 1, 1, T)
        mask[..., [0, T // 2, T - 1]] = torch.finfo(torch.float32).min
    out = perform_streaming_attention(q.to(DEV), pages,
                                      attention_mask=None if mask is None else mask.to(DEV))
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == q.shape
    ref_helm = A.streaming_attention(q, list(zip(ks, vs)), attention_mask=mask)
    ref64 = A.attention_fp64(q.float(), torch.cat(ks, 2).float(), torch.cat(vs, 2).float(),
                             mask=None if mask is None else mask.numpy())
    tol = TOL[dtype]
    assert (out.double().cpu() - torch.from_numpy(ref64)).abs().max().item() <= tol
    assert (out.double().cpu() - ref_helm.double()).abs().max().item() <= tol + TOL[dtype]


def test_streaming_softcap_and_custom_scale():
    q, pages, ks, vs = _paged([3, 5], 2, 8, 2, torch.float32, seed=3)
    out = perform_streaming_attention(q.to(DEV), pages, scale=0.25, softcap=50.0)
    ref = A.attention_fp64(q, torch.cat(ks, 2), torch.cat(vs, 2), scale=0.25, softcap=50.0)
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=1e-5)


def test_streaming_fp32_query_over_bf16_pages():
    q, pages, ks, vs = _paged([16] * 4, 32, 128, 8, torch.bfloat16, seed=8)
    q32 = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(1))
    out = perform_streaming_attention(q32.to(DEV), pages)
    assert out.dtype == torch.float32
    ref = A.attention_fp64(q32, torch.cat(ks, 2).float(), torch.cat(vs, 2).float())
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=1e-5)


def test_streaming_empty_and_zero_used_pages():
    q = torch.randn(1, 2, 1, 8, device=DEV)
    assert torch.all(perform_streaming_attention(q, []) == 0)
    qc, pages, ks, vs = _paged([4], 2, 8, 2, torch.float32, seed=1)
    empty = _page(torch.zeros(1, 2, 4, 8, device=DEV), torch.zeros(1, 2, 4, 8, device=DEV))
    empty.used_tokens = 0
    a = perform_streaming_attention(qc.to(DEV), [empty] + pages)
    b = perform_streaming_attention(qc.to(DEV), pages)
    torch.testing.assert_close(a, b, atol=1e-6, rtol=0)
    assert torch.all(perform_streaming_attention(qc.to(DEV), [empty]) == 0)


def test_streaming_large_logits_finite():
    q = torch.ones(1, 1, 1, 64, device=DEV) * 100.0
    k = torch.ones(1, 1, 8, 64, device=DEV) * 100.0
    v = torch.randn(1, 1, 8, 64, device=DEV)
    out = perform_streaming_attention(q, [_page(k, v)])
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out[0, 0, 0], v[0, 0].mean(0), atol=1e-5, rtol=0)


def test_streaming_fully_masked_page_and_all_masked():
    q, pages, ks, vs = _paged([4, 4], 2, 8, 2, torch.float32, seed=2)
    mask = torch.zeros(1, 1, 1, 8)
    mask[..., :4] = torch.finfo(torch.float32).min
    out = perform_streaming_attention(q.to(DEV), pages, attention_mask=mask.to(DEV))
    ref = A.attention_fp64(q, ks[1], vs[1])
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=1e-5)
    # every key at finfo.min: HELM's loop weighs them uniformly (mean of V)
    mask[...] = torch.finfo(torch.float32).min
    out = perform_streaming_attention(q.to(DEV), pages, attention_mask=mask.to(DEV))
    helm = A.online_softmax_pages(q, list(zip(ks, vs)), attention_mask=mask)
    torch.testing.assert_close(out.cpu(), helm, atol=1e-5, rtol=0)


def test_streaming_prefill_chunk_causal_mask(kernel):
    """q_len > 1 (later prefill chunk) with the pipeline's chunk mask
    (pipeline_runtime.py:94-113): queries at [past, past+n) see keys <= own."""
    q_, pages, ks, vs = _paged([16, 16, 16, 5], 8, 64, 4, torch.float16, seed=4)
    past, n = 37, 16
    T = past + n
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 8, n, 64, generator=g).half()
    mn = torch.finfo(torch.float32).min
    mask = torch.where(torch.arange(T)[None, :] <= past + torch.arange(n)[:, None],
                       torch.zeros(()), torch.full((), mn))[None, None]
    out = perform_streaming_attention(q.to(DEV), pages, attention_mask=mask.to(DEV))
    ref = A.attention_fp64(q.float(), torch.cat(ks, 2).float(), torch.cat(vs, 2).float(),
                           mask=mask.numpy())
    assert np.abs(out.cpu().double().numpy() - ref).max() <= 2e-3


def test_streaming_path1_causal_top_left(kernel):
    """All-GPU, no mask, q_len > 1: HELM's Path 1 SDPA is_causal (top-left)."""
    q_, pages, ks, vs = _paged([8, 8], 4, 16, 2, torch.float32, seed=6)
    q = torch.randn(1, 4, 5, 16, generator=torch.Generator().manual_seed(6))
    out = perform_streaming_attention(q.to(DEV), pages)
    ref = A.attention_fp64(q, torch.cat(ks, 2), torch.cat(vs, 2), causal=True)
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=1e-5)


def test_streaming_batched_query_over_batched_pages():
    """HELM test_output_shape_matches_query: a [B,...] page batch pairs with
    the query batch."""
    g = torch.Generator().manual_seed(12)
    q = torch.randn(2, 4, 1, 16, generator=g)
    k = torch.randn(2, 4, 6, 16, generator=g)
    v = torch.randn(2, 4, 6, 16, generator=g)
    out = perform_streaming_attention(q.to(DEV), [_page(k.to(DEV), v.to(DEV))])
    assert out.shape == (2, 4, 1, 16)
    ref = A.attention_fp64(q, k, v)
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=1e-5)


@pytest.mark.parametrize("Hq,Hkv,S,dtype", [(40, 2, 1, torch.bfloat16), (8, 4, 16, torch.bfloat16),
                                            (4, 4, 5, torch.float16)])
def test_streaming_d128_row_tiles_causal_and_chunk_mask(Hq, Hkv, S, dtype, kernel):
    """D = 128 with more than 16 query rows per KV head (several row tiles):
    a later prefill chunk under the pipeline's chunk mask, and Path 1's
    top-left causal mask."""
    g = torch.Generator().manual_seed(Hq * 7 + S)
    sizes = [16, 16, 16, 16, 9]
    T = sum(sizes)
    ks = [torch.randn(1, Hkv, n, 128, generator=g).to(dtype) for n in sizes]
    vs = [torch.randn(1, Hkv, n, 128, generator=g).to(dtype) for n in sizes]
    pages, start = [], 0
    for i, (k, v) in enumerate(zip(ks, vs)):
        pages.append(_page(k.to(DEV), v.to(DEV), i, start))
        start += k.size(2)
    q = torch.randn(1, Hq, S, 128, generator=g).to(dtype)
    K, V = torch.cat(ks, 2).float(), torch.cat(vs, 2).float()
    past = T - S
    mn = torch.finfo(torch.float32).min
    mask = torch.where(torch.arange(T)[None, :] <= past + torch.arange(S)[:, None],
                       torch.zeros(()), torch.full((), mn))[None, None]
    out = perform_streaming_attention(q.to(DEV), pages, attention_mask=mask.to(DEV))
    ref = A.attention_fp64(q.float(), K, V, mask=mask.numpy())
    assert np.abs(out.cpu().double().numpy() - ref).max() <= TOL[dtype]
    if S > 1:
        out = perform_streaming_attention(q.to(DEV), pages)        # Path 1: is_causal
        ref = A.attention_fp64(q.float(), K, V, causal=True)
        assert np.abs(out.cpu().double().numpy() - ref).max() <= TOL[dtype]


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("pps", [0, 3])
@pytest.mark.parametrize("variant", ["chunk_mask", "causal", "softcap_mask"])
def test_chunk32_workgroup_shapes(waves, pps, variant, monkeypatch):
    """The 32-row chunk kernel with four- and eight-wave workgroups: 320 query
    rows per KV head (an eight-wave workgroup of 256 rows and one with two
    active waves), ragged pages, one or several splits, under HELM's chunk
    mask, Path 1's causal mask and a soft-cap with the mask, against fp64."""
    monkeypatch.setenv("HELM_AMD_CHUNK_WAVES", str(waves))
    if pps:
        monkeypatch.setenv("HELM_AMD_PPS", str(pps))
    Hq, Hkv, S, dtype = 32, 8, 80, torch.bfloat16
    g = torch.Generator().manual_seed(1000 + waves + pps)
    sizes = [16] * 9 + [11, 16, 16, 5, 16, 16, 16, 16, 16]
    T = sum(sizes)
    ks = [torch.randn(1, Hkv, n, 128, generator=g).to(dtype) for n in sizes]
    vs = [torch.randn(1, Hkv, n, 128, generator=g).to(dtype) for n in sizes]
    pages, start = [], 0
    for i, (k, v) in enumerate(zip(ks, vs)):
        pages.append(_page(k.to(DEV), v.to(DEV), i, start))
        start += k.size(2)
    q = (2 * torch.randn(1, Hq, S, 128, generator=g)).to(dtype)
    K, V = torch.cat(ks, 2).float(), torch.cat(vs, 2).float()
    past = T - S
    mn = torch.finfo(torch.float32).min
    mask = torch.where(torch.arange(T)[None, :] <= past + torch.arange(S)[:, None],
                       torch.zeros(()), torch.full((), mn))[None, None]
    if variant == "causal":
        out = perform_streaming_attention(q.to(DEV), pages)
        ref = A.attention_fp64(q.float(), K, V, causal=True)
    elif variant == "chunk_mask":
        out = perform_streaming_attention(q.to(DEV), pages, attention_mask=mask.to(DEV))
        ref = A.attention_fp64(q.float(), K, V, mask=mask.numpy())
    else:
        # a mask that is not the chunk pattern (every 7th key hidden as well),
        # so the kernel reads it, with a soft-cap of 30
        m2 = mask.clone()
        m2[..., ::7] = mn
        m2[..., 0] = 0.0
        out = perform_streaming_attention(q.to(DEV), pages, attention_mask=m2.to(DEV), softcap=30.0)
        ref = A.attention_fp64(q.float(), K, V, mask=m2.numpy(), softcap=30.0)
    # rows that see a few keys reach |out| > 4, where the bf16 output's own
    # rounding (half an ulp: 2^-9 relative) exceeds 1e-2: that term is added
    err = np.abs(out.cpu().double().numpy() - ref)
    assert (err <= TOL[dtype] + np.abs(ref) * 2.0 ** -9).all()


@pytest.mark.parametrize("scale", [0.05, -0.07, 0.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunk32_causal_scale_sign(scale, dtype):
    """The chunk kernel under caller-chosen softmax scales: a custom one, a
    negative one (the running max must follow the scaled logits, not the raw
    q . k) and zero (uniform weights over each row's visible keys).  Path 1's
    causal mask, 320 query rows per KV head, against fp64."""
    Hq, Hkv, S = 32, 8, 80
    g = torch.Generator().manual_seed(77 + int(scale * 100) + (dtype == torch.float16))
    sizes = [16] * 7 + [9, 16, 16, 3]
    ks = [torch.randn(1, Hkv, n, 128, generator=g).to(dtype) for n in sizes]
    vs = [torch.randn(1, Hkv, n, 128, generator=g).to(dtype) for n in sizes]
    pages, start = [], 0
    for i, (k, v) in enumerate(zip(ks, vs)):
        pages.append(_page(k.to(DEV), v.to(DEV), i, start))
        start += k.size(2)
    q = (3 * torch.randn(1, Hq, S, 128, generator=g)).to(dtype)
    K, V = torch.cat(ks, 2).float(), torch.cat(vs, 2).float()
    out = perform_streaming_attention(q.to(DEV), pages, scale=scale)
    ref = A.attention_fp64(q.float(), K, V, scale=scale, causal=True)
    err = np.abs(out.cpu().double().numpy() - ref)
    assert (err <= TOL[dtype] + np.abs(ref) * 2.0 ** -9).all()


def test_kernels_agree_at_full_size():
    """The matrix-core and vector-ALU kernels give the same attention (to
    fp32 rounding of their different summation orders) on the full 32k
    Qwen3-8B shape."""
    import os
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=31, device=DEV)
    outs = {}
    for kind in ("auto", "valu"):
        os.environ["HELM_AMD_KERNEL"] = kind
        try:
            o = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                       case["lens"], max_pages=case["max_pages"])
        finally:
            os.environ.pop("HELM_AMD_KERNEL", None)
        torch.cuda.synchronize()
        outs[kind] = o.float()
    assert (outs["auto"] - outs["valu"]).abs().max().item() <= 2 ** -7


@pytest.mark.parametrize("groups", [2, 4, 32])
def test_merge_kernel_column_groups(groups, monkeypatch):
    """merge_splits_kernel split over column groups gives the same attention."""
    monkeypatch.setenv("HELM_AMD_MERGE", "kernel")
    monkeypatch.setenv("HELM_AMD_MERGE_GROUPS", str(groups))
    w = W.WORKLOADS["qwen3-14b-ragged-b8"]
    case = W.make_pool_case(w, seed=13, device=DEV, lens=[5000, 77, 1200, 3333, 16, 1, 4096, 900])
    out = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                 case["lens"], max_pages=case["max_pages"], pages_per_split=8)
    torch.cuda.synchronize()
    _check_pool(w, case, out)


def test_split_kernel_timing_hook():
    """helm_profile_split_kernels times the attention kernel of exactly the
    next n calls (positive, below each call's whole time) and changes no
    output bit; n = 0 disarms."""
    from helm_amd import _native
    w = W.Workload("t", 1, 32, 8, 128, torch.bfloat16, T=8192)
    case = W.make_pool_case(w, seed=23, device=DEV)
    args = (case["q"], case["k_pool"], case["v_pool"], case["table"], case["lens"])
    ref = paged_decode_attention(*args, max_pages=case["max_pages"])
    lib = _native.load()
    _native.call("helm_profile_split_kernels", 3)
    try:
        outs = [paged_decode_attention(*args, max_pages=case["max_pages"]) for _ in range(5)]
        torch.cuda.synchronize()
        buf = np.zeros(8, dtype=np.float32)
        n = lib.helm_profile_split_read(_native.ptr(buf), 8)
    finally:
        _native.call("helm_profile_split_kernels", 0)
    assert n == 3                                 # only the armed calls
    assert (buf[:3] > 0).all() and (buf[:3] < 10_000).all() and (buf[3:] == 0).all()
    for out in outs:
        assert torch.equal(out, ref)
    assert lib.helm_profile_split_read(_native.ptr(buf), 8) == 0   # disarmed: nothing timed


@pytest.mark.parametrize("T", [2048, 4096], ids=["merge-in-kernel", "merge-kernel"])
def test_static_decode_replays_from_a_hip_graph(T):
    """The decode entry point that allocates nothing, captured in a HIP graph
    (torch.cuda.CUDAGraph): every replay, with eager work and synchronizations
    between the replays, equals the eager call bit for bit — with the split
    merge in the decode kernel (16 splits: its tickets, left zero by every
    call) and in a second kernel (32 splits)."""
    from helm_amd import _native, paged
    w = W.Workload("graph", 1, 32, 8, 128, torch.bfloat16, T=T)
    case = W.make_pool_case(w, seed=29, device=DEV)

    def static_call(out):
        # the C-ABI arguments on torch's current stream (the capture stream
        # inside the graph context)
        args, keep = paged._decode_args(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                        case["lens"], case["max_pages"], sum(case["n_pages"]),
                                        None, None, None, out, 0)
        _native.call("helm_paged_decode_attn_static", *(list(args[:-3]) + [args[-1]]))
        return keep

    eager = torch.empty_like(case["q"])
    keep = [static_call(eager)]
    torch.cuda.synchronize()
    out = torch.empty_like(case["q"])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):            # a warm-up call on a side stream first
        keep.append(static_call(out))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        keep.append(static_call(out))
    x = torch.randn(1024, 1024, device=DEV)
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager call"
        x = (x @ x).clamp_(-1, 1)            # eager work between the replays
        torch.cuda.synchronize()


# ── the committed golden fixtures through the HIP path ───────────────────────
def _golden_cases():
    import os
    d = os.path.join(os.path.dirname(__file__), "golden")
    return sorted(f[:-4] for f in os.listdir(d) if f.endswith(".npz"))


@pytest.mark.parametrize("name", _golden_cases())
def test_golden_fixtures_on_the_gpu(name, kernel):
    """Each fixture of tests/golden/ (seeded inputs in the page sizes it
    lists and their float64 output) through perform_streaming_attention on
    the GPU, within the fixture's tolerance; every kernel and merge choice."""
    import json
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", f"{name}.npz"))
    meta = json.loads(str(z["meta"]))
    dtype = getattr(torch, meta["dtype"])
    q = torch.from_numpy(z["q"]).to(dtype)
    K = torch.from_numpy(z["K"]).to(dtype)
    V = torch.from_numpy(z["V"]).to(dtype)
    pages, t = [], 0
    for i, n in enumerate(meta["page_sizes"]):
        pages.append(_page(K[:, :, t:t + n].to(DEV), V[:, :, t:t + n].to(DEV), i, t))
        t += n
    mask = torch.from_numpy(z["mask"]).to(DEV) if "mask" in z.files else None
    out = perform_streaming_attention(q.to(DEV), pages, scale=meta["scale"],
                                      attention_mask=mask, softcap=meta["softcap"])
    torch.cuda.synchronize()
    err = (out.double().cpu() - torch.from_numpy(z["out"])).abs().max().item()
    assert err <= meta["atol"], err


@pytest.mark.parametrize("merge", ["auto", "fused"])
def test_pool_entry_with_host_lengths(merge, monkeypatch):
    """The ragged Qwen3-14B batch through the pool entry point with the
    lengths also given on the host: the grid holds exactly the sequences'
    splits; every sequence within tolerance of fp64, as without them."""
    monkeypatch.setenv("HELM_AMD_MERGE", merge)
    w = W.WORKLOADS["qwen3-14b-ragged-b8"]
    case = W.make_pool_case(w, seed=23, device=DEV)
    args = dict(max_pages=case["max_pages"], total_pages=sum(case["n_pages"]))
    out_h = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                   case["lens"], host_lens=case["lens_list"], **args)
    out_d = paged_decode_attention(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                   case["lens"], **args)
    torch.cuda.synchronize()
    G = w.Hq // w.Hkv
    for b in range(w.B):
        ref = _pool_reference(case, w, b)
        for out in (out_h, out_d):
            err = (out[b].double().cpu() - ref).abs().max().item()
            assert err <= TOL[w.dtype], (b, err)
