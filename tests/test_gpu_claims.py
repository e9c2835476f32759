"""Dynamic block claiming in the matrix-core decode kernel (GPU,
HELM_AMD_CLAIM=1): the waves of a tile's workgroups share its 16-token blocks
through one counter per tile instead of a fixed split of pages.

Every case is checked against the float64 oracle at HELM's tolerances, on
calls in a row (each call's merge must leave the counters at zero for the
next: a counter left over would make the next call skip blocks), with the
split merge in its own kernel and in-kernel (the last split zeroes the
counter).  The decode step that writes its token inside the attention kernel
(helm_paged_attn_seqs_append) is covered with pages of 16 and 64 tokens: the
wave that claims the token's block writes it first.  The workspace's ticket
region reads zero after every call.
"""
import math

import pytest
import torch

from helm_amd import paged
from helm_amd import workloads as W
from helm_amd.paged import paged_decode_attention
from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager
from helm_amd.runtime.kv_offload import _decode_batched
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(autouse=True)
def claims(monkeypatch):
    monkeypatch.setenv("HELM_AMD_CLAIM", "1")


def _pool_kv(case, w, b):
    """Sequence b's K, V [Hkv, T, D] gathered from the pool on the CPU."""
    T = case["lens_list"][b]
    n = case["n_pages"][b]
    slots = case["table_cpu"][b, :n].long()
    pool = case["pool"][slots.to(DEV)].cpu()
    K = pool[:, 0].permute(1, 0, 2, 3).reshape(w.Hkv, n * w.page_size, w.D)[:, :T]
    V = pool[:, 1].permute(1, 0, 2, 3).reshape(w.Hkv, n * w.page_size, w.D)[:, :T]
    return K, V


def _err(out_b, q_b, K, V, G, heads, mask=None):
    worst = 0.0
    for kvh in heads:
        hs = slice(kvh * G, (kvh + 1) * G)
        ref = A.attention_fp64_batched(q_b[hs].float().cpu(), K[kvh:kvh + 1].float(),
                                       V[kvh:kvh + 1].float(), mask=mask)
        worst = max(worst, (out_b[hs].double().cpu() - ref).abs().max().item())
    return worst


@pytest.mark.parametrize("merge", ["auto", "fused"])
@pytest.mark.parametrize("name", ["qwen3-8b-32k", "qwen3-0.6b-2k", "qwen3-14b-ragged-b8"])
def test_pool_entry_with_claims(name, merge, monkeypatch):
    monkeypatch.setenv("HELM_AMD_MERGE", merge)
    w = W.WORKLOADS[name]
    case = W.make_pool_case(w, seed=41, device=DEV)
    args = dict(max_pages=case["max_pages"], total_pages=sum(case["n_pages"]))
    outs = []
    for _ in range(3):
        outs.append(paged_decode_attention(case["q"], case["k_pool"], case["v_pool"],
                                           case["table"], case["lens"], **args))
    torch.cuda.synchronize()
    need = paged._native.load().helm_query_workspace_bytes(
        w.B, w.Hq, w.Hkv, 1, w.D, case["max_pages"], w.page_size, 0)
    ws = paged.workspace(DEV, need)
    assert not bool(ws[:64 << 10].any()), "ticket region not zero after the calls"
    tol = 2e-3 if w.dtype == torch.float16 else 1e-2
    for b in range(min(w.B, 3)):
        K, V = _pool_kv(case, w, b)
        for out in outs:
            assert _err(out[b], case["q"][b], K, V, w.Hq // w.Hkv, [0, w.Hkv - 1]) <= tol
        # two calls differ at most by the order of fp32 sums
        assert (outs[0][b].float() - outs[2][b].float()).abs().max().item() <= tol


@pytest.mark.parametrize("page", [16, 64])
@pytest.mark.parametrize("masked", [False, True])
def test_decode_steps_write_their_token_with_claims(page, masked):
    """Three decode steps of a ragged batch through _decode_batched: each
    step's token written by the wave that claims its block; the pages hold
    exactly the tokens appended, and each step's output equals fp64."""
    Hq, Hkv, D = 32, 8, 128
    lens = [3000, 1200, 4097, 64]
    g = torch.Generator(device=DEV).manual_seed(page)
    alloc = KVAllocator(1, Hkv, D, page_size=page, dtype=torch.bfloat16)
    mgrs = [KVCacheManager(alloc, gpu_high_watermark_bytes=1 << 40) for _ in lens]
    Ks, Vs = [], []
    for m, T in zip(mgrs, lens):
        k = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=torch.bfloat16)
        v = torch.randn((1, Hkv, T, D), generator=g, device=DEV, dtype=torch.bfloat16)
        m.append_prefill(0, k, v)
        Ks.append(k[0].cpu())
        Vs.append(v[0].cpu())
    for step in range(3):
        B = len(lens)
        q = torch.randn((B, Hq, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
        kn = torch.randn((B, Hkv, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
        vn = torch.randn((B, Hkv, 1, D), generator=g, device=DEV, dtype=torch.bfloat16)
        T = max(lens) + step + 1
        mask = None
        if masked:
            mask = torch.zeros((B, 1, 1, T), device=DEV, dtype=torch.bfloat16)
            mask[:, ..., 7:40] = torch.finfo(torch.bfloat16).min
        out = _decode_batched(mgrs, q, kn, vn, 0, 1 / math.sqrt(D), mask)
        torch.cuda.synchronize()
        for i in range(B):
            Ks[i] = torch.cat([Ks[i], kn[i].cpu()], 1)
            Vs[i] = torch.cat([Vs[i], vn[i].cpu()], 1)
            pages = [p for p in mgrs[i].layers[0].pages if p.used_tokens > 0]
            Kg = torch.cat([p.k_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
            Vg = torch.cat([p.v_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
            assert torch.equal(Kg, Ks[i]) and torch.equal(Vg, Vs[i])
            n = Ks[i].shape[1]
            mk = None if mask is None else mask[i, :, :, :n].float().cpu()
            assert _err(out[i], q[i], Ks[i], Vs[i], Hq // Hkv, [0, 5], mask=mk) <= 1e-2


def test_claims_match_the_static_split_within_rounding(monkeypatch):
    w = W.WORKLOADS["qwen3-8b-32k"]
    case = W.make_pool_case(w, seed=43, device=DEV)
    run = lambda: paged_decode_attention(case["q"], case["k_pool"], case["v_pool"],
                                         case["table"], case["lens"],
                                         max_pages=case["max_pages"])
    dyn = run()
    monkeypatch.setenv("HELM_AMD_CLAIM", "0")
    static = run()
    torch.cuda.synchronize()
    assert (dyn.float() - static.float()).abs().max().item() <= 1e-2
