"""HELM's contiguous all-GPU fast path on the GPU (kv_cache.py:267-354,
kv_offload.py:116-142; HELM turns it on for every all-GPU plan,
inference.py:729-731): decode through the contiguous buffers, past their
capacity, migration into pages, and decode over the pages — every phase
against the fp64 oracle, the migrated pages bit-exact."""
import math

import numpy as np
import pytest
import torch

from helm_amd.runtime.kv_allocator import KVAllocator
from helm_amd.runtime.kv_cache import KVCacheManager
from helm_amd.runtime.kv_offload import (KVOffloadConfig, KVOffloadManager,
                                         _append_prefill_batched, _decode_batched)
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
FMIN = torch.finfo(torch.float32).min


@pytest.mark.parametrize("dtype,Hq,Hkv,tol", [(torch.bfloat16, 32, 8, 1e-2),
                                              (torch.float16, 16, 8, 2e-3),
                                              (torch.float32, 8, 2, 1e-5)])
def test_contiguous_decode_migration_and_paged_decode(dtype, Hq, Hkv, tol):
    """Two sequences, two layers, D = 128: a 300-token prompt (pages and
    buffers), 20 decode steps through buffers of capacity 320, then the
    step that finds them full migrates the decoded tokens into pages and 14
    more steps decode over the pages.  HELM's decode mask with the second
    item's first 7 keys padded out (finfo.min)."""
    B, L, D, P, T0, cap, steps = 2, 2, 128, 16, 300, 320, 34
    g = torch.Generator().manual_seed(71)
    a = KVAllocator(L, Hkv, D, page_size=P, dtype=dtype)
    mgrs = [KVCacheManager(a, gpu_high_watermark_bytes=10 ** 12) for _ in range(B)]
    for m in mgrs:
        assert m.build_contiguous(L, Hkv, D, cap, DEV, dtype) and m.cont_capacity == cap
    hist = [[None] * L for _ in range(B)]      # per item and layer: (K, V) on the CPU
    for lid in range(L):
        k = torch.randn(B, Hkv, T0, D, generator=g).to(dtype)
        v = torch.randn(B, Hkv, T0, D, generator=g).to(dtype)
        assert _append_prefill_batched(mgrs, k.to(DEV), v.to(DEV), lid) == [0, 0]
        for b in range(B):
            hist[b][lid] = (k[b], v[b])
    scale = 1 / math.sqrt(D)
    worst = 0.0
    for step in range(steps):
        T = T0 + step + 1
        mask = torch.zeros(B, 1, 1, T)
        mask[1, :, :, :7] = FMIN
        for lid in range(L):
            q = torch.randn(B, Hq, 1, D, generator=g).to(dtype)
            kn = torch.randn(B, Hkv, 1, D, generator=g).to(dtype)
            vn = torch.randn(B, Hkv, 1, D, generator=g).to(dtype)
            contiguous = mgrs[0].use_contiguous and mgrs[0].cont_seq_len < cap
            out = _decode_batched(mgrs, q.to(DEV), kn.to(DEV), vn.to(DEV), lid, scale,
                                  mask.to(DEV)).cpu()
            assert contiguous == (step < cap - T0)
            for b in range(B):
                K = torch.cat([hist[b][lid][0], kn[b]], 1)
                V = torch.cat([hist[b][lid][1], vn[b]], 1)
                hist[b][lid] = (K, V)
                ref = A.attention_fp64_batched(q[b].float(), K.float(), V.float(),
                                               mask=mask[b])
                worst = max(worst, (out[b].double() - ref).abs().max().item())
        if step == cap - T0:
            # the migration happened in this step's first layer call
            for m in mgrs:
                assert not m.use_contiguous and m.cont_K == {}
    assert worst <= tol, f"max abs error {worst}"
    # pages hold every token bit for bit (prompt pages, migrated decode
    # tokens, and the tokens appended since)
    for b, m in enumerate(mgrs):
        for lid in range(L):
            pages = [p for p in m.layers[lid].pages if p.used_tokens > 0]
            K = torch.cat([p.k_tensor[:, :, :p.used_tokens].cpu() for p in pages], 2)[0]
            V = torch.cat([p.v_tensor[:, :, :p.used_tokens].cpu() for p in pages], 2)[0]
            assert torch.equal(K, hist[b][lid][0]) and torch.equal(V, hist[b][lid][1])
        m.clear()


def test_contiguous_records_cover_the_buffers():
    """The device records of a contiguous arena address each 16-token block
    of every layer's K and V (built once, read by helm_paged_attn_seqs)."""
    from helm_amd import _native
    from helm_amd.runtime.kv_cache import ContiguousKV
    cont = ContiguousKV.allocate(3, 4, 64, 100, DEV, torch.bfloat16)
    rec = cont._rec.cpu().numpy().view(_native.PAGE_DTYPE).reshape(3, -1)
    assert rec.shape == (3, 7)
    for lid in range(3):
        k0, v0 = cont.k_view(lid).data_ptr(), cont.v_view(lid).data_ptr()
        assert list(rec[lid]["k"]) == [k0 + 16 * j * 64 * 2 for j in range(7)]
        assert list(rec[lid]["v"]) == [v0 + 16 * j * 64 * 2 for j in range(7)]
        assert list(rec[lid]["used"]) == [16] * 6 + [4]
        assert list(rec[lid]["tok_off"]) == [16 * j for j in range(7)]
        assert set(rec[lid]["head_stride"]) == {100 * 64}
    assert cont.aligned16


def test_tiny_llama_with_contiguous_cache_matches_hf_greedy():
    """KVOffloadConfig(cont_capacity=48) on a tiny random Llama: the prompt
    and the first decode steps use the contiguous buffers, the step past
    capacity migrates to pages, and the greedy tokens equal HF's."""
    from transformers.models.llama import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    cfg._attn_implementation = "eager"
    ref_model = LlamaForCausalLM(cfg).eval().to(DEV)
    model = LlamaForCausalLM(cfg).eval().to(DEV)
    model.load_state_dict(ref_model.state_dict())
    conf = KVOffloadConfig.from_model(model, page_size=16, cont_capacity=48)
    mgr = KVOffloadManager(model, conf, batch_size=1)
    assert mgr.kvcms[0].use_contiguous and mgr.kvcms[0].cont_capacity == 48
    prompt = torch.randint(0, 97, (1, 30), generator=torch.Generator().manual_seed(1)).to(DEV)
    steps = 36
    with torch.no_grad():
        ids = prompt.clone()
        for _ in range(steps):
            nxt = ref_model(ids, use_cache=False).logits[:, -1].argmax(-1, keepdim=True)
            ids = torch.cat([ids, nxt], 1)
        ref_tokens = ids[0, prompt.shape[1]:].tolist()
        S = prompt.shape[1]
        logits = model(prompt, position_ids=torch.arange(S, device=DEV)[None],
                       use_cache=False).logits
        out_tokens, used_cont = [], []
        tok = logits[:, -1].argmax(-1, keepdim=True)
        for t in range(steps):
            out_tokens.append(int(tok))
            pos = S + t
            used_cont.append(mgr.kvcms[0].use_contiguous)
            logits = model(tok, position_ids=torch.tensor([[pos]], device=DEV),
                           attention_mask=torch.zeros(1, 1, 1, pos + 1, device=DEV),
                           use_cache=False, cache_position=torch.tensor([pos], device=DEV)).logits
            tok = logits[:, -1].argmax(-1, keepdim=True)
    mgr.restore()
    assert out_tokens == ref_tokens
    assert used_cont[0] and not used_cont[-1]
