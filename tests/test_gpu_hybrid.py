"""A CPU + GPU split plan end to end (HELM's hybrid e2e test,
tests/integration/test_kv_eviction_e2e.py:10-66): a tiny random Llama with
layer 0 on the CPU and layer 1 on the GPU generates HF's greedy tokens
through the paged cache with forced eviction, for two requests in a row.

Layer 0's attention runs on the host-CPU kernel (libhelm_cpu.so) over pages
in host memory; layer 1's on the HIP kernels over device pages, most of
them evicted to pinned host memory by a 1 KiB watermark.  Activations move
between the stages the way HELM's stage executor moves them (a hook per
layer moves its inputs to the layer's device).  The prompts are fed as HELM's
pipeline feeds them: 128-token chunks under its chunk mask, then decode
steps under its zero decode mask (helm/runtime/pipeline_runtime.py:79-113).
"""
import pytest
import torch

from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime.kv_offload import KVOffloadConfig, KVOffloadManager

DEV = torch.device("cuda:0")
CHUNK = 128
NEW_TOKENS = 16


def _to(x, dev):
    if isinstance(x, torch.Tensor):
        return x.to(dev)
    if isinstance(x, tuple):
        return tuple(_to(y, dev) for y in x)
    if isinstance(x, list):
        return [_to(y, dev) for y in x]
    if isinstance(x, dict):
        return {k: _to(v, dev) for k, v in x.items()}
    return x


def _stage_hook(dev):
    def hook(module, args, kwargs):
        return _to(args, dev), _to(kwargs, dev)
    return hook


def _models():
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=32, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                      pad_token_id=1, eos_token_id=None, attention_dropout=0.0)
    cfg._attn_implementation = "eager"
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(11)
        ref = LlamaForCausalLM(cfg).eval()
    model = LlamaForCausalLM(cfg).eval()
    model.load_state_dict(ref.state_dict())
    # stage 0 (CPU): embeddings, rotary, layer 0; stage 1 (GPU): layer 1, norm, head
    model.model.layers[1].to(DEV)
    model.model.norm.to(DEV)
    model.lm_head.to(DEV)
    for layer in model.model.layers:
        dev = next(layer.parameters()).device
        layer.register_forward_pre_hook(_stage_hook(dev), with_kwargs=True)
    model.model.norm.register_forward_pre_hook(_stage_hook(DEV), with_kwargs=True)
    return ref, model


def _reference(ref, ids):
    """HF's greedy tokens by full recompute, and the logits each came from."""
    logits = []
    with torch.no_grad():
        for _ in range(NEW_TOKENS):
            last = ref(ids, use_cache=False).logits[:, -1]
            logits.append(last)
            ids = torch.cat([ids, last.argmax(-1, keepdim=True)], 1)
    return ids[0, -NEW_TOKENS:].tolist(), logits


def _generate(model, ids):
    """HELM's pipeline: chunked prefill under its chunk masks, then greedy
    decode steps under its zero decode mask."""
    fmin = torch.finfo(torch.float32).min
    n = ids.shape[1]
    with torch.no_grad():
        past, logits = 0, None
        while past < n:
            c = min(CHUNK, n - past)
            total = past + c
            allowed = torch.arange(total)[None, :] <= past + torch.arange(c)[:, None]
            mask = torch.where(allowed, 0.0, fmin)[None, None]
            logits = model(ids[:, past:total], attention_mask=mask,
                           position_ids=torch.arange(past, total)[None],
                           cache_position=torch.arange(past, total), use_cache=False).logits
            past = total
        out, seen = [], []
        for t in range(NEW_TOKENS):
            seen.append(logits[:, -1].cpu())
            tok = seen[-1].argmax(-1, keepdim=True)
            out.append(int(tok))
            if t == NEW_TOKENS - 1:
                break
            pos = n + t
            logits = model(tok, attention_mask=torch.zeros(1, 1, 1, pos + 1),
                           position_ids=torch.tensor([[pos]]),
                           cache_position=torch.tensor([pos]), use_cache=False).logits
    return out, seen


@pytest.mark.gpu
@pytest.mark.parametrize("disable_async", [False, True])
def test_hybrid_eviction_matches_reference_across_requests(disable_async, monkeypatch):
    """HELM's test of this name (tests/integration/test_kv_eviction_e2e.py:12): a CPU +
    GPU split with forced eviction generates HF's greedy tokens for two requests."""
    monkeypatch.setenv("HELM_DISABLE_ASYNC_KV", "1" if disable_async else "")
    ref, model = _models()
    prompts = [torch.tensor([[2 + i % 30 for i in range(L)]]) for L in (513, 17)]
    expected = [_reference(ref, p) for p in prompts]
    conf = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=1024,
                                      cont_capacity=0)
    mgr = KVOffloadManager(model, conf, batch_size=1)
    try:
        KC.reset_paging_stats()
        tokens, logits = _generate(model, prompts[0])
        assert tokens == expected[0][0]
        # and the logits behind them (fp32 throughout)
        assert max((a - b).abs().max().item() for a, b in zip(logits, expected[0][1])) <= 2e-4
        kvcm = mgr.kvcms[0]
        l0, l1 = kvcm.layers[0].pages, kvcm.layers[1].pages
        # layer 0 lives in host memory, layer 1 on the GPU with its old pages evicted
        assert l0 and all(p.state == "CPU" and p.device.type == "cpu" for p in l0)
        assert any(p.state == "GPU" for p in l1) and any(p.state == "CPU" for p in l1)
        stats = KC.get_paging_stats()
        assert stats["pages_evicted"] > 0
        assert stats["pages_prefetched"] > 0
        placement = [(p.device, p.data_ptr()) for p in model.parameters()]
        mgr.reset()
        tokens, logits = _generate(model, prompts[1])
        assert tokens == expected[1][0]
        assert max((a - b).abs().max().item() for a, b in zip(logits, expected[1][1])) <= 2e-4
        assert [(p.device, p.data_ptr()) for p in model.parameters()] == placement
    finally:
        mgr.restore()
