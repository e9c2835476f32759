"""Long-run offload correctness (GPU): HELM reports 2,048 of 2,048 greedy
tokens identical with and without KV offload (results/paper/
fig6_paging_throughput.json:11, harness experiments/verify_e2e.py:290-337,
test tests/integration/test_kv_eviction_e2e.py:10-66).

Here tiny random Llama and Qwen3 models (two layers, head_dim 128, 4 query /
2 KV heads, so bf16 runs on the matrix-core decode kernel that also writes the
step's token) are driven as HELM's pipeline drives them, under
torch.inference_mode() as HELM's generate: a 32,700-token prompt in 512-token
chunks under HELM's chunk masks, then 512 greedy decode steps under its decode
mask (both in the model's dtype, pipeline_runtime.py:79-113).  The run with a
1 KiB device watermark (every full page but the newest moves to pinned host
memory, and each decode step reads them back) must produce the same 512
tokens as the run that keeps every page on the device.  The decode steps
cross 32 page boundaries and the 2,048-page mark, where the decode call's
split count changes, while the token is written by the attention kernel.
"""
import pytest
import torch

from helm_amd.runtime import kv_cache as KC
from helm_amd.runtime.kv_offload import KVOffloadConfig, KVOffloadManager

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PROMPT = 32700
STEPS = 512
CHUNK = 512
VOCAB = 4096
# per-step logits of the two runs agree to this (same tokens fed, so the
# contexts are equal; the runs read the same pages from different places and
# may split them differently, so the attention sums may round differently)
LOGIT_TOL = {torch.bfloat16: 0.25, torch.float32: 1e-3}


def _model(arch: str, dtype):
    import transformers.models as tm
    common = dict(vocab_size=VOCAB, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                  max_position_embeddings=40000)
    if arch == "qwen3":
        cfg, cls = tm.qwen3.Qwen3Config(**common), tm.qwen3.Qwen3ForCausalLM
    else:
        cfg, cls = tm.llama.LlamaConfig(**common), tm.llama.LlamaForCausalLM
    cfg._attn_implementation = "eager"
    torch.manual_seed(5)
    return cls(cfg).eval().to(device=DEV, dtype=dtype)


def _greedy(model, prompt, watermark, steps=STEPS):
    """HELM's pipeline over the paged cache: chunked prefill, then greedy
    decode; returns the decode tokens, the logits each came from (CPU, fp32),
    the paging counters and the last layer's page states."""
    dtype = next(model.parameters()).dtype
    fmin = torch.finfo(dtype).min
    conf = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=watermark,
                                      cont_capacity=0)
    mgr = KVOffloadManager(model, conf, batch_size=1)
    KC.reset_paging_stats()
    n = prompt.shape[1]
    toks, seen = [], []
    try:
        with torch.inference_mode():
            past = 0
            while past < n:
                c = min(CHUNK, n - past)
                total = past + c
                allowed = (torch.arange(total, device=DEV)[None, :] <=
                           past + torch.arange(c, device=DEV)[:, None])
                mask = torch.where(allowed, torch.zeros((), device=DEV, dtype=dtype),
                                   torch.full((), fmin, device=DEV, dtype=dtype))[None, None]
                logits = model(prompt[:, past:total], attention_mask=mask,
                               position_ids=torch.arange(past, total, device=DEV)[None],
                               cache_position=torch.arange(past, total, device=DEV),
                               use_cache=False).logits
                past = total
            for t in range(steps):
                seen.append(logits[0, -1].float().cpu())
                tok = logits[:, -1].argmax(-1, keepdim=True)
                toks.append(int(tok))
                pos = n + t
                mask = torch.zeros((1, 1, 1, pos + 1), device=DEV, dtype=dtype)
                logits = model(tok, attention_mask=mask,
                               position_ids=torch.tensor([[pos]], device=DEV),
                               cache_position=torch.tensor([pos], device=DEV),
                               use_cache=False).logits
        stats = KC.get_paging_stats()
        states = [p.state for p in mgr.kvcms[0].layers[1].pages]
    finally:
        mgr.restore()
    return toks, torch.stack(seen), stats, states


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("arch", ["llama", "qwen3"])
def test_greedy_tokens_identical_with_and_without_offload(arch, dtype):
    model = _model(arch, dtype)
    g = torch.Generator().manual_seed(9)
    prompt = torch.randint(0, VOCAB, (1, PROMPT), generator=g).to(DEV)
    resident, lg_res, st_res, states_res = _greedy(model, prompt, 1 << 40)
    offload, lg_off, st_off, states_off = _greedy(model, prompt, 1024)
    assert st_res["pages_evicted"] == 0 and all(s == "GPU" for s in states_res)
    # offloaded: every page but the newest one or two lives in pinned host memory
    assert states_off.count("CPU") >= len(states_off) - 2
    assert st_off["pages_evicted"] > 0 and st_off["pages_prefetched"] > 0
    first = next((i for i, (a, b) in enumerate(zip(resident, offload)) if a != b), None)
    assert first is None, f"first differing token at decode step {first}"
    assert len(offload) == STEPS
    # and the logits behind every step
    assert (lg_res - lg_off).abs().max().item() <= LOGIT_TOL[dtype]
    # the run is not degenerate: it visits many tokens
    assert len(set(offload)) > 10, sorted(set(offload))


def test_greedy_2048_tokens_as_helm_reports():
    """HELM's own count: 2,048 greedy tokens (Qwen3, bf16) identical with and
    without offload after the same 32,700-token prompt; the decode steps cross
    128 page boundaries while every full page but the newest lives in pinned
    host memory."""
    model = _model("qwen3", torch.bfloat16)
    g = torch.Generator().manual_seed(11)
    prompt = torch.randint(0, VOCAB, (1, PROMPT), generator=g).to(DEV)
    resident, lg_res, _, _ = _greedy(model, prompt, 1 << 40, steps=2048)
    offload, lg_off, st_off, states_off = _greedy(model, prompt, 1024, steps=2048)
    assert states_off.count("CPU") >= len(states_off) - 2 and st_off["pages_evicted"] > 0
    first = next((i for i, (a, b) in enumerate(zip(resident, offload)) if a != b), None)
    assert first is None, f"first differing token at decode step {first}"
    assert len(offload) == 2048
    assert (lg_res - lg_off).abs().max().item() <= LOGIT_TOL[torch.bfloat16]
