"""The fused decode front end (helm_decode_front): q / k RMSNorm, rotary
embedding and the page write of one decoded token per sequence, against the
HF modules and functions the patched forwards otherwise run
(kv_offload.py:365-373: Qwen3RMSNorm per head, Olmo2RMSNorm over the
projection, apply_rotary_pos_emb) and HELM's append_decode copy."""
import numpy as np
import pytest
import torch

from helm_amd import _native
from helm_amd.runtime import engine as _engine
from helm_amd.runtime import kv_offload as KO

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# one unit in the last place of each element type, relative
_ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -22}


def _reference(qp, kp, vp, cos, sin, norm, qn, kn, Hq, Hkv, D):
    import transformers.models.olmo2.modeling_olmo2 as o2
    B = qp.shape[0]
    if norm == "proj":
        qp, kp = qn(qp), kn(kp)
    q = qp.view(B, 1, Hq, D)
    k = kp.view(B, 1, Hkv, D)
    if norm == "head":
        q, k = qn(q), kn(k)
    q, k = q.transpose(1, 2), k.transpose(1, 2)
    # Olmo-2's apply_rotary_pos_emb: same formula, result cast back to q's
    # dtype (it matters only when cos / sin are fp32)
    return o2.apply_rotary_pos_emb(q, k, cos, sin)


def _close(got, ref, dtype, exact):
    """Bit-exact, or within two units in the last place of the element (or of
    the row's rms, where the rotary sum cancels), and for 16-bit types on
    fewer than 2% of the elements."""
    if exact:
        return torch.equal(got, ref)
    r = ref.float()
    d = (got.float() - r).abs()
    bound = 2 * _ULP[dtype] * (r.abs() + r.pow(2).mean().sqrt())
    if not bool((d <= bound).all()):
        return False
    return dtype == torch.float32 or (d > 0).float().mean().item() < 0.02


@pytest.mark.parametrize("dtype,cs32", [(torch.bfloat16, False), (torch.bfloat16, True),
                                        (torch.float16, False), (torch.float16, True),
                                        (torch.float32, False)])
@pytest.mark.parametrize("norm", ["none", "head", "proj"])
@pytest.mark.parametrize("B,Hq,Hkv,D", [(3, 32, 8, 128), (2, 8, 8, 64), (70, 4, 2, 256)])
def test_decode_front_matches_hf_ops(dtype, cs32, norm, B, Hq, Hkv, D):
    """q and the page's k equal HF's q_norm / k_norm + apply_rotary_pos_emb
    (bit for bit without a norm; within one unit in the last place, on < 2%
    of elements, with one: only the sum of squares is accumulated in another
    order); v lands unchanged; nothing else in the pages changes."""
    import transformers.models.olmo2.modeling_olmo2 as o2
    import transformers.models.qwen3.modeling_qwen3 as q3
    g = torch.Generator(device=DEV).manual_seed(B * 1000 + D)
    qp = (2 * torch.randn(B, 1, Hq * D, generator=g, device=DEV)).to(dtype)
    kp = (2 * torch.randn(B, 1, Hkv * D, generator=g, device=DEV)).to(dtype)
    vp = torch.randn(B, 1, Hkv * D, generator=g, device=DEV).to(dtype)
    pos = torch.randint(0, 5000, (B, 1), generator=g, device=DEV).float()
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, device=DEV).float() / D))
    freqs = pos[..., None] * inv
    emb = torch.cat([freqs, freqs], -1)
    cs_dtype = torch.float32 if cs32 else dtype
    cos, sin = emb.cos().to(cs_dtype), emb.sin().to(cs_dtype)
    qn = kn = None
    mode, eps = 0, 0.0
    if norm == "head":
        qn, kn = q3.Qwen3RMSNorm(D, eps=1e-6), q3.Qwen3RMSNorm(D, eps=1e-6)
        mode, eps = 1, 1e-6
    elif norm == "proj":
        qn, kn = o2.Olmo2RMSNorm(Hq * D, eps=1e-5), o2.Olmo2RMSNorm(Hkv * D, eps=1e-5)
        mode, eps = 2, 1e-5
    if qn is not None:
        for mod in (qn, kn):
            mod.to(DEV, dtype)
            with torch.no_grad():
                mod.weight.copy_(1 + 0.5 * torch.randn(mod.weight.shape, generator=g,
                                                      device=DEV).to(dtype))
    with torch.no_grad():
        q_ref, k_ref = _reference(qp, kp, vp, cos, sin, norm, qn, kn, Hq, Hkv, D)
    P = 16
    pk = torch.zeros(B, 1, Hkv, P, D, dtype=dtype, device=DEV)
    pv = torch.zeros_like(pk)
    toks = torch.randint(0, P, (B,), generator=torch.Generator().manual_seed(B)).tolist()
    dst = np.zeros(B, dtype=_native.APPEND_DTYPE)
    for b in range(B):
        dst[b]["dst_k"] = pk[b].data_ptr()
        dst[b]["dst_v"] = pv[b].data_ptr()
        dst[b]["dst_head_stride"] = P * D
        dst[b]["dst_tok"] = toks[b]
    q_out = torch.full((B, Hq, 1, D), float("nan"), dtype=dtype, device=DEV)
    _native.call("helm_decode_front", qp.data_ptr(), kp.data_ptr(), vp.data_ptr(), Hq * D,
                 Hkv * D, qn.weight.data_ptr() if qn is not None else None,
                 kn.weight.data_ptr() if kn is not None else None, mode, eps, cos.data_ptr(),
                 sin.data_ptr(), D, _native.dtype_code(cs_dtype), q_out.data_ptr(),
                 _native.ptr(dst), B, Hq, Hkv, D, _native.dtype_code(dtype),
                 _engine.stream_ptr(DEV))
    torch.cuda.synchronize()
    exact = norm == "none"
    assert _close(q_out, q_ref, dtype, exact)
    k_got = torch.stack([pk[b, 0, :, toks[b]] for b in range(B)])[:, :, None]
    assert _close(k_got, k_ref, dtype, exact)
    v_got = torch.stack([pv[b, 0, :, toks[b]] for b in range(B)])
    assert torch.equal(v_got, vp.view(B, Hkv, D))
    for b in range(B):
        pk[b, 0, :, toks[b]] = 0
        pv[b, 0, :, toks[b]] = 0
    assert torch.count_nonzero(pk).item() == 0 and torch.count_nonzero(pv).item() == 0


def test_decode_front_rejects_bad_shapes():
    """A head wider than 256 elements is refused before any launch."""
    B, Hq, Hkv, D = 1, 4, 2, 130 * 2
    x = torch.zeros(Hq * 300, dtype=torch.bfloat16, device=DEV)
    dst = np.zeros(1, dtype=_native.APPEND_DTYPE)
    dst[0]["dst_k"] = dst[0]["dst_v"] = x.data_ptr()
    dst[0]["dst_head_stride"] = 16 * D
    with pytest.raises(ValueError, match="at most 256"):
        _native.call("helm_decode_front", x.data_ptr(), x.data_ptr(), x.data_ptr(), Hq * D,
                     Hkv * D, None, None, 0, 0.0, x.data_ptr(), x.data_ptr(), 0,
                     _native.dtype_code(torch.bfloat16), x.data_ptr(), _native.ptr(dst), B, Hq,
                     Hkv, D, _native.dtype_code(torch.bfloat16), _engine.stream_ptr(DEV))


@pytest.mark.parametrize("arch", ["qwen3", "llama", "olmo2"])
def test_patched_decode_uses_front_and_matches_torch_ops(arch, monkeypatch):
    """A tiny bf16 model decodes through the patched forward: the fused front
    end serves every decode step (its launch is counted) and gives the same
    logits, within bf16 rounding of the norm, as the forward's torch ops
    (HELM_AMD_FRONT=0)."""
    import transformers.models as tm
    from helm_amd.runtime.kv_offload import KVOffloadConfig, KVOffloadManager
    common = dict(vocab_size=97, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    if arch == "qwen3":
        cfg, cls = tm.qwen3.Qwen3Config(head_dim=64, **common), tm.qwen3.Qwen3ForCausalLM
    elif arch == "olmo2":
        cfg, cls = tm.olmo2.Olmo2Config(**common), tm.olmo2.Olmo2ForCausalLM
    else:
        cfg, cls = tm.llama.LlamaConfig(**common), tm.llama.LlamaForCausalLM
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = cls(cfg).eval().to(DEV, torch.bfloat16)
    ids = torch.randint(0, 97, (2, 40), generator=torch.Generator().manual_seed(3)).to(DEV)
    real = KO._decode_front
    served = []

    def spy(*args):
        out = real(*args)
        served.append(out is not None)
        return out
    monkeypatch.setattr(KO, "_decode_front", spy)
    runs = {}
    for front in ("1", "0"):
        monkeypatch.setenv("HELM_AMD_FRONT", front)
        conf = KVOffloadConfig.from_model(model, page_size=16)
        mgr = KVOffloadManager(model, conf, batch_size=2)
        logits = []
        with torch.no_grad():
            S = 24
            model(ids[:, :S], position_ids=torch.arange(S, device=DEV)[None].expand(2, -1),
                  use_cache=False)
            for t in range(S, ids.shape[1]):
                out = model(ids[:, t:t + 1], position_ids=torch.full((2, 1), t, device=DEV),
                            use_cache=False, cache_position=torch.tensor([t], device=DEV))
                logits.append(out.logits.float())
        mgr.restore()
        runs[front] = torch.cat(logits, 1)
    n_steps = (ids.shape[1] - 24) * cfg.num_hidden_layers
    assert served[:n_steps] == [True] * n_steps and served[n_steps:] == [False] * n_steps
    assert (runs["1"] - runs["0"]).abs().max().item() <= 5e-2


def test_bf16_model_d128_matrix_core_paths_match_hf():
    """A bf16 Qwen3-shaped model with head_dim 128, so that every attention
    call runs on the matrix-core kernels: the first prompt chunk on the chunk
    kernel over its own K/V, the second over the cached pages (32x32 tiles,
    chunk mask), then decode steps through the fused front end and the decode
    kernel, with eviction to pinned host pages along the way.  Logits stay
    within bf16 rounding of HF's own eager forward over the same tokens."""
    import transformers.models.qwen3 as q3
    from helm_amd.runtime import kv_cache as KC
    from helm_amd.runtime.kv_offload import KVOffloadConfig, KVOffloadManager
    cfg = q3.Qwen3Config(vocab_size=97, hidden_size=512, intermediate_size=512,
                         num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=4,
                         head_dim=128, max_position_embeddings=1024)
    cfg._attn_implementation = "eager"
    torch.manual_seed(1)
    ref_model = q3.Qwen3ForCausalLM(cfg).eval().to(DEV, torch.bfloat16)
    model = q3.Qwen3ForCausalLM(cfg).eval().to(DEV, torch.bfloat16)
    model.load_state_dict(ref_model.state_dict())
    conf = KVOffloadConfig.from_model(model, page_size=16, gpu_watermark_bytes=64 * 1024)
    mgr = KVOffloadManager(model, conf, batch_size=1)
    g = torch.Generator().manual_seed(4)
    S, c1, steps = 200, 120, 24
    ids = torch.randint(0, 97, (1, S + steps), generator=g).to(DEV)
    KC.reset_paging_stats()
    diffs = []
    with torch.no_grad():
        lg = model(ids[:, :c1], position_ids=torch.arange(c1, device=DEV)[None],
                   use_cache=False).logits
        ref = ref_model(ids[:, :S], use_cache=False).logits
        diffs.append((lg.float() - ref[:, :c1].float()).abs())
        n2 = S - c1
        cm = torch.zeros(1, 1, n2, S, device=DEV)
        cm[0, 0][torch.arange(S, device=DEV)[None, :] >
                 (c1 + torch.arange(n2, device=DEV))[:, None]] = torch.finfo(torch.float32).min
        lg = model(ids[:, c1:S], position_ids=torch.arange(c1, S, device=DEV)[None],
                   attention_mask=cm, use_cache=False,
                   cache_position=torch.arange(c1, S, device=DEV)).logits
        diffs.append((lg.float() - ref[:, c1:S].float()).abs())
        for t in range(steps):
            pos = S + t
            lg = model(ids[:, pos:pos + 1], position_ids=torch.tensor([[pos]], device=DEV),
                       use_cache=False, cache_position=torch.tensor([pos], device=DEV)).logits
            r = ref_model(ids[:, :pos + 1], use_cache=False).logits[:, -1:]
            diffs.append((lg.float() - r.float()).abs())
    mgr.restore()
    d = torch.cat([x.flatten() for x in diffs])
    assert KC.get_paging_stats()["pages_evicted"] > 0
    assert d.max().item() <= 0.25 and d.mean().item() <= 0.02, (d.max().item(), d.mean().item())
