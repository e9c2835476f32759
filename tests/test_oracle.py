"""The oracle is pinned before anything is compared against it.

Checks (CPU only):
* the restated online-softmax loop and Path 2 against the float64 textbook
  formula on seeded inputs (ragged pages, GQA, masks, soft-cap, fp16);
* the float64 formula itself against closed forms (single key -> its value,
  q = 0 -> mean of V, identical keys -> mean of V) and against torch SDPA;
* the known answers and cases HELM's own tests hold for this path
  (tests/unit/runtime/test_streaming_attention.py, test_kv_offload.py);
* golden fixtures committed under tests/golden/ (fp64 outputs of seeded inputs).
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _pages(sizes, H, D, seed, kv_heads=None, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    kvh = kv_heads or H
    ks = [torch.randn(1, kvh, n, D, generator=g).to(dtype) for n in sizes]
    vs = [torch.randn(1, kvh, n, D, generator=g).to(dtype) for n in sizes]
    q = torch.randn(1, H, 1, D, generator=g).to(dtype)
    return q, list(zip(ks, vs)), torch.cat(ks, 2), torch.cat(vs, 2)


@pytest.mark.parametrize("sizes,H,kvh,D", [
    ([4], 2, 2, 8), ([4, 3], 2, 2, 8), ([3, 5, 2], 1, 1, 16), ([4, 3], 4, 2, 8),
    ([16] * 8 + [5], 8, 2, 64), ([16] * 4, 32, 8, 128),
])
def test_restatements_match_fp64(sizes, H, kvh, D):
    q, pages, K, V = _pages(sizes, H, D, seed=sum(sizes) + H, kv_heads=kvh)
    ref = A.attention_fp64(q, K, V)
    mask = torch.zeros(1, 1, 1, K.size(2))
    got_loop = A.online_softmax_pages(q, pages, attention_mask=mask)
    got_p2 = A.concat_sdpa(q, pages)
    np.testing.assert_allclose(got_loop.double().numpy(), ref, atol=1e-5)
    np.testing.assert_allclose(got_p2.double().numpy(), ref, atol=1e-5)


def test_masks_softcap_match_fp64():
    q, pages, K, V = _pages([4, 4, 3], 4, 16, seed=11, kv_heads=2)
    mask = torch.zeros(1, 1, 1, 11)
    mask[..., [0, 3, 4, 10]] = torch.finfo(torch.float32).min
    ref = A.attention_fp64(q, K, V, mask=mask.numpy(), softcap=5.0)
    got = A.online_softmax_pages(q, pages, attention_mask=mask, softcap=5.0)
    np.testing.assert_allclose(got.double().numpy(), ref, atol=1e-5)


@pytest.mark.parametrize("scale", [1.0, 0.5])
def test_softcap_two_keys_known_answer(scale):
    """Soft-cap pinned by hand: with one-dimensional q = 1 and keys k_i, the
    logits are x_i = cap * tanh(k_i * scale / cap) (HELM scales first, then
    caps: kv_cache.py:516-517, :532-533), the weights are exp(x_i) / sum, and
    the output is their mean of the values.  A cap applied before the scale,
    a missing tanh or a cap applied to the weights gives another number."""
    cap = 2.0
    k = [3.0, -1.5]
    v = [10.0, -4.0]
    x = [cap * math.tanh(ki * scale / cap) for ki in k]
    w = [math.exp(xi) for xi in x]
    want = (w[0] * v[0] + w[1] * v[1]) / (w[0] + w[1])
    q = torch.ones(1, 1, 1, 1)
    K = torch.tensor(k).view(1, 1, 2, 1)
    V = torch.tensor(v).view(1, 1, 2, 1)
    got64 = A.attention_fp64(q, K, V, scale=scale, softcap=cap)[0, 0, 0, 0]
    assert abs(got64 - want) <= 1e-12
    for pages in ([(K, V)], [(K[:, :, :1], V[:, :, :1]), (K[:, :, 1:], V[:, :, 1:])]):
        got = A.online_softmax_pages(q, pages, scale=scale, softcap=cap)[0, 0, 0, 0].item()
        assert abs(got - want) <= 1e-5
        got = A.streaming_attention(q, pages, scale=scale, softcap=cap)[0, 0, 0, 0].item()
        assert abs(got - want) <= 1e-5
    # the wrong orders give numbers far from it
    x_wrong = [cap * math.tanh(ki / cap) * scale for ki in k]
    w_wrong = [math.exp(xi) for xi in x_wrong]
    wrong = (w_wrong[0] * v[0] + w_wrong[1] * v[1]) / sum(w_wrong)
    if scale != 1.0:
        assert abs(wrong - want) > 1e-3


def test_softcap_large_cap_is_uncapped_sdpa():
    """cap * tanh(x / cap) -> x as cap grows: at cap = 1e6 the capped formula
    equals float64 SDPA without a cap (logits of order 10: the cap changes
    them by ~x^3 / (3 cap^2) < 1e-9)."""
    q, pages, K, V = _pages([16, 16, 5], 8, 32, seed=17, kv_heads=4)
    q = q * 3
    Ke = K.repeat_interleave(2, dim=1).double()
    Ve = V.repeat_interleave(2, dim=1).double()
    sdpa = F.scaled_dot_product_attention(q.double(), Ke, Ve).numpy()
    np.testing.assert_allclose(A.attention_fp64(q, K, V, softcap=1e6), sdpa, atol=1e-9)
    got = A.online_softmax_pages(q, pages, softcap=1e6)
    np.testing.assert_allclose(got.double().numpy(), sdpa, atol=1e-5)
    # and a small cap moves the answer (the branch is not a no-op)
    assert np.abs(A.attention_fp64(q, K, V, softcap=1.0) - sdpa).max() > 1e-2


def test_fp16_within_helm_tolerance():
    # HELM: fp16 accumulates in fp32, atol 2e-3 (test_streaming_attention.py:353-365)
    q, pages, K, V = _pages([16] * 8, 16, 128, seed=5, kv_heads=8, dtype=torch.float16)
    ref = A.attention_fp64(q.float(), K.float(), V.float())
    got = A.online_softmax_pages(q, pages, attention_mask=torch.zeros(1, 1, 1, 128))
    assert got.dtype == torch.float16
    assert np.abs(got.double().numpy() - ref).max() <= 2e-3


# ── the float64 formula against closed forms and a library routine ───────────
def test_fp64_single_key_returns_its_value():
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 3, 1, 8, generator=g) for _ in range(3))
    np.testing.assert_allclose(A.attention_fp64(q, k, v), v.double().numpy(), atol=1e-12)


def test_fp64_zero_query_is_mean_of_values():
    g = torch.Generator().manual_seed(2)
    k, v = torch.randn(1, 2, 7, 8, generator=g), torch.randn(1, 2, 7, 8, generator=g)
    q = torch.zeros(1, 2, 1, 8)
    np.testing.assert_allclose(A.attention_fp64(q, k, v)[0, :, 0],
                               v.double().numpy()[0].mean(axis=1), atol=1e-12)


def test_fp64_matches_torch_sdpa_gqa_and_causal():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 8, 5, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, 2, 9, 16, generator=g, dtype=torch.float64)
    v = torch.randn(2, 2, 9, 16, generator=g, dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1))
    np.testing.assert_allclose(A.attention_fp64(q, k, v), ref.numpy(), atol=1e-12)
    # top-left causal == SDPA is_causal with q_len <= kv_len
    ref_c = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1),
                                           v.repeat_interleave(4, 1), is_causal=True)
    np.testing.assert_allclose(A.attention_fp64(q, k, v, causal=True), ref_c.numpy(), atol=1e-12)


def test_fp64_gqa_map_is_h_div_groups():
    # distinct KV heads: head h must read KV head h // G, not h % Hkv
    q = torch.zeros(1, 4, 1, 2)
    k = torch.zeros(1, 2, 1, 2)
    v = torch.tensor([[[[1.0, 1.0]], [[2.0, 2.0]]]])
    out = A.attention_fp64(q, k, v)
    assert out[0, :, 0, 0].tolist() == [1.0, 1.0, 2.0, 2.0]


# ── HELM's own known answers and cases ────────────────────────────────────────
def test_no_pages_returns_zeros():
    q = torch.randn(1, 2, 1, 8)
    assert torch.all(A.streaming_attention(q, []) == 0)


def test_zero_used_page_skipped():
    q, pages, K, V = _pages([4], 2, 8, seed=7)
    empty = (pages[0][0][:, :, :0], pages[0][1][:, :, :0])
    torch.testing.assert_close(A.streaming_attention(q, [empty] + pages),
                               A.streaming_attention(q, pages), atol=1e-6, rtol=0)


def test_fully_masked_page_contributes_nothing():
    q, pages, K, V = _pages([4, 4], 2, 8, seed=2)
    mask = torch.zeros(1, 1, 1, 8)
    mask[..., :4] = torch.finfo(torch.float32).min
    got = A.online_softmax_pages(q, pages, attention_mask=mask)
    ref = A.attention_fp64(q, K[:, :, 4:], V[:, :, 4:])
    np.testing.assert_allclose(got.double().numpy(), ref, atol=1e-5)


def test_large_logits_finite():
    q = torch.ones(1, 1, 1, 64) * 100.0
    k = torch.ones(1, 1, 8, 64) * 100.0
    v = torch.randn(1, 1, 8, 64)
    out = A.online_softmax_pages(q, [(k, v)], softcap=None, attention_mask=torch.zeros(1, 1, 1, 8))
    assert torch.isfinite(out).all()


def test_gemma2_sliding_window_known_answer():
    # test_kv_offload.py:367-413: q = 1, keys (10, 0, 0), values (100, 1, 2),
    # scale 1, window 2 -> query 2 sees keys 1 and 2 equally -> 1.5
    q = torch.ones(1, 1, 1, 1)
    k = torch.tensor([10.0, 0.0, 0.0]).view(1, 1, 3, 1)
    v = torch.tensor([100.0, 1.0, 2.0]).view(1, 1, 3, 1)
    mask = torch.zeros(1, 1, 1, 3)
    mask[..., 0] = torch.finfo(torch.float32).min
    got = A.online_softmax_pages(q, [(k, v)], scale=1.0, attention_mask=mask)
    assert got.item() == pytest.approx(1.5, abs=1e-4)
    assert A.attention_fp64(q, k, v, scale=1.0, mask=mask.numpy())[0, 0, 0, 0] == pytest.approx(1.5)


def _poison_case():
    # test_kv_offload.py:168-210: pad keys aligned with q dominate an unmasked
    # softmax, so only a working mask reproduces the real-token reference
    torch.manual_seed(0)
    q = torch.randn(1, 1, 1, 4)
    real_k, real_v = torch.randn(1, 1, 3, 4), torch.randn(1, 1, 3, 4)
    pad_k = q.expand(1, 1, 2, 4) * 50.0
    pad_v = torch.full((1, 1, 2, 4), 1000.0)
    k_dec, v_dec = torch.randn(1, 1, 1, 4), torch.randn(1, 1, 1, 4)
    K = torch.cat([real_k, pad_k, k_dec], 2)
    V = torch.cat([real_v, pad_v, v_dec], 2)
    mask = torch.zeros(1, 1, 1, 6)
    mask[..., 3:5] = float("-inf")
    expected = F.scaled_dot_product_attention(q, torch.cat([real_k, k_dec], 2),
                                              torch.cat([real_v, v_dec], 2), scale=1.0)
    return q, K, V, mask, expected


def test_poison_pad_mask_honoured():
    q, K, V, mask, expected = _poison_case()
    got = A.online_softmax_pages(q, [(K, V)], scale=1.0, attention_mask=mask)
    torch.testing.assert_close(got, expected, atol=1e-4, rtol=0)
    unmasked = A.streaming_attention(q, [(K, V)], scale=1.0)
    assert not torch.allclose(unmasked, expected, atol=1e-4)


# ── committed golden fixtures ─────────────────────────────────────────────────
def _golden_files():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


@pytest.mark.parametrize("name", _golden_files())
def test_golden_fixture(name):
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    q = torch.from_numpy(z["q"]).to(getattr(torch, meta["dtype"]))
    K = torch.from_numpy(z["K"]).to(q.dtype)
    V = torch.from_numpy(z["V"]).to(q.dtype)
    mask = torch.from_numpy(z["mask"]) if "mask" in z.files else None
    pages = A.split_pages(K, V, meta["page_sizes"])
    got = A.streaming_attention(q, pages, scale=meta["scale"], attention_mask=mask,
                                softcap=meta.get("softcap"))
    np.testing.assert_allclose(got.double().numpy(), z["out"], atol=meta["atol"])


@pytest.mark.parametrize("Hq,Hkv,S,T,cap", [(8, 2, 1, 37, None), (40, 8, 1, 64, 30.0),
                                             (4, 4, 3, 9, None)])
def test_batched_fp64_equals_loop_fp64(Hq, Hkv, S, T, cap):
    g = torch.Generator().manual_seed(Hq + T)
    q = torch.randn(1, Hq, S, 16, generator=g)
    K = torch.randn(1, Hkv, T, 16, generator=g)
    V = torch.randn(1, Hkv, T, 16, generator=g)
    mask = torch.zeros(1, 1, S, T)
    mask[..., ::5] = float("-inf")
    ref = A.attention_fp64(q, K, V, mask=mask.numpy(), softcap=cap)
    got = A.attention_fp64_batched(q[0], K[0], V[0], mask=mask[0], softcap=cap)
    np.testing.assert_allclose(got.numpy(), ref[0], atol=1e-12)
