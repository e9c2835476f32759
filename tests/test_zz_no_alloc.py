"""helm_paged_decode_attn_static — the decode entry point that allocates
nothing (its scratch is a fixed array in the library's device memory) —
against helm_paged_decode_attn with a caller workspace, through the C-ABI."""
import numpy as np
import pytest
import torch

from helm_amd import _native
from helm_amd import paged
from helm_amd import workloads as W
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _both(case, w, mask=None, softcap=None):
    """(workspace-call output, static-call output) on the same inputs."""
    out_ws = torch.empty_like(case["q"])
    args, keep = paged._decode_args(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                    case["lens"], case["max_pages"], sum(case["n_pages"]), None,
                                    softcap, mask, out_ws, 0)
    _native.call("helm_paged_decode_attn", *args)
    out_st = torch.empty_like(case["q"])
    st_args = list(args[:-3]) + [args[-1]]
    st_args[1] = out_st.data_ptr()
    _native.call("helm_paged_decode_attn_static", *st_args)
    torch.cuda.synchronize()
    return out_ws, out_st, keep


def _check_fp64(case, w, out, heads, mask=None, softcap=None):
    tol = 2e-3 if w.dtype == torch.float16 else 1e-2
    for b, t in enumerate(case["lens_list"]):
        n = case["n_pages"][b]
        slots = case["table_cpu"][b, :n].long().to(DEV)
        K = case["pool"][slots, 0].permute(1, 0, 2, 3).reshape(w.Hkv, -1, w.D)[:, :t]
        V = case["pool"][slots, 1].permute(1, 0, 2, 3).reshape(w.Hkv, -1, w.D)[:, :t]
        G = w.Hq // w.Hkv
        for kvh in heads:
            hs = slice(kvh * G, (kvh + 1) * G)
            m = None if mask is None else mask[b if mask.size(0) > 1 else 0].cpu()
            ref = A.attention_fp64_batched(case["q"][b, hs].float().cpu(),
                                           K[kvh:kvh + 1].float().cpu(),
                                           V[kvh:kvh + 1].float().cpu(), mask=m,
                                           softcap=softcap)
            assert (out[b, hs].double().cpu() - ref).abs().max().item() <= tol


def test_static_scratch_call_equals_workspace_call_then_smaller_call():
    """Two calls in a row, the second on a smaller input (Qwen3-8B 32k bf16,
    then a ragged Qwen3-0.6B-shaped fp16 batch with a mask and soft-cap):
    each equals the workspace call bit for bit (same plan, same kernels) and
    the fp64 oracle on sampled KV heads; a shape whose plan needs more
    scratch than the array holds is refused before any launch."""
    w1 = W.WORKLOADS["qwen3-8b-32k"]
    c1 = W.make_pool_case(w1, seed=1, device=DEV)
    a, b, _ = _both(c1, w1)
    assert torch.equal(a, b)
    _check_fp64(c1, w1, b, heads=[0, 7])

    w2 = W.Workload("small", 3, 16, 8, 128, torch.float16)
    c2 = W.make_pool_case(w2, seed=2, device=DEV, lens=[700, 33, 1500])
    mask = torch.zeros(3, 1, 1, 1500, device=DEV)
    mask[1, ..., 5:9] = torch.finfo(torch.float32).min
    a, b, _ = _both(c2, w2, mask=mask, softcap=30.0)
    assert torch.equal(a, b)
    _check_fp64(c2, w2, b, heads=[0, 3, 7], mask=mask, softcap=30.0)

    # the first shape again: nothing left behind by the smaller call matters
    a, b, _ = _both(c1, w1)
    assert torch.equal(a, b)

    # a plan beyond HELM_STATIC_SCRATCH_BYTES: refused, nothing launched
    lib = _native.load()
    Bq, Hq, Hkv, D, maxp = 64, 64, 8, 128, 8192
    need = lib.helm_query_workspace_bytes(Bq, Hq, Hkv, 1, D, maxp, 16, 0)
    assert need > _native.HELM_STATIC_SCRATCH_BYTES
    q = torch.zeros(Bq, Hq, 1, D, dtype=torch.bfloat16, device=DEV)
    pool = torch.zeros(1, 2, Hkv, 16, D, dtype=torch.bfloat16, device=DEV)
    table = torch.zeros(Bq, maxp, dtype=torch.int32, device=DEV)
    lens = torch.ones(Bq, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    rc = lib.helm_paged_decode_attn_static(
        q.data_ptr(), out.data_ptr(), pool[:, 0].data_ptr(), pool[:, 1].data_ptr(),
        pool.stride(0), pool.stride(2), table.data_ptr(), maxp, lens.data_ptr(), Bq, Hq, Hkv,
        1, D, 16, maxp, 0, None, 1.0, 0.0, None, 0, 0, 0, _native.HELM_F32, _native.HELM_BF16, _native.HELM_BF16, 0,
        None)
    assert rc == _native.HELM_E_WORKSPACE
    assert b"static scratch" in lib.helm_last_error_string()
