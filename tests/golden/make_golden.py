"""Writes the golden fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Each fixture holds seeded inputs (q, the concatenated K/V of a page list, an
optional additive mask) and the float64 textbook output of
oracle.attention.attention_fp64, plus the tolerance the output dtype is held
to (fp32 1e-5, fp16 2e-3, bf16 1e-2).  The shapes are the HELM test shapes
and small slices of the benchmark shapes, stored in float32 (exact for fp16 /
bf16 values).
"""
import json
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.attention import attention_fp64  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, Hq, Hkv, D, page sizes, dtype, mask kind, softcap, atol
    ("mha_ragged_fp32", 2, 2, 8, [3, 5, 2], "float32", None, None, 1e-5),
    ("gqa_masked_fp32", 4, 2, 8, [4, 3], "float32", "pad", None, 1e-5),
    ("softcap_fp32", 2, 2, 8, [3, 5], "float32", None, 50.0, 1e-5),
    ("qwen3_0p6b_slice_fp16", 16, 8, 128, [16] * 3 + [7], "float16", "zero", None, 2e-3),
    ("qwen3_8b_slice_bf16", 32, 8, 128, [16] * 4, "bfloat16", "zero", None, 1e-2),
    ("qwen3_14b_slice_bf16", 40, 8, 128, [16] * 3 + [1], "bfloat16", "pad", None, 1e-2),
    ("llama2_13b_slice_fp16", 40, 40, 128, [16, 9], "float16", None, None, 2e-3),
]


def main():
    for i, (name, Hq, Hkv, D, sizes, dt, mkind, cap, atol) in enumerate(CASES):
        g = torch.Generator().manual_seed(1000 + i)
        T = sum(sizes)
        dtype = getattr(torch, dt)
        q = torch.randn(1, Hq, 1, D, generator=g).to(dtype).float()
        K = torch.randn(1, Hkv, T, D, generator=g).to(dtype).float()
        V = torch.randn(1, Hkv, T, D, generator=g).to(dtype).float()
        arrays = {"q": q.numpy(), "K": K.numpy(), "V": V.numpy()}
        mask = None
        if mkind is not None:
            mask = torch.zeros(1, 1, 1, T)
            if mkind == "pad":
                idx = torch.randperm(T, generator=g)[: max(1, T // 5)]
                mask[..., idx] = torch.finfo(torch.float32).min
            arrays["mask"] = mask.numpy()
        scale = 1.0 / float(np.sqrt(D))
        out = attention_fp64(q, K, V, scale=scale, mask=None if mask is None else mask.numpy(),
                             softcap=cap)
        meta = {"dtype": dt, "page_sizes": sizes, "scale": scale, "softcap": cap, "atol": atol,
                "Hq": Hq, "Hkv": Hkv, "D": D}
        np.savez_compressed(os.path.join(OUT, f"{name}.npz"), out=out, meta=json.dumps(meta),
                            **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
