"""KVPage — the page record of helm/runtime/kv_cache.py:65-75.

Same nine fields, same meaning.  Two optional fields say where an
allocator-made page lives: ``arena`` (index of the slot arena, None for a page
built by hand around arbitrary tensors) and ``slot`` (slot inside the arena).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class KVPage:
    page_id: int
    layer_id: int
    start_token: int
    used_tokens: int
    capacity_tokens: int
    k_tensor: torch.Tensor
    v_tensor: torch.Tensor
    device: torch.device
    state: str  # 'FREE', 'GPU', 'CPU', 'DEAD'
    arena: Optional[int] = field(default=None, repr=False, compare=False)
    slot: int = field(default=-1, repr=False, compare=False)
