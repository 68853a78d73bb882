"""PhysicalCacheRequest: a one-way dense -> physical conversion request
(same fields and validation as unicache/core/decisions.py:51-85)."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import torch


@dataclass
class PhysicalCacheRequest:
    operator: str
    segment_id: str
    token_count: int
    segment_mask: torch.Tensor
    params: dict[str, Any] = field(default_factory=dict)
    per_kv_head_scores: torch.Tensor | None = None
    metadata: dict[str, Any] = field(default_factory=dict)

    def __post_init__(self) -> None:
        if self.token_count < 0:
            raise ValueError("PhysicalCacheRequest token count must be non-negative")
        mask = self.segment_mask
        if mask.dtype != torch.bool or mask.dim() != 1 or int(mask.numel()) != self.token_count:
            raise ValueError("PhysicalCacheRequest segment_mask must be boolean and match token_count")
        scores = self.per_kv_head_scores
        if scores is not None:
            if scores.dim() != 2:
                raise ValueError("Physical per-KV-head scores must be [kv_heads, tokens]")
            if int(scores.shape[-1]) != self.token_count:
                raise ValueError("Physical per-KV-head scores must match token_count")
