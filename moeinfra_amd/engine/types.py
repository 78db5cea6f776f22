"""Request / result types of the inference engine (mirrors engine/types.py:1-64 of the
reference: PrefetchPolicy, ForwardRequest, ForwardResult with the same fields)."""
from __future__ import annotations

import dataclasses
import enum
from typing import Optional

import torch


class PrefetchPolicy(enum.Enum):
    """Expert prefetch strategy (engine/types.py:15-28), plus NEXT_ROUTER: the next layer's
    router applied to the current layer's MoE input predicts the next layer's experts."""

    NONE = "none"
    NEXT_LAYER = "next_layer"
    LOOKAHEAD = "lookahead"
    NEXT_ROUTER = "next_router"


@dataclasses.dataclass
class ForwardRequest:
    """One generation request (engine/types.py:31-44): prompt ids [batch, seq]."""

    input_ids: torch.Tensor
    attention_mask: Optional[torch.Tensor] = None
    max_new_tokens: int = 128


@dataclasses.dataclass
class ForwardResult:
    """Result of a request (engine/types.py:47-64): the last logits, the greedy token ids,
    time to first token (prefill, ms), decode tokens per second and per-stage timings (ms)."""

    logits: torch.Tensor
    token_ids: list
    ttft_ms: float
    tps: float
    stage_timings: dict
