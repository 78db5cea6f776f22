"""Top-k expert router (mirrors engine/router.py:16-105 of the reference).

``logits`` / ``route`` / ``route_with_logits`` run the HIP router kernel: the gate linear
with fp32 accumulation rounded to bf16 logits, an fp32 softmax, top-k (descending; ties
keep the lower index) and renormalisation, in one launch.  Activations and gate are bf16
GPU tensors (Mixtral's dtype); other dtypes or CPU tensors raise ``ValueError`` -- there
is no host implementation.  ``bias`` (keyword, optional) adds an fp32 per-expert offset
to the logits before the softmax; the reference has none.
"""
from __future__ import annotations

import logging
from typing import Optional

import torch

from .. import ops


class ExpertRouter:
    """Top-k router for a Mixtral MoE layer."""

    def __init__(self, gate_weight: torch.Tensor, num_experts_per_tok: int = 2,
                 logger: Optional[logging.Logger] = None, *,
                 bias: Optional[torch.Tensor] = None) -> None:
        if gate_weight.ndim != 2:
            raise ValueError(f"gate_weight must be 2D, got shape {tuple(gate_weight.shape)}")
        self.num_experts = gate_weight.shape[0]
        self.hidden_size = gate_weight.shape[1]
        self.num_experts_per_tok = num_experts_per_tok
        self._logger = logger or logging.getLogger(__name__)
        if num_experts_per_tok <= 0:
            raise ValueError("num_experts_per_tok must be positive")
        if num_experts_per_tok > self.num_experts:
            raise ValueError(f"num_experts_per_tok ({num_experts_per_tok}) must be <= "
                             f"num_experts ({self.num_experts})")
        self.gate_weight = gate_weight
        self.bias = bias

    @property
    def device(self) -> torch.device:
        return self.gate_weight.device

    def _check(self, hidden_states: torch.Tensor) -> None:
        if hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"hidden_states last dim {hidden_states.shape[-1]} != "
                             f"hidden_size {self.hidden_size}")
        if hidden_states.device != self.gate_weight.device:
            raise ValueError(f"hidden_states device {hidden_states.device} != "
                             f"gate device {self.gate_weight.device}")

    def _run(self, hidden_states: torch.Tensor, want_logits: bool):
        self._check(hidden_states)
        lead = hidden_states.shape[:-1]
        x = hidden_states.reshape(-1, self.hidden_size).contiguous()
        gate = self.gate_weight.contiguous()
        logits, w, idx = ops.router_topk(x, gate, self.num_experts_per_tok, bias=self.bias,
                                         want_logits=want_logits)
        k = self.num_experts_per_tok
        if logits is not None:
            logits = logits.reshape(*lead, self.num_experts)
        return logits, w.reshape(*lead, k), idx.reshape(*lead, k)

    def logits(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """Gate logits in the activation dtype (bf16)."""
        return self._run(hidden_states, True)[0]

    def route(self, hidden_states: torch.Tensor):
        """(expert indices int64 [..., k], expert weights fp32 [..., k])."""
        _, w, idx = self._run(hidden_states, False)
        return idx, w

    def route_with_logits(self, hidden_states: torch.Tensor):
        """(logits, expert weights fp32, expert indices int64)."""
        return self._run(hidden_states, True)

    def predict_next_layer_experts(self, current_expert_indices: torch.Tensor) -> list[int]:
        """Sorted distinct experts of the current selection (engine/router.py:96-105)."""
        flat = current_expert_indices.reshape(-1)
        return sorted(int(v) for v in flat.unique().tolist())
