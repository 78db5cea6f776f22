"""Helpers of the end-to-end tests: the oracle's reference decoder and comparisons."""
from __future__ import annotations

import numpy as np
import torch

from oracle.decoder_oracle import RefDecoder, rmsnorm, rope  # noqa: F401


def top2_gap(logits: torch.Tensor) -> float:
    v = torch.topk(logits.float().reshape(-1), 2).values
    return float(v[0] - v[1])


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float().reshape(-1).numpy(), b.float().reshape(-1).numpy()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
