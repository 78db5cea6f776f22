"""Seeded synthetic Mixtral-shaped MoE data.

Generation order is fixed so that every consumer sees the same tensors for a seed: the
gate [E,H], then for each expert e = 0..E-1 its w1 [F,H], w3 [F,H], w2 [H,F], then the
activations [T,H].  Weights and gate are N(0, 0.02) and activations N(0, 1), drawn in
fp32 and rounded to bf16.  Skewed routing adds a Zipf-shaped per-expert logit bias
b_e = beta * ln(p_e), p_e proportional to rank(e)^-s over a seeded permutation of the
experts (s = 1.2, beta = 4).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

MIXTRAL_HIDDEN = 4096
MIXTRAL_FFN = 14336
MIXTRAL_EXPERTS = 8
MIXTRAL_TOPK = 2


@dataclass
class LayerWeights:
    gate: torch.Tensor                                  # bf16 [E, H]
    experts: list = field(default_factory=list)         # [(w1 [F,H], w3 [F,H], w2 [H,F]) bf16]


def _normal(shape, gen: torch.Generator, device, std: float) -> torch.Tensor:
    t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t.to(torch.bfloat16)


def make_generator(seed: int, device="cpu") -> torch.Generator:
    return torch.Generator(device=device).manual_seed(int(seed))


def make_layer(hidden: int, inter: int, num_experts: int, gen: torch.Generator, device="cpu",
               std: float = 0.02, expert_sink=None) -> LayerWeights:
    """Gate then per-expert (w1, w3, w2).  ``expert_sink(e, w1, w3, w2)`` may consume each
    expert as it is generated (e.g. quantise and drop the bf16 copy); its return value is
    stored instead of the bf16 triple."""
    gate = _normal((num_experts, hidden), gen, device, std)
    lw = LayerWeights(gate=gate)
    for e in range(num_experts):
        w1 = _normal((inter, hidden), gen, device, std)
        w3 = _normal((inter, hidden), gen, device, std)
        w2 = _normal((hidden, inter), gen, device, std)
        lw.experts.append(expert_sink(e, w1, w3, w2) if expert_sink else (w1, w3, w2))
    return lw


def make_activations(tokens: int, hidden: int, gen: torch.Generator, device="cpu") -> torch.Tensor:
    return _normal((tokens, hidden), gen, device, 1.0)


def zipf_bias(num_experts: int, seed: int, s: float = 1.2, beta: float = 4.0) -> torch.Tensor:
    """fp32 [E] logit bias that makes routing Zipf-skewed (on the CPU; move as needed)."""
    g = torch.Generator().manual_seed(int(seed) + 7919)
    perm = torch.randperm(num_experts, generator=g)
    ranks = torch.empty(num_experts, dtype=torch.float64)
    ranks[perm] = torch.arange(1, num_experts + 1, dtype=torch.float64)
    p = ranks.pow(-s)
    p = p / p.sum()
    return (beta * torch.log(p)).to(torch.float32)


def nf4_bytes_per_expert(hidden: int, inter: int, blocksize: int = 64) -> int:
    """Packed nibbles + fp32 absmax of w1, w3 and w2."""
    n = hidden * inter
    return 3 * (n // 2 + math.ceil(n / blocksize) * 4)
