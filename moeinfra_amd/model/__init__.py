"""NF4 expert containers and the MoE layer."""
from .expert import PrequantizedNF4Expert, QuantizedMixtralExpert
from .moe_layer import MoELayer

__all__ = ["MoELayer", "PrequantizedNF4Expert", "QuantizedMixtralExpert"]
