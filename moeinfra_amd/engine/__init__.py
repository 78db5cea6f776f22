"""Router and decoder-layer glue of the MoE expert path."""
from .router import ExpertRouter

__all__ = ["ExpertRouter"]
