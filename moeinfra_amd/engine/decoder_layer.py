"""Decoder-layer glue (mirrors engine/decoder_layer.py:7-42 of the reference).

``MoELayerAdapter`` gives the token-level MoELayer the [batch, sequence, hidden] interface
of a transformer block's MLP; ``MoEInfraDecoderLayer`` is Hugging Face's
MixtralDecoderLayer with its sparse-MoE block replaced (available when transformers is
installed).
"""
from __future__ import annotations

import torch


class MoELayerAdapter(torch.nn.Module):
    """Adapt MoELayer (tokens x hidden) to the 3-D interface of a decoder block."""

    def __init__(self, moe_layer):
        super().__init__()
        self.moe_layer = moe_layer

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must have shape (batch, sequence, hidden)")
        b, s, h = hidden_states.shape
        out = self.moe_layer.forward(hidden_states.reshape(b * s, h))
        return out.reshape(b, s, h)


def _make_decoder_layer_class():
    try:
        from transformers.models.mixtral.modeling_mixtral import MixtralDecoderLayer
    except ImportError:  # transformers is optional: only this adapter class needs it
        return None

    class MoEInfraDecoderLayer(MixtralDecoderLayer):
        """Mixtral decoder layer whose MoE block is an MoEInfra MoELayer."""

        def set_moe(self, moe_layer) -> None:
            self.mlp = MoELayerAdapter(moe_layer)

    return MoEInfraDecoderLayer


MoEInfraDecoderLayer = _make_decoder_layer_class()
