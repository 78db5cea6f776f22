"""GPU expert reconstructed from transferred NF4 state (mirrors
transfer/nf4_reconstruct.py:17-166 of the reference).

Reconstruction is metadata-only, as in the reference: the packed nibbles, absmax and
codebook that arrived on the device are wrapped, never re-quantised or copied.  The
forward pass ``w2(silu(w1 x) * w3 x)`` (:152-155) runs on the HIP kernels (fused NF4
dequant + bf16 MFMA, fp32 accumulation) instead of bitsandbytes' Linear4bit.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .._lib import MoeNf4Expert
from ..model.expert import NF4Linear, NF4QuantState, expert_struct, swiglu_forward
from ..nf4 import (NF4_BLOCKSIZE, NF4_DTYPE, NF4_NESTED_BLOCKSIZE, NF4_QUANT_STORAGE,
                   NF4_QUANT_TYPE)

_NESTED_DTYPE = torch.float32


def _build_quant_state(state: dict, shape: tuple[int, int]) -> NF4QuantState:
    """QuantState of one projection from its transferred tensors (:17-54)."""
    state2 = None
    s2_absmax = state.get("state2_absmax")
    s2_code = state.get("state2_code")
    if s2_absmax is not None or s2_code is not None:
        if s2_absmax is None or s2_code is None:
            raise ValueError("Incomplete nested NF4 quantization state")
        # The nested state quantises the main absmax tensor (:32-34).
        state2 = NF4QuantState(absmax=s2_absmax, code=s2_code, shape=state["absmax"].shape,
                               blocksize=NF4_NESTED_BLOCKSIZE, quant_type=None,
                               dtype=_NESTED_DTYPE, offset=state.get("state2_offset"))
    return NF4QuantState(absmax=state["absmax"], code=state["code"], shape=torch.Size(shape),
                         blocksize=NF4_BLOCKSIZE, quant_type=NF4_QUANT_TYPE, dtype=NF4_DTYPE,
                         offset=state.get("offset"), state2=state2)


def _reconstruct_linear(state: dict, *, in_features: int, out_features: int) -> NF4Linear:
    """NF4 projection shell around already-transferred tensors (:57-114)."""
    weight = state.get("weight")
    if weight is None:
        raise ValueError("NF4 state is missing packed weight")
    if weight.dtype != NF4_QUANT_STORAGE:
        raise ValueError(f"Expected packed NF4 weight dtype {NF4_QUANT_STORAGE}, got {weight.dtype}")
    qs = _build_quant_state(state, (out_features, in_features))
    return NF4Linear(weight, in_features=in_features, out_features=out_features, quant_state=qs)


class ReconstructedNF4Expert(nn.Module):
    """GPU-resident Mixtral expert reconstructed from transferred NF4 state."""

    def __init__(self, original_expert, gpu_state) -> None:
        super().__init__()
        hidden_size = getattr(original_expert, "hidden_size", None)
        intermediate_size = getattr(original_expert, "intermediate_size", None)
        if hidden_size is None or intermediate_size is None:
            raise ValueError("Prequantized expert must expose hidden_size and intermediate_size")
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.w1 = _reconstruct_linear(gpu_state["w1"], in_features=hidden_size,
                                      out_features=intermediate_size)
        self.w2 = _reconstruct_linear(gpu_state["w2"], in_features=intermediate_size,
                                      out_features=hidden_size)
        self.w3 = _reconstruct_linear(gpu_state["w3"], in_features=hidden_size,
                                      out_features=intermediate_size)
        self._struct: Optional[MoeNf4Expert] = None
        # Completion event of the copy that brings the tensors in (None: already there);
        # kernels that read them are ordered after it by wait_ready().
        self.ready_event: Optional[torch.cuda.Event] = None
        # Whatever keeps the tensors' device memory reserved for this expert (a slot lease
        # of the transfer scheduler's arena); dropped with the expert.
        self.device_lease = None

    def wait_ready(self) -> None:
        """Order the current stream's later work after the expert's arrival (a stream wait,
        no host synchronisation)."""
        ev = self.ready_event
        if ev is None:
            return
        if ev.query():
            self.ready_event = None
        else:
            torch.cuda.current_stream(self.device).wait_event(ev)

    def c_struct(self) -> MoeNf4Expert:
        """Device pointers of the three projections (moe_nf4_expert_t); the current stream
        first waits for the expert's arrival."""
        self.wait_ready()
        if self._struct is None:
            self._struct = expert_struct(self.w1, self.w2, self.w3)
        return self._struct

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        self.wait_ready()
        return swiglu_forward(self, x)

    @property
    def device(self) -> torch.device:
        return self.w1.weight.device

    @property
    def size_bytes(self) -> int:
        """Packed weight bytes only (:161-166)."""
        return sum(l.weight.numel() * l.weight.element_size() for l in (self.w1, self.w2, self.w3))
