"""Bounded, reusable pinned-memory staging slots for expert H2D transfers (mirrors
transfer/reusable_staging.py:20-284 of the reference).

A slot is not handed out again until the event recorded after its last DMA has completed
(:72-93), so a host buffer is never overwritten while a copy still reads it.  Experts are
staged in the canonical per-projection representation
``weight, absmax, code, offset [, state2_absmax, state2_code, state2_offset]`` (:126-222),
accepting either that form or bitsandbytes' serialized Linear4bit.state_dict() keys; the
serialized metadata blob is decoded here without bitsandbytes.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from ..model.expert import parse_blob
from .pinned_memory import PinnedMemoryBudget

_BLOB = "weight.quant_state.bitsandbytes__nf4"


@dataclass
class StagingSlot:
    slot_id: int
    size_bytes: int
    tensors: dict
    in_use: bool = False
    ready_event: Optional[torch.cuda.Event] = None
    expert_key: Optional[tuple[int, int]] = None


class ReusablePinnedStagingPool:
    """Pinned slots reused once the event of their previous transfer has completed."""

    _PROJECTIONS = ("w1", "w2", "w3")

    def __init__(self, budget: PinnedMemoryBudget, slot_size_bytes: int):
        if slot_size_bytes <= 0:
            raise ValueError("slot_size_bytes must be positive")
        self.budget = budget
        self.slot_size_bytes = slot_size_bytes
        self._slots: dict[int, StagingSlot] = {}

    @property
    def slot_count(self) -> int:
        return len(self._slots)

    @property
    def active_slots(self) -> int:
        return sum(slot.in_use for slot in self._slots.values())

    def _create_slot(self, slot_id: int) -> Optional[StagingSlot]:
        if not self.budget.reserve(self.slot_size_bytes):
            return None
        slot = StagingSlot(slot_id=slot_id, size_bytes=self.slot_size_bytes, tensors={})
        self._slots[slot_id] = slot
        return slot

    def acquire(self) -> Optional[StagingSlot]:
        """A free slot whose last transfer has finished, a new one within budget, or None."""
        for slot in self._slots.values():
            if slot.in_use:
                continue
            if slot.ready_event is not None:
                if not slot.ready_event.query():
                    continue
                slot.ready_event = None
            slot.in_use = True
            return slot
        slot = self._create_slot(len(self._slots))
        if slot is not None:
            slot.in_use = True
        return slot

    def mark_transfer_complete(self, slot: StagingSlot, stream) -> None:
        """Record the event that gates the slot's reuse on `stream` (after its DMA)."""
        if not slot.in_use:
            raise RuntimeError("Cannot mark an inactive slot")
        event = torch.cuda.Event()
        event.record(stream)
        slot.ready_event = event

    def release(self, slot: StagingSlot) -> None:
        if not slot.in_use:
            raise RuntimeError("Slot is not in use")
        slot.in_use = False

    def destroy(self) -> None:
        self._slots.clear()
        self.budget.used_bytes = 0

    @staticmethod
    def _tensor_bytes(tensor: Optional[torch.Tensor]) -> int:
        return 0 if tensor is None else tensor.numel() * tensor.element_size()

    @classmethod
    def _projection_state(cls, expert, name: str) -> dict:
        """One projection in the canonical staging representation."""
        projection = getattr(expert, name)
        if isinstance(projection, dict):
            raw = projection
        else:
            raw = getattr(projection, "state", None)
            if raw is None and hasattr(projection, "serialized"):
                raw = projection.serialized()
        if not isinstance(raw, dict):
            raise TypeError(f"Expert projection {name!r} does not expose serialized NF4 state")
        if "weight" not in raw:
            raise ValueError(f"Projection {name!r} is missing 'weight'")

        if "absmax" in raw and ("code" in raw or "quant_map" in raw):
            canonical = {"weight": raw["weight"], "absmax": raw["absmax"],
                         "code": raw.get("code", raw.get("quant_map")),
                         "offset": raw.get("offset")}
            for key in ("state2_absmax", "state2_code", "state2_offset"):
                if key in raw:
                    canonical[key] = raw[key]
            if canonical["code"] is None:
                raise ValueError(f"Projection {name!r} is missing NF4 code/quant_map")
            return canonical

        required = {"weight.absmax", "weight.quant_map", _BLOB}
        missing = required - raw.keys()
        if missing:
            raise ValueError(f"Projection {name!r} is missing serialized NF4 state tensors: "
                             f"{sorted(missing)}")
        meta = parse_blob(raw[_BLOB])
        canonical = {"weight": raw["weight"], "absmax": raw["weight.absmax"],
                     "code": raw["weight.quant_map"], "offset": None}
        if "weight.nested_absmax" in raw:
            canonical["state2_absmax"] = raw["weight.nested_absmax"]
            canonical["state2_code"] = raw.get("weight.nested_quant_map")
            off = meta.get("nested_offset")
            canonical["state2_offset"] = None
            canonical["offset"] = None if off is None else torch.tensor(off, dtype=torch.float32)
        return canonical

    @classmethod
    def _expert_staging_size(cls, expert) -> int:
        return sum(cls._tensor_bytes(t) for name in cls._PROJECTIONS
                   for t in cls._projection_state(expert, name).values())

    def stage_expert(self, slot: StagingSlot, expert, layer_id: int, expert_id: int) -> None:
        """Copy the expert's NF4 tensors into the slot's pinned buffers (reused in place
        when shapes match)."""
        if not slot.in_use:
            raise RuntimeError("Slot must be acquired before staging")
        old = slot.tensors
        staged = {}
        for name in self._PROJECTIONS:
            source = self._projection_state(expert, name)
            prev = old.get(name, {})
            staged[name] = {key: self._copy_into_pinned(t, prev.get(key))
                            for key, t in source.items()}
        slot.tensors = staged
        slot.expert_key = (layer_id, expert_id)

    @staticmethod
    def _copy_into_pinned(source: Optional[torch.Tensor],
                          existing: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
        if source is None:
            return None
        if existing is None:
            existing = torch.empty_like(source, device="cpu", pin_memory=True)
        if existing.shape != source.shape or existing.dtype != source.dtype:
            raise ValueError("Existing staging buffer does not match source tensor")
        existing.copy_(source)
        return existing
