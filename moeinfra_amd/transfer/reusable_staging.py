"""Pinned host staging for expert transfers: the ReusablePinnedStagingPool / StagingSlot API
of the reference's transfer/reusable_staging.py:20-284.

A slot is a pinned host buffer set that one transfer reads from.  Its ``ready_event`` is
recorded on the transfer stream behind the copies that read it; ``acquire`` hands a slot
out again only once that event has completed, so a host buffer is never rewritten under a
DMA.  Slots are created lazily within a PinnedMemoryBudget and never shrink.

Staging an expert fills ``slot.tensors`` with its canonical per-projection tensors
(expert_image.canonical_projection).  Tensors that already live in pinned memory -- the
offload store is pinned once, see host_store.py -- are referenced as they are: nothing is
copied and the DMA reads the store directly.  Pageable tensors are copied into buffers the
slot owns, which later stagings of the same shapes reuse in place, so the slot's addresses
stay fixed; the source expert is never modified or pinned.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch

from .expert_image import PROJECTIONS, canonical_projection
from .pinned_memory import PinnedMemoryBudget


@dataclasses.dataclass
class StagingSlot:
    slot_id: int
    size_bytes: int
    tensors: dict
    in_use: bool = False
    ready_event: Optional[torch.cuda.Event] = None
    expert_key: Optional[tuple[int, int]] = None
    # pinned buffers owned by the slot, per (projection, key)
    owned: dict = dataclasses.field(default_factory=dict)
    # bytes of the last staging that had to be copied (0 when everything was pinned)
    copied_bytes: int = 0


class ReusablePinnedStagingPool:
    """Bounded set of reusable pinned staging slots."""

    _PROJECTIONS = PROJECTIONS

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
        return sum(1 for s in self._slots.values() if s.in_use)

    @staticmethod
    def _reusable(slot: StagingSlot) -> bool:
        if slot.in_use:
            return False
        ev = slot.ready_event
        if ev is not None and not ev.query():
            return False
        slot.ready_event = None
        return True

    def acquire(self) -> Optional[StagingSlot]:
        """An idle slot whose last DMA has finished, else a new slot if the budget allows,
        else None."""
        slot = next((s for s in self._slots.values() if self._reusable(s)), None)
        if slot is None:
            if not self.budget.reserve(self.slot_size_bytes):
                return None
            slot = StagingSlot(slot_id=len(self._slots), size_bytes=self.slot_size_bytes,
                               tensors={})
            self._slots[slot.slot_id] = slot
        slot.in_use = True
        return slot

    def mark_transfer_complete(self, slot: StagingSlot, stream) -> None:
        """Gate the slot's reuse on everything issued to `stream` so far (its copies)."""
        if not slot.in_use:
            raise RuntimeError(f"staging slot {slot.slot_id} is not acquired")
        ev = torch.cuda.Event()
        ev.record(stream)
        slot.ready_event = ev

    def release(self, slot: StagingSlot) -> None:
        if not slot.in_use:
            raise RuntimeError(f"staging slot {slot.slot_id} is not acquired")
        slot.in_use = False

    def destroy(self) -> None:
        self._slots.clear()
        self.budget.used_bytes = 0

    @classmethod
    def _projection_state(cls, expert, name: str) -> dict:
        return canonical_projection(expert, name)

    @classmethod
    def _expert_staging_size(cls, expert) -> int:
        return sum(t.numel() * t.element_size() for name in PROJECTIONS
                   for t in canonical_projection(expert, name).values() if t is not None)

    def _pinned_copy(self, slot: StagingSlot, where: tuple, src: torch.Tensor) -> torch.Tensor:
        buf = slot.owned.get(where)
        if buf is None or buf.shape != src.shape or buf.dtype != src.dtype:
            buf = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
            slot.owned[where] = buf
        buf.copy_(src)
        slot.copied_bytes += buf.numel() * buf.element_size()
        return buf

    def stage_expert(self, slot: StagingSlot, expert, layer_id: int, expert_id: int) -> None:
        """Point the slot at the expert's device tensors, copying only what is pageable."""
        if not slot.in_use:
            raise RuntimeError(f"staging slot {slot.slot_id} must be acquired before staging")
        slot.copied_bytes = 0
        staged = {}
        for name in PROJECTIONS:
            state = {}
            for key, t in canonical_projection(expert, name).items():
                if t is None:
                    state[key] = None
                elif t.device.type == "cpu" and t.is_pinned():
                    state[key] = t
                else:
                    state[key] = self._pinned_copy(slot, (name, key), t)
            staged[name] = state
        slot.tensors = staged
        slot.expert_key = (layer_id, expert_id)
