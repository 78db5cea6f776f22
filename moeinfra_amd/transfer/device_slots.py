"""Device memory of the GPU expert tier: equal slots carved from one allocation.

A transferred expert lives in one slot, its tensors views into it (the image layout of
expert_image.py).  A slot is held by a lease that the expert owns; when the last reference to the
expert goes (the GPU tier dropped it and so did every caller that still held it, such as a
layer that routed to it), the slot returns to the arena together with a fence: an event
recorded on the current (compute) stream at that moment, after every kernel already queued
that may read the slot.  The next copy into the slot is issued on the transfer
stream behind a wait on that fence, so the device never overwrites weights a queued kernel
still reads, and the host never blocks for it.  Copies into slots are ordered by the one
transfer stream, so a slot given back while its own copy is still in flight (a cancelled
prefetch) is safe to reuse as well.

One allocation instead of one per tensor also keeps the caching allocator out of the
offload loop: no per-transfer allocation, no cross-stream reuse to track.
"""
from __future__ import annotations

import collections
import weakref
from typing import Optional

import torch

from .expert_image import IMAGE_ALIGN


class DeviceExpertSlots:
    """`count` device slots of at least `slot_bytes` bytes each."""

    def __init__(self, count: int, slot_bytes: int, device) -> None:
        if count < 1 or slot_bytes < 1:
            raise ValueError("DeviceExpertSlots needs a positive count and slot size")
        self.count = int(count)
        self.slot_bytes = -(-int(slot_bytes) // IMAGE_ALIGN) * IMAGE_ALIGN
        self.device = torch.device(device)
        self._mem = torch.empty((self.count * self.slot_bytes,), dtype=torch.uint8,
                                device=self.device)
        self._free = collections.deque(range(self.count))
        self._fence: list[Optional[torch.cuda.Event]] = [None] * self.count

    @property
    def free_count(self) -> int:
        return len(self._free)

    def take(self) -> Optional[int]:
        """A free slot id (its fence still to be honoured by the caller), or None."""
        return self._free.popleft() if self._free else None

    def fence(self, slot: int) -> Optional[torch.cuda.Event]:
        return self._fence[slot]

    def region(self, slot: int, nbytes: int) -> torch.Tensor:
        if nbytes > self.slot_bytes:
            raise ValueError(f"{nbytes} bytes do not fit a {self.slot_bytes}-byte slot")
        base = slot * self.slot_bytes
        return self._mem[base:base + nbytes]

    def give_back(self, slot: int, fence: Optional[torch.cuda.Event]) -> None:
        self._fence[slot] = fence
        self._free.append(slot)

    def lease(self, slot: int) -> "SlotLease":
        """A lease on `slot`: the slot comes back (fenced) when the lease is collected."""
        return SlotLease(self, slot)


def _return_slot(slots: DeviceExpertSlots, slot: int) -> None:
    fence = torch.cuda.Event()
    fence.record(torch.cuda.current_stream(slots.device))
    slots.give_back(slot, fence)


class SlotLease:
    """Holds one slot while alive (CPython frees it as soon as its owner goes)."""

    def __init__(self, slots: DeviceExpertSlots, slot: int) -> None:
        self.slot = slot
        fin = weakref.finalize(self, _return_slot, slots, slot)
        fin.atexit = False
