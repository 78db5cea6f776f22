"""Host-to-device copy of a staged NF4 expert: transfer_staged_expert_to_gpu, the API of the
reference's transfer/nf4_transfer.py:8-40.

Every tensor of the staging slot is copied with a non-blocking copy (hipMemcpyAsync from
pinned memory) enqueued on `stream`; the returned device tensors are allocated on that
stream.  The caller orders consumers after the copies (an event recorded on `stream`) and
keeps the slot until they have run.  The transfer scheduler itself copies into preallocated
device slots instead (scheduler.py); this function is the per-tensor form for callers of
the reference's API.
"""
from __future__ import annotations

import torch

from .reusable_staging import StagingSlot


def transfer_staged_expert_to_gpu(slot: StagingSlot, stream, device="cuda") -> dict:
    if not slot.in_use:
        raise RuntimeError(f"staging slot {slot.slot_id} must be acquired before its transfer")
    with torch.cuda.stream(stream):
        return {name: {key: None if t is None else t.to(device, non_blocking=True)
                       for key, t in state.items()}
                for name, state in slot.tensors.items()}
