"""Asynchronous host-to-device copy of a staged NF4 expert (mirrors
transfer/nf4_transfer.py:8-40 of the reference).

Each tensor of the pinned slot is copied with a non-blocking copy (hipMemcpyAsync from
pinned memory) on the given side stream, so the transfer can overlap expert compute on
the default stream.  The caller orders the consumer after the copies (stream sync or the
event of mark_transfer_complete) and keeps the slot until they complete.
"""
from __future__ import annotations

import torch

from .reusable_staging import StagingSlot


def transfer_staged_expert_to_gpu(slot: StagingSlot, stream, device="cuda") -> dict:
    if not slot.in_use:
        raise RuntimeError("Slot must be acquired before transfer")
    gpu_state: dict = {}
    with torch.cuda.stream(stream):
        for name in ("w1", "w2", "w3"):
            gpu_state[name] = {key: (None if t is None else t.to(device=device, non_blocking=True))
                               for key, t in slot.tensors[name].items()}
    return gpu_state
