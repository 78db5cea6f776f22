"""Expert prefetch ahead of the compute (mirrors engine/prefetch.py:53-309 of the reference).

After a layer completes, the experts it routed to are taken as the prediction for the next
layer (NEXT_LAYER) or the next ``depth`` layers (LOOKAHEAD) and their CPU->GPU copies are
started on the transfer scheduler's side stream (``submit_async``), so that the H2D of
layer l+1 overlaps the compute of layer l.  Requests for layers already passed are cancelled.
Same policy names, method names, return values and bookkeeping as the reference.
"""
from __future__ import annotations

import logging
import time
import uuid
from typing import List, Optional

import torch

from ..transfer.types import TransferDirection, TransferPriority, TransferRequest, TransferStatus
from .types import PrefetchPolicy


class PrefetchEngine:
    """Lookahead expert prefetch scheduler (engine/prefetch.py:53)."""

    def __init__(self, cache_manager, transfer_scheduler, policy: PrefetchPolicy, depth: int,
                 logger: Optional[logging.Logger] = None) -> None:
        self._cache_manager = cache_manager
        self._transfer_scheduler = transfer_scheduler
        self.policy: PrefetchPolicy = policy
        self.depth: int = depth
        self._logger = logger or logging.getLogger(__name__)
        # (layer_id, expert_id) -> request_id of the prefetches in flight.
        self._in_flight: dict[tuple[int, int], str] = {}

    def _is_gpu_resident(self, layer_id: int, expert_id: int) -> bool:
        return self._cache_manager.is_gpu_resident(layer_id, expert_id)

    def _submit_if_needed(self, layer_id: int, expert_id: int) -> Optional[str]:
        """Start a CPU->GPU prefetch unless it is in flight or resident (prefetch.py:128-181)."""
        key = (layer_id, expert_id)
        if key in self._in_flight:
            return None
        if self._is_gpu_resident(layer_id, expert_id):
            return None
        request_id = str(uuid.uuid4())
        request = TransferRequest(request_id=request_id, layer_id=layer_id, expert_id=expert_id,
                                  direction=TransferDirection.CPU_TO_GPU,
                                  priority=TransferPriority.LOW, issued_at=time.monotonic())
        handle = self._transfer_scheduler.submit_async(request)
        if handle.status != TransferStatus.IN_FLIGHT:
            self._logger.debug("prefetch not accepted: layer=%d expert=%d status=%s", layer_id,
                               expert_id, handle.status.value)
            return None
        self._in_flight[key] = request_id
        return request_id

    def _predict_experts(self, expert_indices: torch.Tensor) -> List[int]:
        """Sorted distinct expert ids of a routing result (prefetch.py:183-194)."""
        return sorted(int(x) for x in expert_indices.reshape(-1).unique().tolist())

    def schedule_prefetch(self, current_layer: int, expert_indices: torch.Tensor) -> List[str]:
        """Submit prefetches for the layers after ``current_layer`` (prefetch.py:200-250)."""
        if self.policy == PrefetchPolicy.NONE:
            return []
        predicted = self._predict_experts(expert_indices)
        if self.policy == PrefetchPolicy.NEXT_LAYER:
            targets = [current_layer + 1]
        else:
            targets = list(range(current_layer + 1, current_layer + self.depth + 1))
        submitted: List[str] = []
        for target in targets:
            for expert_id in predicted:
                req_id = self._submit_if_needed(target, expert_id)
                if req_id is not None:
                    submitted.append(req_id)
        return submitted

    def on_layer_complete(self, layer_id: int, expert_indices: torch.Tensor) -> None:
        """Cancel stale prefetches, then schedule the next ones (prefetch.py:252-277)."""
        self.cancel_stale(current_layer=layer_id + 1)
        self.schedule_prefetch(current_layer=layer_id, expert_indices=expert_indices)

    def cancel_stale(self, current_layer: int) -> int:
        """Cancel in-flight prefetches for layers below ``current_layer`` (prefetch.py:279-309)."""
        stale = [key for key in self._in_flight if key[0] < current_layer]
        cancelled = 0
        for key in stale:
            request_id = self._in_flight.pop(key)
            if self._transfer_scheduler.cancel(request_id):
                cancelled += 1
        return cancelled

    def poll(self) -> None:
        """Finish the prefetches whose copies have completed (makes them GPU-resident)."""
        for key in list(self._in_flight):
            status = self._transfer_scheduler.poll_async(*key)
            if status in (TransferStatus.READY, TransferStatus.CANCELLED, TransferStatus.REJECTED):
                self._in_flight.pop(key, None)
