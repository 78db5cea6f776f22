"""Expert prefetch: the PrefetchEngine API of the reference's engine/prefetch.py:53-309
(schedule_prefetch / on_layer_complete / cancel_stale, policies NONE / NEXT_LAYER /
LOOKAHEAD), plus NEXT_ROUTER.

A prefetch is a low-priority ``submit_async`` on the transfer scheduler: the expert's copy
starts on the transfer stream and the expert joins the GPU tier behind the copy's event,
so a layer that routes to it later finds it resident and only orders its kernels after the
copy.  What differs between the policies is the prediction of which (layer, expert) pairs
to start:

* NONE: nothing.
* NEXT_LAYER / LOOKAHEAD (the reference's heuristic, prefetch.py:177-192): the experts the
  completed layer routed to, for the next layer or the next ``depth`` layers.
* NEXT_ROUTER: the caller supplies the prediction through ``prefetch(layer, experts)`` or
  ``prefetch_prefix(layer, experts, nbytes)`` -- the engine runs the next layer's router on
  the current layer's MoE input.

On a host link that demand copies already keep busy (the offload decode loop moves two
99 MB experts per layer over PCIe) a wrong full-copy guess costs a whole copy, while a right
one saves at most the link's idle gap between two layers' copies.  A bounded prefix
(``prefetch_prefix``) copies only the first bytes of each guessed expert, sized to that gap:
a right guess leaves only the rest of the image to copy once the layer routes, a wrong one
costs no more than the gap.

``_in_flight`` maps (layer_id, expert_id) to the request id of each prefetch still in
flight, as in the reference (its tests inspect it); ``poll`` retires finished ones and
``cancel_stale`` cancels those for layers already passed, and drops their unused prefixes.
"""
from __future__ import annotations

import itertools
import logging
import time
from typing import Iterable, List, Optional

import torch

from ..transfer.types import TransferDirection, TransferPriority, TransferRequest, TransferStatus
from .types import PrefetchPolicy


class PrefetchEngine:
    """Starts expert copies ahead of the layers that will need them."""

    def __init__(self, cache_manager, transfer_scheduler, policy: PrefetchPolicy, depth: int,
                 logger: Optional[logging.Logger] = None) -> None:
        self._cache_manager = cache_manager
        self._transfer_scheduler = transfer_scheduler
        self.policy = policy
        self.depth = depth
        self._logger = logger or logging.getLogger(__name__)
        self._in_flight: dict[tuple[int, int], str] = {}
        self._prefixes: set[tuple[int, int]] = set()
        self._ids = itertools.count()
        self.counts = {"started": 0, "refused": 0, "cancelled": 0,
                       "prefixes": 0, "prefixes_used": 0, "prefixes_dropped": 0}

    # ------------------------------------------------------------------ starting copies
    def _start(self, layer_id: int, expert_id: int) -> Optional[str]:
        key = (layer_id, expert_id)
        if key in self._in_flight or self._cache_manager.is_gpu_resident(layer_id, expert_id):
            return None
        rid = f"prefetch-{layer_id}-{expert_id}-{next(self._ids)}"
        handle = self._transfer_scheduler.submit_async(TransferRequest(
            request_id=rid, layer_id=layer_id, expert_id=expert_id,
            direction=TransferDirection.CPU_TO_GPU, priority=TransferPriority.LOW,
            issued_at=time.monotonic()))
        if handle.status != TransferStatus.IN_FLIGHT:
            self.counts["refused"] += 1
            return None
        self._in_flight[key] = rid
        self.counts["started"] += 1
        return rid

    def prefetch(self, layer_id: int, expert_ids: Iterable[int]) -> List[str]:
        """Start the copies of the given experts of `layer_id` (ascending, each once)."""
        started = (self._start(layer_id, e) for e in sorted({int(e) for e in expert_ids}))
        return [rid for rid in started if rid is not None]

    def prefetch_prefix(self, layer_id: int, expert_ids: Iterable[int], nbytes: int) -> List[int]:
        """Start bounded prefix copies (the first `nbytes` of each image) of the given
        experts of `layer_id`; the experts whose prefix was started."""
        started = []
        for e in sorted({int(e) for e in expert_ids}):
            if self._transfer_scheduler.start_prefix(layer_id, e, nbytes):
                self._prefixes.add((layer_id, e))
                started.append(e)
        self.counts["prefixes"] += len(started)
        return started

    # ------------------------------------------------------------------ policies
    def _target_layers(self, current_layer: int) -> range:
        if self.policy == PrefetchPolicy.NEXT_LAYER:
            return range(current_layer + 1, current_layer + 2)
        if self.policy == PrefetchPolicy.LOOKAHEAD:
            return range(current_layer + 1, current_layer + 1 + self.depth)
        return range(0)                      # NONE, and NEXT_ROUTER (caller-driven)

    def schedule_prefetch(self, current_layer: int, expert_indices: torch.Tensor) -> List[str]:
        """Prefetch what the policy predicts from the current layer's routing; the request
        ids of the copies started."""
        layers = self._target_layers(current_layer)
        if not layers:
            return []
        experts = sorted({int(v) for v in expert_indices.reshape(-1).tolist()})
        return [rid for layer in layers for rid in self.prefetch(layer, experts)]

    def on_layer_complete(self, layer_id: int, expert_indices: torch.Tensor) -> None:
        """After layer `layer_id`: cancel what is now stale, then prefetch ahead."""
        self.cancel_stale(layer_id + 1)
        self.schedule_prefetch(layer_id, expert_indices)

    # ------------------------------------------------------------------ retiring
    def cancel_stale(self, current_layer: int) -> int:
        """Cancel the prefetches still in flight for layers below `current_layer`; drop
        their bookkeeping either way.  Returns how many the scheduler cancelled."""
        stale = [k for k in self._in_flight if k[0] < current_layer]
        n = 0
        for key in stale:
            if self._transfer_scheduler.cancel(self._in_flight.pop(key)):
                n += 1
        self.counts["cancelled"] += n
        for key in [k for k in self._prefixes if k[0] < current_layer]:
            self._prefixes.discard(key)
            if self._transfer_scheduler.drop_prefix(*key):
                self.counts["prefixes_dropped"] += 1
            else:                              # the layer's transfer completed it
                self.counts["prefixes_used"] += 1
        return n

    def poll(self) -> None:
        """Retire the prefetches whose copies have finished."""
        for key in list(self._in_flight):
            if self._transfer_scheduler.poll_async(*key) != TransferStatus.IN_FLIGHT:
                del self._in_flight[key]
