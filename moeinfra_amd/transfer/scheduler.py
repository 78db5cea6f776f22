"""Expert-residency transfer scheduler: the TransferScheduler API of the reference's
transfer/scheduler.py:35-628 (submit / execute_next / drain / cancel / pending_count /
submit_async / poll_async / bandwidth_monitor), built for this package's offload path.

Bringing expert (layer, expert) onto the GPU:

1. *Room.*  ``cache.make_room_gpu`` evicts what the policy picks.
2. *Destination.*  A slot of the device arena, created on the first transfer with one slot
   per GPU-tier entry, sized by the first expert's image.  The expert owns the slot's lease:
   once nothing references the expert any more (the tier dropped it and so did every layer
   that held it), the slot goes back behind a fence on the compute stream
   (device_slots.py), and the next copy into it waits on that fence on the transfer stream,
   so no queued kernel still reading the slot is overtaken.  When every slot is held, the
   expert gets a buffer of its own, equally fenced.
3. *Source.*  An expert of the pinned store (host_store.py) crosses as one hipMemcpyAsync
   of its contiguous image; any other CPU expert is staged through a pinned staging slot
   (pageable tensors copied, pinned ones referenced) and copied tensor by tensor.  The
   staging slot's reuse is gated on the copies' completion event.
4. *Residency.*  The expert -- a ReconstructedNF4Expert whose tensors are views into the
   slot -- enters the GPU tier at once, carrying the copy's completion event as its
   ``ready_event``.  Consumers order their kernels after it with a stream wait
   (``ReconstructedNF4Expert.wait_ready``); the host does not wait.

``execute_next`` additionally waits on the host for the copy to finish (the reference's
synchronous contract) and records per-stage timings in ``EXECUTE_NEXT_PROFILE``;
``submit_async`` returns a TransferHandle at once, ``poll_async`` reports and retires it,
and ``cancel`` of an in-flight transfer drops the expert from the GPU tier (its slot is
rewritten only after the copy, which the transfer stream orders anyway).

The request queue is a heap ordered by (priority, issue time, submission order) with
cancelled entries skipped when they surface; duplicates -- the same request id, or the
same (layer, expert, direction) queued, executing or in flight -- are refused.
"""
from __future__ import annotations

import heapq
import itertools
import logging
import time
from typing import Optional

import torch

from .bandwidth import BandwidthMonitor
from .device_slots import DeviceExpertSlots
from .expert_image import ImageLayout
from .nf4_reconstruct import ReconstructedNF4Expert
from .types import (TransferDirection, TransferHandle, TransferRequest, TransferResult,
                    TransferStatus)

#: Per-stage timings (ms) of every execute_next call: staging_ms, h2d_wall_ms, h2d_cuda_ms,
#: total_execute_next_ms, plus layer_id, expert_id, direction, source ("image" or
#: "staged"), success and bytes_transferred.
EXECUTE_NEXT_PROFILE: list[dict] = []


class _Rejected(Exception):
    """No staging or device slot for a transfer right now."""


class TransferScheduler:
    """Priority queue and copy engine for expert residency changes."""

    def __init__(self, cache_manager, bandwidth_gbps: float, max_concurrent: int,
                 staging_pool=None, transfer_stream=None,
                 logger: Optional[logging.Logger] = None,
                 device_slots: Optional[DeviceExpertSlots] = None) -> None:
        if max_concurrent <= 0:
            raise ValueError("max_concurrent must be positive")
        self._cache_manager = cache_manager
        self.bandwidth_gbps = bandwidth_gbps
        self.max_concurrent = max_concurrent
        self._logger = logger or logging.getLogger(__name__)
        self._bw_monitor = BandwidthMonitor(window_s=5.0)
        self._staging_pool = staging_pool
        self._transfer_stream = transfer_stream
        self._device_slots = device_slots
        self._heap: list = []
        self._order = itertools.count()
        self._queued: dict[str, TransferRequest] = {}
        self._busy: dict[tuple, str] = {}          # (layer, expert, direction) -> request id
        self._async: dict[tuple[int, int], TransferHandle] = {}
        #: When a list: each host-to-device copy appends (kind, start event, end event,
        #: bytes) with timing events on the transfer stream ("image", "staged" or
        #: "prefix"), for a timeline of the host link (observability; None costs nothing).
        self.timeline: Optional[list] = None
        #: Copies issued so far, by source, and the bytes they moved over the host link
        #: ("prefix": bounded prefix copies, see start_prefix).
        self.copies = {"image": 0, "staged": 0, "prefix": 0, "bytes": 0}
        #: (layer, expert) -> (device region, slot lease, bytes already copied) of the
        #: bounded prefixes started and not yet completed or dropped.
        self._prefixes: dict[tuple[int, int], tuple] = {}

    # ------------------------------------------------------------------ queue
    def _is_duplicate(self, request: TransferRequest) -> bool:
        if request.request_id in self._queued or request.request_id in self._busy.values():
            return True
        if (request.layer_id, request.expert_id, request.direction) in self._busy:
            return True
        return (request.direction == TransferDirection.CPU_TO_GPU and
                self._live_handle(request.layer_id, request.expert_id) is not None)

    def _live_handle(self, layer_id: int, expert_id: int) -> Optional[TransferHandle]:
        """The in-flight handle of (layer_id, expert_id) whose expert is still the GPU tier's
        (one evicted before its copy finished no longer counts)."""
        h = self._async.get((layer_id, expert_id))
        if h is None or h.status != TransferStatus.IN_FLIGHT or \
                self._cache_manager.peek_gpu(layer_id, expert_id) is not h.gpu_state:
            return None
        return h

    def submit(self, request: TransferRequest) -> bool:
        """Queue a request; False (and nothing queued) for a duplicate."""
        if self._is_duplicate(request):
            return False
        key = (request.priority.value, request.issued_at, next(self._order))
        heapq.heappush(self._heap, (key, request.request_id))
        self._queued[request.request_id] = request
        self._busy[(request.layer_id, request.expert_id, request.direction)] = request.request_id
        return True

    def _pop(self) -> Optional[TransferRequest]:
        while self._heap:
            _, rid = heapq.heappop(self._heap)
            request = self._queued.pop(rid, None)
            if request is not None:
                return request
        return None

    def pending_count(self) -> int:
        return len(self._queued)

    def cancel(self, request_id: str) -> bool:
        """Withdraw a queued request, or stop an in-flight async transfer from becoming
        resident (the copy itself runs to completion).  False if there is nothing to
        cancel under that id."""
        request = self._queued.pop(request_id, None)
        if request is not None:
            self._busy.pop((request.layer_id, request.expert_id, request.direction), None)
            return True
        for key, h in self._async.items():
            if h.request_id == request_id and h.status == TransferStatus.IN_FLIGHT:
                h.status = TransferStatus.CANCELLED
                if self._cache_manager.peek_gpu(*key) is h.gpu_state:
                    self._cache_manager.demote_to_cpu(*key)
                return True
        return False

    @property
    def bandwidth_monitor(self) -> BandwidthMonitor:
        return self._bw_monitor

    # ------------------------------------------------------------------ copies
    def _slots_for(self, nbytes: int) -> DeviceExpertSlots:
        if self._device_slots is None:
            count = max(1, int(getattr(self._cache_manager, "gpu_slots", 1)))
            self._device_slots = DeviceExpertSlots(count, nbytes, self._transfer_stream.device)
        return self._device_slots

    def _destination(self, nbytes: int):
        """(device region, fence to wait on, lease to keep) for an image of `nbytes` bytes:
        a slot of the arena, or -- when every slot is held (experts still referenced beyond
        the GPU tier) or the image is larger than a slot -- a buffer of its own, whose fence
        orders the copy after the work already queued on the current stream."""
        slots = self._slots_for(nbytes)
        slot = slots.take() if nbytes <= slots.slot_bytes else None
        if slot is not None:
            return slots.region(slot, nbytes), slots.fence(slot), slots.lease(slot)
        region = torch.empty((nbytes,), dtype=torch.uint8, device=slots.device)
        region.record_stream(self._transfer_stream)
        fence = torch.cuda.Event()
        fence.record(torch.cuda.current_stream(slots.device))
        return region, fence, region

    def _issue(self, request: TransferRequest, cpu_expert, profile: dict):
        """Start the copy of `cpu_expert` into a device slot and publish it in the GPU tier.
        Returns (gpu expert, completion event); raises _Rejected without side effects when
        no staging or device slot is free."""
        if self._transfer_stream is None:
            raise RuntimeError("a CPU_TO_GPU transfer needs a transfer_stream")
        image = getattr(cpu_expert, "image", None)
        layout = getattr(cpu_expert, "image_layout", None)
        staging = None
        t0 = time.perf_counter()
        if image is None or layout is None:
            if self._staging_pool is None:
                raise RuntimeError("a CPU expert without a pinned image needs a staging_pool")
            staging = self._staging_pool.acquire()
            if staging is None:
                raise _Rejected("no staging slot")
            try:
                self._staging_pool.stage_expert(staging, cpu_expert, request.layer_id,
                                                request.expert_id)
            except Exception:
                self._staging_pool.release(staging)
                raise
            layout = ImageLayout.of(staging.tensors)
        profile["staging_ms"] = (time.perf_counter() - t0) * 1e3
        profile["source"] = "staged" if staging is not None else "image"
        key = (request.layer_id, request.expert_id)
        prefix = self._prefixes.pop(key, None) if staging is None else None
        try:
            self._cache_manager.make_room_gpu(request.layer_id, request.expert_id)
            self._in_flight_count()           # retire finished handles (they hold experts)
            if prefix is not None:            # the slot already holds the image's first bytes
                region, lease, done_bytes = prefix
                fence = None                  # honoured when the prefix was issued
            else:
                region, fence, lease = self._destination(layout.nbytes)
                done_bytes = 0
        except Exception:
            if staging is not None:
                self._staging_pool.release(staging)
            raise
        stream = self._transfer_stream
        timing = profile.get("_timing")
        tl = self.timeline
        with torch.cuda.stream(stream):
            if fence is not None:
                stream.wait_event(fence)
            if timing:
                timing[0].record(stream)
            if tl is not None:
                t_start = torch.cuda.Event(enable_timing=True)
                t_start.record(stream)
            if staging is None:                # the copy goes out before any host bookkeeping
                region[done_bytes:].copy_(image[done_bytes:], non_blocking=True)
            else:
                staged = layout.views(region)
                for f in layout.fields:
                    staged[f.projection][f.key].copy_(staging.tensors[f.projection][f.key],
                                                      non_blocking=True)
            done = torch.cuda.Event(enable_timing=bool(timing) or tl is not None)
            done.record(stream)
        if tl is not None:
            tl.append((profile["source"], t_start, done, layout.nbytes - done_bytes))
        views = layout.views(region)
        if staging is not None:
            self._staging_pool.mark_transfer_complete(staging, stream)
            self._staging_pool.release(staging)
        self.copies[profile["source"]] += 1
        self.copies["bytes"] += layout.nbytes - done_bytes
        expert = ReconstructedNF4Expert(cpu_expert, views)
        expert.ready_event = done
        expert.device_lease = lease            # the slot is reused once the expert is gone
        self._cache_manager.put(request.layer_id, request.expert_id, expert, device="cuda:0")
        return expert, done

    # ------------------------------------------------------------------ bounded prefixes
    def start_prefix(self, layer_id: int, expert_id: int, nbytes: int) -> bool:
        """Copy the first `nbytes` of the pinned image of (layer_id, expert_id) into a free
        slot of the device arena, on the transfer stream, without publishing the expert: a
        later transfer of the expert copies only the rest into the same slot.  A prefix
        costs the host link `nbytes` whether or not the expert is routed, so a caller sizes
        it to the link's idle time between two layers' copies.  False (nothing started) when
        the expert is resident, in flight or already has a prefix, has no pinned image, or
        no arena slot is free (a prefix never allocates)."""
        key = (layer_id, expert_id)
        if self._transfer_stream is None or key in self._prefixes or \
                self._live_handle(*key) is not None or self._cache_manager.is_gpu_resident(*key):
            return False
        cpu_expert = self._cache_manager.peek_cpu(*key)
        image = getattr(cpu_expert, "image", None)
        layout = getattr(cpu_expert, "image_layout", None)
        if image is None or layout is None:
            return False
        nbytes = min(int(nbytes), layout.nbytes)
        slots = self._slots_for(layout.nbytes)
        if nbytes <= 0 or layout.nbytes > slots.slot_bytes:
            return False
        slot = slots.take()
        if slot is None:
            return False
        region, fence, lease = slots.region(slot, layout.nbytes), slots.fence(slot), slots.lease(slot)
        stream = self._transfer_stream
        tl = self.timeline
        with torch.cuda.stream(stream):
            if fence is not None:
                stream.wait_event(fence)
            if tl is not None:
                t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t_start.record(stream)
            region[:nbytes].copy_(image[:nbytes], non_blocking=True)
            if tl is not None:
                t_end.record(stream)
                tl.append(("prefix", t_start, t_end, nbytes))
        self._prefixes[key] = (region, lease, nbytes)
        self.copies["prefix"] += 1
        self.copies["bytes"] += nbytes
        return True

    def drop_prefix(self, layer_id: int, expert_id: int) -> bool:
        """Give back the slot of an unused prefix (fenced like any slot: the transfer stream
        orders a later copy into it after the prefix copy).  False if there is none -- the
        expert's transfer consumed it, or none was started."""
        return self._prefixes.pop((layer_id, expert_id), None) is not None

    # ------------------------------------------------------------------ synchronous path
    def execute_next(self) -> Optional[TransferResult]:
        """Run the highest-priority queued request to completion (host waits for its copy)."""
        request = self._pop()
        if request is None:
            return None
        triple = (request.layer_id, request.expert_id, request.direction)
        started = time.perf_counter()
        profile = {"layer_id": request.layer_id, "expert_id": request.expert_id,
                   "direction": request.direction.value}
        nbytes, success, error = 0, False, None
        try:
            nbytes = self._cache_manager.get_size_bytes(request.layer_id, request.expert_id)
            if request.direction == TransferDirection.CPU_TO_GPU:
                success = self._bring_in(request, profile)
            elif request.direction == TransferDirection.GPU_TO_CPU:
                success = self._cache_manager.demote_to_cpu(request.layer_id, request.expert_id)
            else:
                raise ValueError(f"Unsupported transfer direction: {request.direction!r}")
            if not success:
                error = (f"Transfer failed for layer={request.layer_id}, "
                         f"expert={request.expert_id}, direction={request.direction.value}")
        except Exception as exc:            # reported in the result, as the reference does
            error = str(exc) or repr(exc)
            self._logger.error("execute_next: request %s failed: %s", request.request_id, error)
        finally:
            self._busy.pop(triple, None)
        elapsed_ms = (time.perf_counter() - started) * 1e3
        profile.pop("_timing", None)
        profile.update(total_execute_next_ms=elapsed_ms, success=success,
                       bytes_transferred=nbytes if success else 0)
        EXECUTE_NEXT_PROFILE.append(profile)
        if success:
            self._bw_monitor.record(nbytes)
        return TransferResult(request_id=request.request_id, success=success,
                              elapsed_ms=elapsed_ms, bytes_transferred=nbytes if success else 0,
                              error=error)

    def _bring_in(self, request: TransferRequest, profile: dict) -> bool:
        key = (request.layer_id, request.expert_id)
        resident = self._cache_manager.peek_gpu(*key)
        if resident is not None:             # arriving already (async) or resident
            ev = getattr(resident, "ready_event", None)
            if ev is not None:
                ev.synchronize()
            return True
        cpu_expert = self._cache_manager.peek_cpu(*key)
        if cpu_expert is None:
            raise RuntimeError(f"CPU expert not found in cache: layer={key[0]}, expert={key[1]}")
        profile["_timing"] = (torch.cuda.Event(enable_timing=True),)
        t = time.perf_counter()
        try:
            _, done = self._issue(request, cpu_expert, profile)
        except _Rejected:
            # Every staging slot is gated on a copy still in flight: wait for them, once.
            self._transfer_stream.synchronize()
            try:
                _, done = self._issue(request, cpu_expert, profile)
            except _Rejected as exc:
                raise RuntimeError(f"No staging slot available for synchronous transfer ({exc})")
        done.synchronize()
        profile["h2d_wall_ms"] = (time.perf_counter() - t) * 1e3 - profile.get("staging_ms", 0.0)
        profile["h2d_cuda_ms"] = profile["_timing"][0].elapsed_time(done)
        return True

    def drain(self) -> list[TransferResult]:
        """Run every queued request in priority order."""
        results = []
        while self._queued:
            r = self.execute_next()
            if r is not None:
                results.append(r)
        return results

    # ------------------------------------------------------------------ asynchronous path
    def _in_flight_count(self) -> int:
        n = 0
        for key, h in list(self._async.items()):
            if h.status == TransferStatus.IN_FLIGHT and h.event.query():
                h.status = TransferStatus.READY
                self._bw_monitor.record(h.nbytes)
            if h.status == TransferStatus.CANCELLED and h.event.query():
                del self._async[key]
            elif h.status == TransferStatus.READY and \
                    self._cache_manager.peek_gpu(*key) is not h.gpu_state:
                del self._async[key]           # finished and already evicted: nothing to report
            elif h.status == TransferStatus.IN_FLIGHT:
                n += 1
        return n

    def submit_async(self, request: TransferRequest) -> TransferHandle:
        """Start a CPU->GPU transfer and return at once: a handle IN_FLIGHT (the expert is
        already in the GPU tier, ordered behind handle.event), READY if it was resident,
        the existing handle if it is in flight, REJECTED if no slot is free, the in-flight
        limit is reached, or the CPU tier does not hold the expert."""
        if request.direction != TransferDirection.CPU_TO_GPU:
            raise ValueError("submit_async() only supports CPU_TO_GPU transfers")
        key = (request.layer_id, request.expert_id)
        handle = lambda status, event=None: TransferHandle(
            request_id=request.request_id, layer_id=key[0], expert_id=key[1], slot=None,
            event=event, status=status)
        in_flight = self._in_flight_count()
        existing = self._live_handle(*key)
        if existing is not None:
            return existing
        if self._cache_manager.is_gpu_resident(*key):
            return handle(TransferStatus.READY)
        if in_flight >= self.max_concurrent:
            return handle(TransferStatus.REJECTED)
        cpu_expert = self._cache_manager.peek_cpu(*key)
        if cpu_expert is None:
            return handle(TransferStatus.REJECTED)
        try:
            expert, done = self._issue(request, cpu_expert, {})
        except _Rejected:
            return handle(TransferStatus.REJECTED)
        h = handle(TransferStatus.IN_FLIGHT, done)
        h.gpu_state, h.cpu_expert = expert, cpu_expert
        h.nbytes = self._cache_manager.get_size_bytes(*key)   # the expert is in the GPU tier now
        self._async[key] = h
        return h

    def poll_async(self, layer_id: int, expert_id: int) -> TransferStatus:
        """Status of the async transfer of (layer_id, expert_id): IN_FLIGHT while its copy
        runs; READY once (then the handle is retired); CANCELLED for a cancelled one;
        REJECTED if there is none."""
        key = (layer_id, expert_id)
        h = self._async.get(key)
        if h is None:
            return TransferStatus.REJECTED
        done = h.event.query()
        if h.status == TransferStatus.CANCELLED:
            if done:
                del self._async[key]
            return TransferStatus.CANCELLED
        if not done:
            return TransferStatus.IN_FLIGHT
        if h.status == TransferStatus.IN_FLIGHT:
            self._bw_monitor.record(h.nbytes)
        h.status = TransferStatus.READY
        del self._async[key]
        return TransferStatus.READY

    def __repr__(self) -> str:
        return (f"TransferScheduler(pending={len(self._queued)}, "
                f"in_flight={sum(h.status == TransferStatus.IN_FLIGHT for h in self._async.values())}, "
                f"bandwidth={self.bandwidth_gbps:.1f} GB/s)")
