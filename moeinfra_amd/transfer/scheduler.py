"""Expert-transfer scheduler (mirrors transfer/scheduler.py:35-628 of the reference).

The scheduler orders, deduplicates and cancels residency requests; the CacheManager owns
the experts.  A CPU_TO_GPU transfer stages the CPU-authoritative NF4 expert into a pinned
slot, copies it to the device on the transfer stream, wraps it as a
ReconstructedNF4Expert and inserts it in the GPU tier.  ``execute_next`` waits for the
copy (the reference's synchronous path); ``submit_async``/``poll_async`` leave it in
flight and finish it when its event has completed.
"""
from __future__ import annotations

import heapq
import logging
import time
from typing import Optional

import torch

from .bandwidth import BandwidthMonitor
from .nf4_reconstruct import ReconstructedNF4Expert
from .nf4_transfer import transfer_staged_expert_to_gpu
from .types import (TransferDirection, TransferHandle, TransferRequest, TransferResult,
                    TransferStatus)

#: Per-stage timings of every execute_next call (ms), as the reference records them.
EXECUTE_NEXT_PROFILE: list[dict] = []


def _keep_for_compute(gpu_state: dict) -> None:
    """The copies were allocated on the transfer stream and are read by kernels on the
    current stream: tell the caching allocator so their memory is not reused early."""
    cur = torch.cuda.current_stream()
    for proj in gpu_state.values():
        for t in proj.values():
            if t is not None:
                t.record_stream(cur)


class TransferScheduler:
    """Priority-queue scheduler for expert residency transfers."""

    def __init__(self, cache_manager, bandwidth_gbps: float, max_concurrent: int,
                 staging_pool=None, transfer_stream=None,
                 logger: Optional[logging.Logger] = None) -> None:
        if max_concurrent <= 0:
            raise ValueError("max_concurrent must be positive")
        self._cache_manager = cache_manager
        self.bandwidth_gbps = bandwidth_gbps
        self.max_concurrent = max_concurrent
        self._logger = logger or logging.getLogger(__name__)
        self._bw_monitor = BandwidthMonitor(window_s=5.0)
        self._heap: list = []
        self._queue: list[TransferRequest] = []
        self._in_flight: list[TransferRequest] = []
        self._staging_pool = staging_pool
        self._transfer_stream = transfer_stream
        self._async_in_flight: dict[tuple[int, int], TransferHandle] = {}
        self._seq = 0

    # ------------------------------------------------------------------ queue
    def _is_duplicate(self, request: TransferRequest) -> bool:
        triple = (request.layer_id, request.expert_id, request.direction)
        for other in (*self._queue, *self._in_flight):
            if other.request_id == request.request_id:
                return True
            if (other.layer_id, other.expert_id, other.direction) == triple:
                return True
        return (request.layer_id, request.expert_id) in self._async_in_flight

    @staticmethod
    def _sort_key(request: TransferRequest) -> tuple[int, float]:
        return (request.priority.value, request.issued_at)

    def submit(self, request: TransferRequest) -> bool:
        """Queue a request unless an equivalent one is queued or executing."""
        if self._is_duplicate(request):
            return False
        self._seq += 1
        heapq.heappush(self._heap, (self._sort_key(request), self._seq, request))
        self._queue.append(request)
        return True

    def pending_count(self) -> int:
        return len(self._queue)

    @property
    def bandwidth_monitor(self) -> BandwidthMonitor:
        return self._bw_monitor

    # ------------------------------------------------------------------ synchronous path
    def execute_next(self) -> Optional[TransferResult]:
        """Run the highest-priority pending transfer and wait for it."""
        if not self._heap:
            return None
        _, _, request = heapq.heappop(self._heap)
        self._queue.remove(request)
        self._in_flight.append(request)
        started = time.perf_counter()
        nbytes = 0
        error: Optional[str] = None
        success = False
        profile = {"layer_id": request.layer_id, "expert_id": request.expert_id,
                   "direction": request.direction.value}
        try:
            nbytes = self._cache_manager.get_size_bytes(request.layer_id, request.expert_id)
            if request.direction == TransferDirection.CPU_TO_GPU:
                success = self._cpu_to_gpu(request, profile)
            elif request.direction == TransferDirection.GPU_TO_CPU:
                t = time.perf_counter()
                success = self._cache_manager.demote_to_cpu(request.layer_id, request.expert_id)
                profile["demotion_ms"] = (time.perf_counter() - t) * 1e3
            else:
                raise ValueError(f"Unsupported transfer direction: {request.direction!r}")
            if not success:
                error = (f"Transfer failed for layer={request.layer_id}, "
                         f"expert={request.expert_id}, direction={request.direction.value}")
        except Exception as exc:  # the failure is reported in the result
            error = str(exc)
            self._logger.error("execute_next: FAILED id=%s error=%s", request.request_id, error)
        elapsed_ms = (time.perf_counter() - started) * 1e3
        profile.update(total_execute_next_ms=elapsed_ms, success=success,
                       bytes_transferred=nbytes if success else 0)
        EXECUTE_NEXT_PROFILE.append(profile)
        self._in_flight.remove(request)
        if success:
            self._bw_monitor.record(nbytes)
        return TransferResult(request_id=request.request_id, success=success,
                              elapsed_ms=elapsed_ms, bytes_transferred=nbytes if success else 0,
                              error=error)

    def _cpu_to_gpu(self, request: TransferRequest, profile: dict) -> bool:
        if self._staging_pool is None or self._transfer_stream is None:
            raise RuntimeError("Synchronous CPU_TO_GPU transfer requires staging_pool and "
                               "transfer_stream")
        cpu_expert = self._cache_manager.peek_cpu(request.layer_id, request.expert_id)
        if cpu_expert is None:
            raise RuntimeError(f"CPU expert not found in cache: layer={request.layer_id}, "
                               f"expert={request.expert_id}")
        slot = self._staging_pool.acquire()
        if slot is None:
            raise RuntimeError("No staging slot available for synchronous transfer")
        try:
            t = time.perf_counter()
            self._staging_pool.stage_expert(slot, cpu_expert, request.layer_id, request.expert_id)
            profile["staging_ms"] = (time.perf_counter() - t) * 1e3
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            t = time.perf_counter()
            start.record(self._transfer_stream)
            gpu_state = transfer_staged_expert_to_gpu(slot, self._transfer_stream)
            end.record(self._transfer_stream)
            self._transfer_stream.synchronize()
            profile["h2d_wall_ms"] = (time.perf_counter() - t) * 1e3
            profile["h2d_cuda_ms"] = start.elapsed_time(end)
            _keep_for_compute(gpu_state)
            t = time.perf_counter()
            gpu_expert = ReconstructedNF4Expert(cpu_expert, gpu_state)
            profile["reconstruction_call_ms"] = (time.perf_counter() - t) * 1e3
            t = time.perf_counter()
            self._cache_manager.put(request.layer_id, request.expert_id, gpu_expert,
                                    device="cuda:0")
            profile["cache_put_call_ms"] = (time.perf_counter() - t) * 1e3
            return True
        finally:
            self._staging_pool.release(slot)

    def drain(self) -> list[TransferResult]:
        results = []
        while self._heap:
            r = self.execute_next()
            if r is not None:
                results.append(r)
        return results

    def cancel(self, request_id: str) -> bool:
        """Drop a queued request, or mark an in-flight async transfer cancelled (its DMA
        cannot be aborted; the slot is kept until the copy's event completes)."""
        target = next((r for r in self._queue if r.request_id == request_id), None)
        if target is not None:
            self._queue.remove(target)
            self._heap = [(self._sort_key(r), i, r) for i, r in enumerate(self._queue)]
            heapq.heapify(self._heap)
            return True
        handle = next((h for h in self._async_in_flight.values() if h.request_id == request_id),
                      None)
        if handle is None or handle.status != TransferStatus.IN_FLIGHT:
            return False
        handle.status = TransferStatus.CANCELLED
        return True

    # ------------------------------------------------------------------ asynchronous path
    def submit_async(self, request: TransferRequest) -> TransferHandle:
        """Start a CPU->GPU transfer on the transfer stream without waiting for it."""
        if request.direction != TransferDirection.CPU_TO_GPU:
            raise ValueError("submit_async() only supports CPU_TO_GPU transfers")
        key = (request.layer_id, request.expert_id)
        mk = lambda status, slot=None, event=None: TransferHandle(
            request_id=request.request_id, layer_id=request.layer_id,
            expert_id=request.expert_id, slot=slot, event=event, status=status)
        if self._cache_manager.is_gpu_resident(*key):
            return mk(TransferStatus.READY)
        existing = self._async_in_flight.get(key)
        if existing is not None:
            return existing
        if len(self._async_in_flight) >= self.max_concurrent:
            return mk(TransferStatus.REJECTED)
        if self._staging_pool is None or self._transfer_stream is None:
            raise RuntimeError("Async transfer requires staging_pool and transfer_stream")
        slot = self._staging_pool.acquire()
        if slot is None:
            return mk(TransferStatus.REJECTED)
        expert = self._cache_manager.peek_cpu(*key)
        if expert is None:
            self._staging_pool.release(slot)
            return mk(TransferStatus.REJECTED)
        try:
            self._staging_pool.stage_expert(slot, expert, *key)
            gpu_state = transfer_staged_expert_to_gpu(slot, self._transfer_stream)
            event = torch.cuda.Event()
            event.record(self._transfer_stream)
            handle = mk(TransferStatus.IN_FLIGHT, slot, event)
            handle.gpu_state = gpu_state
            handle.cpu_expert = expert
            self._async_in_flight[key] = handle
            return handle
        except Exception:
            self._staging_pool.release(slot)
            raise

    def poll_async(self, layer_id: int, expert_id: int) -> TransferStatus:
        """Finish an async transfer whose copy has completed."""
        key = (layer_id, expert_id)
        handle = self._async_in_flight.get(key)
        if handle is None:
            return TransferStatus.REJECTED
        done = handle.event.query()
        if handle.status == TransferStatus.CANCELLED:
            if not done:
                return TransferStatus.CANCELLED
            self._staging_pool.mark_transfer_complete(handle.slot, self._transfer_stream)
            self._staging_pool.release(handle.slot)
            del self._async_in_flight[key]
            return TransferStatus.CANCELLED
        if not done:
            return TransferStatus.IN_FLIGHT
        try:
            _keep_for_compute(handle.gpu_state)
            expert = ReconstructedNF4Expert(handle.cpu_expert, handle.gpu_state)
            self._cache_manager.put(layer_id, expert_id, expert, device="cuda")
            handle.status = TransferStatus.READY
            self._staging_pool.mark_transfer_complete(handle.slot, self._transfer_stream)
            self._staging_pool.release(handle.slot)
            del self._async_in_flight[key]
            return TransferStatus.READY
        except Exception:
            handle.status = TransferStatus.REJECTED
            self._staging_pool.release(handle.slot)
            del self._async_in_flight[key]
            raise

    def __repr__(self) -> str:
        return (f"TransferScheduler(pending={len(self._queue)}, in_flight={len(self._in_flight)}, "
                f"bandwidth={self.bandwidth_gbps:.1f} GB/s)")
