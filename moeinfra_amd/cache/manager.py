"""Two-tier (GPU + CPU) expert cache -- the residency hand-off of the MoE path.

Mirrors CacheManager of the reference (cache/manager.py:122-508): the CPU tier holds the
authoritative NF4 expert, the GPU tier a disposable device copy.  Device strings starting
with "cuda" or "gpu" select the GPU tier, anything else the CPU tier
(cache/manager.py:177-190).  Single-threaded by design, like the reference.

Addition: ``residency_epoch`` increases whenever the GPU tier changes, so callers can
cache per-layer views of the resident experts (the MoE layer's kernel argument table).
"""
from __future__ import annotations

import collections
import logging
import time
from typing import Any, Optional

from .types import CacheEntry, CacheStats, EvictionPolicy

Key = tuple[int, int]


def _is_gpu(device: str) -> bool:
    return device.startswith(("cuda", "gpu"))


class _Arc:
    """Adaptive Replacement Cache bookkeeping for one tier: T1 (seen once), T2 (seen
    again), ghost lists B1/B2 of recent victims, and the adaptive target size p of T1."""

    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.p = 0
        self.t1: collections.OrderedDict[Key, None] = collections.OrderedDict()
        self.t2: collections.OrderedDict[Key, None] = collections.OrderedDict()
        self.b1: collections.OrderedDict[Key, None] = collections.OrderedDict()
        self.b2: collections.OrderedDict[Key, None] = collections.OrderedDict()

    def hit(self, key: Key) -> None:
        if key in self.t1:
            del self.t1[key]
            self.t2[key] = None
        elif key in self.t2:
            self.t2.move_to_end(key)

    def insert(self, key: Key) -> None:
        if key in self.b1:   # T1 was too small: grow its target
            self.p = min(self.capacity, self.p + max(1, len(self.b2) // max(1, len(self.b1))))
            del self.b1[key]
        elif key in self.b2:  # T2 was too small: shrink T1's target
            self.p = max(0, self.p - max(1, len(self.b1) // max(1, len(self.b2))))
            del self.b2[key]
        self.t1[key] = None
        for ghost in (self.b1, self.b2):
            while len(ghost) > self.capacity:
                ghost.popitem(last=False)

    def victim(self) -> Optional[Key]:
        if not self.t1 and not self.t2:
            return None
        if self.t1 and (len(self.t1) > self.p or not self.t2):
            key, _ = self.t1.popitem(last=False)
            self.b1[key] = None
        else:
            key, _ = self.t2.popitem(last=False)
            self.b2[key] = None
        return key

    def remove(self, key: Key) -> None:
        self.t1.pop(key, None)
        self.t2.pop(key, None)


class CacheManager:
    """Two-level LRU/LFU/ARC expert cache (GPU tier disposable, CPU tier authoritative)."""

    def __init__(self, gpu_slots: int, cpu_slots: int, policy: EvictionPolicy,
                 logger: Optional[logging.Logger] = None) -> None:
        self.gpu_slots = gpu_slots
        self.cpu_slots = cpu_slots
        self.policy = policy
        self._gpu_cache: dict[Key, CacheEntry] = {}
        self._cpu_cache: dict[Key, CacheEntry] = {}
        self._stats = CacheStats()
        self._logger = logger or logging.getLogger(__name__)
        self._arc_gpu = _Arc(gpu_slots)
        self._arc_cpu = _Arc(cpu_slots)
        self._epoch = 0

    # ------------------------------------------------------------------ helpers
    def _tier(self, device: str) -> dict[Key, CacheEntry]:
        return self._gpu_cache if _is_gpu(device) else self._cpu_cache

    def _limit(self, device: str) -> int:
        return self.gpu_slots if _is_gpu(device) else self.cpu_slots

    def _arc(self, device: str) -> _Arc:
        return self._arc_gpu if _is_gpu(device) else self._arc_cpu

    def _touch(self, key: Key, entry: CacheEntry) -> None:
        entry.last_access = time.monotonic()
        entry.access_count += 1
        if self.policy == EvictionPolicy.ARC:
            self._arc(entry.device).hit(key)

    def _sync_slots(self) -> None:
        self._stats.gpu_slots_used = len(self._gpu_cache)
        self._stats.cpu_slots_used = len(self._cpu_cache)

    @property
    def residency_epoch(self) -> int:
        """Increases on every change of the GPU tier."""
        return self._epoch

    # ------------------------------------------------------------------ public API
    def get(self, layer_id: int, expert_id: int) -> Optional[Any]:
        """GPU tier first, then CPU; updates access metadata and hit/miss counters."""
        key = (layer_id, expert_id)
        for tier in (self._gpu_cache, self._cpu_cache):
            entry = tier.get(key)
            if entry is not None:
                self._touch(key, entry)
                self._stats.hits += 1
                return entry.expert
        self._stats.misses += 1
        return None

    def put(self, layer_id: int, expert_id: int, expert: Any, device: str) -> None:
        """Insert (evicting from a full tier first) or refresh an entry."""
        key = (layer_id, expert_id)
        tier = self._tier(device)
        if key in tier:
            entry = tier[key]
            entry.expert = expert
            entry.device = device
            self._touch(key, entry)
            if _is_gpu(device):
                self._epoch += 1
            return
        if len(tier) >= self._limit(device):
            if self.evict(device) is None:
                self._logger.warning(
                    "put: eviction returned None despite tier being full "
                    "(layer=%d expert=%d device=%s)", layer_id, expert_id, device)
        tier[key] = CacheEntry(expert_id=expert_id, layer_id=layer_id, device=device,
                               expert=expert, last_access=time.monotonic(), access_count=1,
                               size_bytes=expert.size_bytes)
        if self.policy == EvictionPolicy.ARC:
            self._arc(device).insert(key)
        if _is_gpu(device):
            self._epoch += 1
        self._sync_slots()

    def evict(self, device: str) -> Optional[CacheEntry]:
        """Remove one entry of the tier chosen by the policy; None if the tier is empty."""
        tier = self._tier(device)
        if not tier:
            return None
        if self.policy == EvictionPolicy.LRU:
            key = min(tier, key=lambda k: tier[k].last_access)
        elif self.policy == EvictionPolicy.LFU:
            key = min(tier, key=lambda k: (tier[k].access_count, tier[k].last_access))
        else:
            key = self._arc(device).victim()
            if key is None or key not in tier:
                key = min(tier, key=lambda k: tier[k].last_access)
        entry = tier.pop(key)
        if _is_gpu(device):
            # GPU entries are disposable working copies; the CPU tier keeps the
            # authoritative expert (cache/manager.py:369-373).
            entry.device = "cuda"
            self._epoch += 1
        if self.policy == EvictionPolicy.ARC:
            self._arc(device).remove(key)
        self._stats.evictions += 1
        self._sync_slots()
        return entry

    def promote_to_gpu(self, layer_id: int, expert_id: int) -> bool:
        """True if already GPU-resident; residency is otherwise established by the
        TransferScheduler (cache/manager.py:390-418)."""
        return self.is_gpu_resident(layer_id, expert_id)

    def demote_to_cpu(self, layer_id: int, expert_id: int) -> bool:
        """Drop the GPU copy, keeping the CPU backing copy."""
        key = (layer_id, expert_id)
        entry = self._gpu_cache.pop(key, None)
        if entry is None:
            return False
        if self.policy == EvictionPolicy.ARC:
            self._arc_gpu.remove(key)
        self._epoch += 1
        self._sync_slots()
        return True

    def get_size_bytes(self, layer_id: int, expert_id: int) -> int:
        key = (layer_id, expert_id)
        entry = self._gpu_cache.get(key) or self._cpu_cache.get(key)
        if entry is None:
            raise KeyError(f"Expert not present in cache: layer={layer_id}, expert={expert_id}")
        return entry.size_bytes

    def stats(self) -> CacheStats:
        return self._stats

    def is_gpu_resident(self, layer_id: int, expert_id: int) -> bool:
        return (layer_id, expert_id) in self._gpu_cache

    def peek_cpu(self, layer_id: int, expert_id: int) -> Optional[Any]:
        entry = self._cpu_cache.get((layer_id, expert_id))
        return None if entry is None else entry.expert

    def peek_gpu(self, layer_id: int, expert_id: int) -> Optional[Any]:
        entry = self._gpu_cache.get((layer_id, expert_id))
        return None if entry is None else entry.expert

    def __repr__(self) -> str:
        return (f"CacheManager(gpu={len(self._gpu_cache)}/{self.gpu_slots}, "
                f"cpu={len(self._cpu_cache)}/{self.cpu_slots}, policy={self.policy.value})")
