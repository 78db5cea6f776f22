"""Two-tier expert cache: the CacheManager API of the reference's cache/manager.py:122-508
(get / put / evict / promote_to_gpu / demote_to_cpu / get_size_bytes / stats /
is_gpu_resident / peek_cpu / peek_gpu), built around this package's offload path.

* The CPU tier holds the authoritative NF4 experts (in the engine's offload mode, views
  into a store pinned once); the GPU tier holds disposable working copies.  Both are dicts
  keyed by (layer_id, expert_id) -- ``_cpu_cache`` / ``_gpu_cache``, the names the
  reference's tests inspect -- ranked for eviction by one replacement policy per tier.
* Policies are small objects with admit / touch / forget / victim: LRU is an ordered set
  (most recent last); LFU ranks by access count, then by a logical clock; ARC is the
  adaptive replacement cache of Megiddo and Modha ("ARC: A Self-Tuning, Low Overhead
  Replacement Cache", FAST 2003).
* ``gpu_slots_per_layer`` partitions the GPU tier by layer: a layer's experts then evict
  only each other.  Layer-by-layer decoding visits (layer, expert) keys cyclically, so one
  global recency order over a tier smaller than the store evicts every expert before its
  layer comes round again; per layer, a tier keeps each layer's recent experts.
* ``residency_epoch`` changes whenever the GPU tier changes, so callers can cache derived
  state (device pointer tables) per epoch.

Single-threaded, like the reference (cache/manager.py:21-22).
"""
from __future__ import annotations

import itertools
import logging
import time
from collections import OrderedDict
from typing import Any, Iterable, Optional

from .types import CacheEntry, CacheStats, EvictionPolicy

Key = tuple[int, int]


def _is_gpu(device: str) -> bool:
    """Device-string convention of the reference (cache/manager.py:177-190): "cuda",
    "cuda:N" and "gpu" name the GPU tier, anything else the CPU tier."""
    return device.startswith(("cuda", "gpu"))


# ------------------------------------------------------------------------- policies
class _LRU:
    """Least recently used first: an ordered set, most recent at the end."""

    def __init__(self, capacity: int) -> None:
        self._order: OrderedDict[Key, None] = OrderedDict()

    def admit(self, key: Key) -> None:
        self._order[key] = None
        self._order.move_to_end(key)

    def touch(self, key: Key) -> None:
        if key in self._order:
            self._order.move_to_end(key)

    def forget(self, key: Key) -> None:
        self._order.pop(key, None)

    def victim(self, allowed: Optional[set], incoming: Optional[Key]) -> Optional[Key]:
        for key in self._order:
            if allowed is None or key in allowed:
                return key
        return None

    def evicted(self, key: Key) -> None:
        self.forget(key)


class _LFU:
    """Fewest accesses first; equal counts go least recently used first."""

    def __init__(self, capacity: int) -> None:
        self._rank: dict[Key, tuple[int, int]] = {}
        self._clock = itertools.count()

    def admit(self, key: Key) -> None:
        self._rank[key] = (1, next(self._clock))

    def touch(self, key: Key) -> None:
        if key in self._rank:
            self._rank[key] = (self._rank[key][0] + 1, next(self._clock))

    def forget(self, key: Key) -> None:
        self._rank.pop(key, None)

    def victim(self, allowed: Optional[set], incoming: Optional[Key]) -> Optional[Key]:
        keys = self._rank if allowed is None else [k for k in self._rank if k in allowed]
        return min(keys, key=self._rank.__getitem__, default=None)

    def evicted(self, key: Key) -> None:
        self.forget(key)


class _ARC:
    """Adaptive replacement (Megiddo & Modha, FAST 2003).  Live keys sit in T1 (seen once
    since entering) or T2 (seen again); B1 / B2 remember keys evicted from T1 / T2.  A miss
    on a B1 ghost means T1 was too small, so its target size p grows by max(1, |B2|/|B1|);
    a B2 ghost shrinks it by max(1, |B1|/|B2|); ghosts re-enter in T2.  The victim comes
    from T1 when |T1| exceeds p (or equals it and the incoming key is a B2 ghost), else
    from T2; each ghost list keeps at most `capacity` keys."""

    def __init__(self, capacity: int) -> None:
        self.capacity = max(1, int(capacity))
        self.p = 0
        self.t1: OrderedDict[Key, None] = OrderedDict()
        self.t2: OrderedDict[Key, None] = OrderedDict()
        self.b1: OrderedDict[Key, None] = OrderedDict()
        self.b2: OrderedDict[Key, None] = OrderedDict()

    def _target(self, key: Optional[Key]) -> int:
        if key in self.b1:
            return min(self.capacity, self.p + max(1, len(self.b2) // max(1, len(self.b1))))
        if key in self.b2:
            return max(0, self.p - max(1, len(self.b1) // max(1, len(self.b2))))
        return self.p

    def admit(self, key: Key) -> None:
        self.p = self._target(key)
        if key in self.b1 or key in self.b2:
            self.b1.pop(key, None)
            self.b2.pop(key, None)
            self.t2[key] = None
        else:
            self.t1[key] = None

    def touch(self, key: Key) -> None:
        if key in self.t1:
            del self.t1[key]
            self.t2[key] = None
        elif key in self.t2:
            self.t2.move_to_end(key)

    def forget(self, key: Key) -> None:
        for lst in (self.t1, self.t2, self.b1, self.b2):
            lst.pop(key, None)

    def victim(self, allowed: Optional[set], incoming: Optional[Key]) -> Optional[Key]:
        ok = (lambda k: True) if allowed is None else (lambda k: k in allowed)
        t1 = [k for k in self.t1 if ok(k)]
        t2 = [k for k in self.t2 if ok(k)]
        p = self._target(incoming)
        from_t1 = bool(t1) and (not t2 or len(self.t1) > p or
                                (incoming in self.b2 and len(self.t1) == p))
        return (t1 if from_t1 else t2)[0] if (t1 or t2) else None

    def evicted(self, key: Key) -> None:
        if key in self.t1:
            del self.t1[key]
            self.b1[key] = None
        elif key in self.t2:
            del self.t2[key]
            self.b2[key] = None
        for ghosts in (self.b1, self.b2):
            while len(ghosts) > self.capacity:
                ghosts.popitem(last=False)


_POLICIES = {EvictionPolicy.LRU: _LRU, EvictionPolicy.LFU: _LFU, EvictionPolicy.ARC: _ARC}


# ------------------------------------------------------------------------- manager
class CacheManager:
    """Two-level (GPU working copies, CPU authoritative copies) expert cache."""

    def __init__(self, gpu_slots: int, cpu_slots: int, policy: EvictionPolicy,
                 logger: Optional[logging.Logger] = None,
                 gpu_slots_per_layer: Optional[int] = None) -> None:
        if gpu_slots_per_layer is not None and gpu_slots_per_layer < 1:
            raise ValueError("gpu_slots_per_layer must be positive")
        self.gpu_slots = gpu_slots
        self.cpu_slots = cpu_slots
        self.policy = policy
        self.gpu_slots_per_layer = gpu_slots_per_layer
        self._logger = logger or logging.getLogger(__name__)
        self._gpu_cache: dict[Key, CacheEntry] = {}
        self._cpu_cache: dict[Key, CacheEntry] = {}
        make = _POLICIES[policy]
        self._rank = {True: make(gpu_slots), False: make(cpu_slots)}
        self._stats = CacheStats()
        self._epoch = 0
        self._per_layer: dict[int, int] = {}

    # ---------------------------------------------------------------- internals
    def _tier(self, gpu: bool) -> dict[Key, CacheEntry]:
        return self._gpu_cache if gpu else self._cpu_cache

    def _recount(self) -> None:
        self._stats.gpu_slots_used = len(self._gpu_cache)
        self._stats.cpu_slots_used = len(self._cpu_cache)

    def _touch(self, gpu: bool, key: Key, entry: CacheEntry) -> None:
        entry.last_access = time.monotonic()
        entry.access_count += 1
        self._rank[gpu].touch(key)

    def _remove(self, gpu: bool, key: Key, ghost: bool) -> CacheEntry:
        entry = self._tier(gpu).pop(key)
        if ghost:
            self._rank[gpu].evicted(key)
        else:
            self._rank[gpu].forget(key)
        if gpu:
            self._per_layer[key[0]] -= 1
            self._epoch += 1
        self._recount()
        return entry

    def _evict_one(self, gpu: bool, allowed: Optional[Iterable[Key]],
                   incoming: Optional[Key]) -> Optional[CacheEntry]:
        tier = self._tier(gpu)
        allowed = None if allowed is None else set(allowed)
        pool = tier.keys() if allowed is None else allowed
        if not pool:
            return None
        key = self._rank[gpu].victim(allowed, incoming)
        if key is None or key not in tier:     # a ranking out of step: oldest access
            key = min(pool, key=lambda k: tier[k].last_access)
        entry = self._remove(gpu, key, ghost=True)
        self._stats.evictions += 1
        self._logger.debug("cache: evicted layer=%d expert=%d from the %s tier", key[0], key[1],
                           "GPU" if gpu else "CPU")
        return entry

    def _make_room(self, gpu: bool, incoming: Key) -> None:
        tier = self._tier(gpu)
        if gpu and self.gpu_slots_per_layer is not None and \
                self._per_layer.get(incoming[0], 0) >= self.gpu_slots_per_layer:
            mine = [k for k in tier if k[0] == incoming[0]]
            self._evict_one(True, mine, incoming)
        limit = self.gpu_slots if gpu else self.cpu_slots
        while tier and len(tier) >= limit:
            if self._evict_one(gpu, None, incoming) is None:
                break
        if len(tier) >= limit:
            self._logger.warning("cache: the %s tier is over its %d slots (layer=%d expert=%d)",
                                 "GPU" if gpu else "CPU", limit, incoming[0], incoming[1])

    # ---------------------------------------------------------------- lookup
    def get(self, layer_id: int, expert_id: int) -> Optional[Any]:
        """The GPU copy if there is one, else the CPU copy, else None; counts a hit or miss
        and updates the entry's recency and frequency."""
        key = (layer_id, expert_id)
        for gpu in (True, False):
            entry = self._tier(gpu).get(key)
            if entry is not None:
                self._touch(gpu, key, entry)
                self._stats.hits += 1
                return entry.expert
        self._stats.misses += 1
        return None

    def peek_cpu(self, layer_id: int, expert_id: int) -> Optional[Any]:
        """The CPU copy, without touching statistics or ranking."""
        entry = self._cpu_cache.get((layer_id, expert_id))
        return None if entry is None else entry.expert

    def peek_gpu(self, layer_id: int, expert_id: int) -> Optional[Any]:
        """The GPU copy, without touching statistics or ranking."""
        entry = self._gpu_cache.get((layer_id, expert_id))
        return None if entry is None else entry.expert

    def is_gpu_resident(self, layer_id: int, expert_id: int) -> bool:
        return (layer_id, expert_id) in self._gpu_cache

    def get_size_bytes(self, layer_id: int, expert_id: int) -> int:
        """Bytes of the cached expert (GPU copy first), without touching statistics."""
        key = (layer_id, expert_id)
        entry = self._gpu_cache.get(key) or self._cpu_cache.get(key)
        if entry is None:
            raise KeyError(f"Expert not present in cache: layer={layer_id}, expert={expert_id}")
        return entry.size_bytes

    # ---------------------------------------------------------------- residency changes
    def put(self, layer_id: int, expert_id: int, expert: Any, device: str) -> None:
        """Insert an expert in the tier `device` names, evicting by policy when the tier
        (or, with a per-layer GPU partition, the layer's share) is full.  An existing entry
        is refreshed in place and takes no extra slot."""
        gpu = _is_gpu(device)
        key = (layer_id, expert_id)
        tier = self._tier(gpu)
        entry = tier.get(key)
        if entry is not None:
            if gpu and entry.expert is not expert:
                self._epoch += 1
            entry.expert, entry.device = expert, device
            self._touch(gpu, key, entry)
            return
        self._make_room(gpu, key)
        tier[key] = CacheEntry(expert_id=expert_id, layer_id=layer_id, device=device,
                               expert=expert, last_access=time.monotonic(), access_count=1,
                               size_bytes=expert.size_bytes)
        self._rank[gpu].admit(key)
        if gpu:
            self._per_layer[layer_id] = self._per_layer.get(layer_id, 0) + 1
            self._epoch += 1
        self._recount()

    def make_room_gpu(self, layer_id: int, expert_id: int) -> None:
        """Evict what a later put of (layer_id, expert_id) into the GPU tier would, now --
        so that its device slot is free before the copy into it is issued."""
        if (layer_id, expert_id) not in self._gpu_cache:
            self._make_room(True, (layer_id, expert_id))

    def evict(self, device: str) -> Optional[CacheEntry]:
        """Remove the policy's victim from the tier `device` names; None if it is empty."""
        return self._evict_one(_is_gpu(device), None, None)

    def promote_to_gpu(self, layer_id: int, expert_id: int) -> bool:
        """True if the expert is GPU-resident.  GPU copies are made by the transfer
        scheduler (staged host-to-device copy), never by moving the CPU copy, so a CPU-only
        expert reports False."""
        return self.is_gpu_resident(layer_id, expert_id)

    def demote_to_cpu(self, layer_id: int, expert_id: int) -> bool:
        """Drop the GPU working copy; the CPU copy stays authoritative.  False if there was
        none."""
        key = (layer_id, expert_id)
        if key not in self._gpu_cache:
            return False
        self._remove(True, key, ghost=False)
        return True

    # ---------------------------------------------------------------- reporting
    @property
    def residency_epoch(self) -> int:
        """Changes whenever an expert enters, leaves or is replaced in the GPU tier."""
        return self._epoch

    def stats(self) -> CacheStats:
        return self._stats

    def __repr__(self) -> str:
        return (f"CacheManager(gpu={len(self._gpu_cache)}/{self.gpu_slots}, "
                f"cpu={len(self._cpu_cache)}/{self.cpu_slots}, policy={self.policy.value})")
