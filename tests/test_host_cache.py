"""CacheManager (cache/manager.py:122-508 of the reference) -- host logic, CPU only.

Mirrors the behaviours the reference's tests/test_cache.py checks (slot accounting,
LRU / LFU order, the "gpu" alias, statistics, promote/demote under the two-copy model)
and adds ARC and the residency epoch.
"""
from __future__ import annotations

import time
import types

import pytest

from moeinfra_amd.cache.manager import CacheManager
from moeinfra_amd.cache.types import CacheEntry, CacheStats, EvictionPolicy


class Fake:
    def __init__(self, size_bytes=1024, device="cpu"):
        self.size_bytes = size_bytes
        self.device = types.SimpleNamespace(type=device.split(":")[0])


def cm(policy=EvictionPolicy.LRU, gpu=2, cpu=4):
    return CacheManager(gpu_slots=gpu, cpu_slots=cpu, policy=policy)


def test_init_and_repr():
    c = cm(EvictionPolicy.LFU)
    assert (c.gpu_slots, c.cpu_slots, c.policy) == (2, 4, EvictionPolicy.LFU)
    assert "gpu=0/2" in repr(c) and "cpu=0/4" in repr(c) and "lfu" in repr(c)
    s = c.stats()
    assert (s.hits, s.misses, s.evictions, s.gpu_slots_used, s.cpu_slots_used) == (0,) * 5
    assert s.hit_rate == 0.0 and c.stats() is s


def test_entry_and_stats_types():
    e = CacheEntry(1, 2, "cuda:0", None, time.monotonic() - 0.05, 1, 8)
    assert e.is_on_gpu and not CacheEntry(1, 2, "cpu", None, 0.0, 1, 8).is_on_gpu
    assert e.age >= 0.05
    assert CacheStats(hits=3, misses=1).hit_rate == pytest.approx(0.75)
    assert CacheStats(hits=5).hit_rate == 1.0


def test_put_get_refresh_and_counters():
    c = cm()
    a, b = Fake(), Fake()
    c.put(0, 0, a, "cpu")
    assert c.get(0, 0) is a and c.stats().hits == 1
    assert c.get(0, 1) is None and c.stats().misses == 1
    c.put(0, 0, b, "cpu")
    assert c.stats().cpu_slots_used == 1 and c.get(0, 0) is b
    g = Fake(device="cuda")
    c.put(0, 0, g, "cuda:0")
    assert c.get(0, 0) is g                    # GPU tier first
    assert c.stats().gpu_slots_used == 1 and c.peek_cpu(0, 0) is b


def test_lru_order_and_auto_eviction():
    c = cm(cpu=3)
    for i in range(3):
        c.put(0, i, Fake(), "cpu")
        time.sleep(0.002)
    c.get(0, 0)
    c.put(0, 3, Fake(), "cpu")                 # evicts expert 1, the least recently used
    assert c.peek_cpu(0, 1) is None and c.peek_cpu(0, 0) is not None
    assert c.stats().cpu_slots_used == 3 and c.stats().evictions == 1
    for i in range(4, 8):
        c.put(0, i, Fake(), "cpu")
    assert c.stats().cpu_slots_used == 3 and c.stats().evictions == 5


def test_lfu_order_with_lru_tiebreak():
    c = cm(EvictionPolicy.LFU, cpu=3)
    for i in range(3):
        c.put(0, i, Fake(), "cpu")
        time.sleep(0.002)
    c.get(0, 0)
    c.get(0, 0)
    c.get(0, 2)
    assert c.evict("cpu").expert_id == 1       # fewest accesses
    c.get(0, 0)
    assert c.evict("cpu").expert_id == 2


def test_arc_keeps_frequent_entries_under_a_scan():
    c = cm(EvictionPolicy.ARC, cpu=4)
    for i in range(2):                         # the working set, seen twice -> T2
        c.put(0, i, Fake(), "cpu")
        c.get(0, i)
    for i in range(10, 30):                    # a one-pass scan through T1
        c.put(0, i, Fake(), "cpu")
    assert c.peek_cpu(0, 0) is not None and c.peek_cpu(0, 1) is not None
    assert c.stats().cpu_slots_used == 4


def test_arc_ghost_hit_adapts_target():
    c = cm(EvictionPolicy.ARC, cpu=2)
    c.put(0, 0, Fake(), "cpu")
    c.put(0, 1, Fake(), "cpu")
    c.put(0, 2, Fake(), "cpu")                 # evicts 0 into the T1 ghost list
    assert c.peek_cpu(0, 0) is None
    p0 = c._arc_cpu.p
    c.put(0, 0, Fake(), "cpu")                 # ghost hit grows T1's target
    assert c._arc_cpu.p > p0
    assert c.stats().cpu_slots_used == 2


@pytest.mark.parametrize("policy", list(EvictionPolicy))
def test_evict_empty_and_gpu_alias(policy):
    c = CacheManager(gpu_slots=1, cpu_slots=1, policy=policy)
    assert c.evict("cpu") is None and c.evict("gpu") is None
    cpu_e, gpu_e = Fake(123), Fake(123, "cuda")
    c.put(0, 0, cpu_e, "cpu")
    c.put(0, 0, gpu_e, "cuda")
    ev = c.evict("gpu")
    assert ev.expert is gpu_e and c.peek_gpu(0, 0) is None and c.peek_cpu(0, 0) is cpu_e
    ev = c.evict("cpu")
    assert ev.device == "cpu" and c.stats().evictions == 2


def test_get_size_bytes():
    c = cm()
    c.put(1, 2, Fake(4096), "cpu")
    c.put(1, 3, Fake(777, "cuda"), "cuda:0")
    assert c.get_size_bytes(1, 2) == 4096 and c.get_size_bytes(1, 3) == 777
    with pytest.raises(KeyError):
        c.get_size_bytes(9, 9)


def test_promote_reports_residency_and_demote_keeps_cpu_copy():
    c = cm()
    assert c.promote_to_gpu(0, 99) is False
    c.put(0, 0, Fake(), "cpu")
    assert c.promote_to_gpu(0, 0) is False     # residency is the scheduler's job
    c.put(0, 0, Fake(device="cuda"), "cuda")
    assert c.promote_to_gpu(0, 0) is True and c.is_gpu_resident(0, 0)
    assert c.demote_to_cpu(0, 0) is True
    assert not c.is_gpu_resident(0, 0) and c.peek_cpu(0, 0) is not None
    assert c.stats().gpu_slots_used == 0 and c.stats().cpu_slots_used == 1
    assert c.demote_to_cpu(0, 0) is False


def test_residency_epoch_changes_only_with_gpu_tier():
    c = cm(gpu=1)
    e0 = c.residency_epoch
    c.put(0, 0, Fake(), "cpu")
    c.get(0, 0)
    assert c.residency_epoch == e0
    c.put(0, 0, Fake(device="cuda"), "cuda")
    e1 = c.residency_epoch
    assert e1 > e0
    c.put(0, 1, Fake(device="cuda"), "cuda")   # evicts (0, 0) and inserts (0, 1)
    e2 = c.residency_epoch
    assert e2 > e1
    c.demote_to_cpu(0, 1)
    assert c.residency_epoch > e2
