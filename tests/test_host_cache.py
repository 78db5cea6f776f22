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
    p0 = c._rank[False].p
    c.put(0, 0, Fake(), "cpu")                 # ghost hit grows T1's target
    assert c._rank[False].p > p0
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


def _decode_trace(layers, experts, tokens, seed=0, k=2):
    """(layer, expert) GPU-tier accesses of layer-by-layer decoding with random top-k
    routing: every token visits layers 0..L-1 in order."""
    import random

    rng = random.Random(seed)
    return [(l, e) for _ in range(tokens) for l in range(layers)
            for e in sorted(rng.sample(range(experts), k))]


def _hits(c, trace):
    hits = 0
    for key in trace:
        if c.is_gpu_resident(*key):
            hits += 1
            c.get(*key)
        else:
            c.put(*key, Fake(device="cuda"), "cuda")
    return hits


def test_global_lru_never_hits_a_cyclic_decode_while_a_per_layer_tier_does():
    """Layer-by-layer decoding visits (layer, expert) keys cyclically.  A global LRU tier
    with fewer slots (12) than one token's keys (8 layers x 2 routed) has flushed every key
    before its layer comes round again: no hit at all.  One slot per layer (8 of the 12
    used) keeps each layer's last expert, which the next token's first routed expert
    sometimes is."""
    trace = _decode_trace(layers=8, experts=8, tokens=400)
    glob = CacheManager(gpu_slots=12, cpu_slots=64, policy=EvictionPolicy.LRU)
    part = CacheManager(gpu_slots=12, cpu_slots=64, policy=EvictionPolicy.LRU,
                        gpu_slots_per_layer=1)
    assert _hits(glob, trace) == 0
    rate = _hits(part, trace) / len(trace)
    assert rate > 0.02, rate
    assert part.stats().gpu_slots_used == 8
    assert all(sum(1 for k in part._gpu_cache if k[0] == l) == 1 for l in range(8))


def test_per_layer_partition_evicts_within_the_layer():
    c = CacheManager(gpu_slots=6, cpu_slots=8, policy=EvictionPolicy.LRU, gpu_slots_per_layer=2)
    for key in ((0, 0), (1, 0), (0, 1), (1, 1)):
        c.put(*key, Fake(device="cuda"), "cuda")
    c.get(0, 0)
    c.put(0, 2, Fake(device="cuda"), "cuda")   # layer 0 is full: its LRU entry (0, 1) goes
    assert set(c._gpu_cache) == {(0, 0), (0, 2), (1, 0), (1, 1)}
    with pytest.raises(ValueError):
        CacheManager(gpu_slots=1, cpu_slots=1, policy=EvictionPolicy.LRU, gpu_slots_per_layer=0)


@pytest.mark.parametrize("policy", list(EvictionPolicy))
def test_make_room_evicts_ahead_of_the_put(policy):
    c = CacheManager(gpu_slots=2, cpu_slots=4, policy=policy)
    c.put(0, 0, Fake(device="cuda"), "cuda")
    c.put(0, 1, Fake(device="cuda"), "cuda")
    c.make_room_gpu(0, 1)                      # already resident: nothing to do
    assert c.stats().evictions == 0
    c.make_room_gpu(0, 2)
    assert c.stats().gpu_slots_used == 1 and c.stats().evictions == 1
    c.put(0, 2, Fake(device="cuda"), "cuda")   # fits without another eviction
    assert c.stats().evictions == 1 and c.is_gpu_resident(0, 2)


def test_arc_matches_the_paper_on_a_small_trace():
    """ARC with capacity 2: a key seen twice moves to T2; a miss on a T1 ghost raises p and
    re-enters in T2; with T1 under its target the victim comes from T2."""
    c = cm(EvictionPolicy.ARC, cpu=2)
    arc = c._rank[False]
    c.put(0, 0, Fake(), "cpu")
    c.get(0, 0)                                # (0,0) -> T2
    c.put(0, 1, Fake(), "cpu")                 # T1 = [(0,1)], T2 = [(0,0)]
    assert list(arc.t1) == [(0, 1)] and list(arc.t2) == [(0, 0)]
    c.put(0, 2, Fake(), "cpu")                 # |T1| = 1 > p = 0: T1's LRU (0,1) -> B1
    assert list(arc.b1) == [(0, 1)] and c.peek_cpu(0, 0) is not None
    c.put(0, 1, Fake(), "cpu")                 # B1 ghost hit: p -> 1, victim from T2? |T1|=1==p
    assert arc.p == 1 and (0, 1) in arc.t2
    assert c.stats().cpu_slots_used == 2
