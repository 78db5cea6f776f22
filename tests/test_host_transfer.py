"""Transfer path host logic (transfer/*.py of the reference) -- CPU only.

PinnedMemoryBudget and the staging pool's slot accounting (tests/test_pinned_memory.py,
tests/test_reusable_staging.py of the reference), BandwidthMonitor and the
TransferScheduler queue (tests/test_transfer.py) with a fake cache manager.  Pinned
buffers and H2D copies need a GPU and are covered by the GPU tests.
"""
from __future__ import annotations

import itertools
import time
import types

import numpy as np
import pytest
import torch

from moeinfra_amd.transfer.bandwidth import BandwidthMonitor
from moeinfra_amd.transfer.pinned_memory import PinnedMemoryBudget
from moeinfra_amd.transfer.reusable_staging import ReusablePinnedStagingPool
from moeinfra_amd.transfer.scheduler import EXECUTE_NEXT_PROFILE, TransferScheduler
from moeinfra_amd.transfer.types import (TransferDirection, TransferPriority, TransferRequest,
                                         TransferResult)

_ids = itertools.count()


def req(layer=0, expert=0, direction=TransferDirection.CPU_TO_GPU,
        priority=TransferPriority.NORMAL, rid=None, issued=None):
    return TransferRequest(request_id=rid or f"r{next(_ids)}", layer_id=layer, expert_id=expert,
                           direction=direction, priority=priority,
                           issued_at=time.monotonic() if issued is None else issued)


class FakeCM:
    def __init__(self):
        self.gpu, self.cpu, self.demoted = {}, {}, []

    def get_size_bytes(self, layer, expert):
        key = (layer, expert)
        if key in self.gpu:
            return self.gpu[key]
        if key in self.cpu:
            return self.cpu[key]
        raise KeyError(f"Expert not present in cache: layer={layer}, expert={expert}")

    def demote_to_cpu(self, layer, expert):
        self.demoted.append((layer, expert))
        return self.gpu.pop((layer, expert), None) is not None

    def is_gpu_resident(self, layer, expert):
        return (layer, expert) in self.gpu

    def peek_gpu(self, layer, expert):
        return None

    def peek_cpu(self, layer, expert):
        return self.cpu_objs.get((layer, expert)) if hasattr(self, "cpu_objs") else None


# --------------------------------------------------------------------------- budget
def test_budget_accounting():
    b = PinnedMemoryBudget(100)
    assert (b.budget_bytes, b.used_bytes, b.available_bytes) == (100, 0, 100)
    assert b.reserve(60) and b.reserve(40) and b.available_bytes == 0
    assert not b.reserve(1) and b.used_bytes == 100
    assert b.can_reserve(0) and b.reserve(0)
    b.release(30)
    assert b.can_reserve(30) and not b.can_reserve(31) and b.used_bytes == 70
    with pytest.raises(ValueError, match="underflow"):
        b.release(71)
    for bad in (lambda: b.reserve(-1), lambda: b.can_reserve(-5), lambda: b.release(-1),
                lambda: PinnedMemoryBudget(-1)):
        with pytest.raises(ValueError):
            bad()
    assert "used_bytes=70" in repr(b)


# --------------------------------------------------------------------------- staging slots
class Event:
    def __init__(self, done):
        self.done = done

    def query(self):
        return self.done


def test_staging_pool_slot_lifecycle():
    b = PinnedMemoryBudget(300)
    pool = ReusablePinnedStagingPool(b, 100)
    assert pool.slot_count == 0 and pool.active_slots == 0
    s0, s1, s2 = pool.acquire(), pool.acquire(), pool.acquire()
    assert [s.slot_id for s in (s0, s1, s2)] == [0, 1, 2] and b.used_bytes == 300
    assert pool.acquire() is None                           # budget exhausted
    pool.release(s1)
    assert pool.acquire() is s1 and pool.slot_count == 3    # reused, not reallocated
    pool.release(s1)
    with pytest.raises(RuntimeError):
        pool.release(s1)
    s1.ready_event = Event(False)                           # its DMA is still running
    assert pool.acquire() is None
    s1.ready_event = Event(True)
    assert pool.acquire() is s1 and s1.ready_event is None
    pool.release(s0)
    with pytest.raises(RuntimeError):
        pool.mark_transfer_complete(s0, None)
    with pytest.raises(ValueError):
        ReusablePinnedStagingPool(b, 0)
    pool.destroy()
    assert pool.slot_count == 0 and b.used_bytes == 0


def _serialized_projection(rows, cols, seed):
    from oracle import moe_oracle as orc
    from moeinfra_amd.model.expert import NF4QuantState

    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(rows * cols, generator=g) * 0.02).to(torch.bfloat16)
    packed, absmax = orc.nf4_quantize(w.view(torch.int16).numpy().view(np.uint16))
    qs = NF4QuantState(absmax=torch.from_numpy(absmax), code=torch.from_numpy(orc.NF4_CODE.copy()),
                       shape=torch.Size((rows, cols)))
    return {"weight": torch.from_numpy(packed).reshape(-1, 1), "weight.absmax": qs.absmax,
            "weight.quant_map": qs.code, "weight.quant_state.bitsandbytes__nf4": qs.blob()}


def test_staging_canonical_state_from_serialized_keys():
    from moeinfra_amd.model.expert import PrequantizedNF4Expert, parse_blob

    H, F = 64, 128
    ex = PrequantizedNF4Expert.from_serialized(_serialized_projection(F, H, 1),
                                               _serialized_projection(H, F, 2),
                                               _serialized_projection(F, H, 3), H, F)
    st = ReusablePinnedStagingPool._projection_state(ex, "w2")
    assert set(st) == {"weight", "absmax", "code", "offset"} and st["offset"] is None
    assert st["weight"] is ex.w2["weight"] and st["code"].shape == (16,)
    meta = parse_blob(ex.w1["weight.quant_state.bitsandbytes__nf4"])
    assert meta == {"quant_type": "nf4", "blocksize": 64, "dtype": "bfloat16", "shape": [F, H]}
    want = sum(t.numel() * t.element_size() for p in (ex.w1, ex.w2, ex.w3)
               for k, t in p.items() if not k.endswith("nf4"))
    assert ReusablePinnedStagingPool._expert_staging_size(ex) == want
    bad = dict(ex.w1)
    del bad["weight.absmax"]
    with pytest.raises(ValueError, match="weight.absmax"):
        PrequantizedNF4Expert.from_serialized(bad, ex.w2, ex.w3, H, F)
    with pytest.raises(ValueError, match="missing serialized"):
        ReusablePinnedStagingPool._projection_state(types.SimpleNamespace(w1=bad), "w1")
    with pytest.raises(TypeError):
        ReusablePinnedStagingPool._projection_state(types.SimpleNamespace(w1=3), "w1")


def test_parse_blob_tolerates_garbage():
    from moeinfra_amd.model.expert import parse_blob

    assert parse_blob(None) == {}
    assert parse_blob(torch.tensor([0xFF, 0xFE], dtype=torch.uint8)) == {}
    assert parse_blob(torch.tensor(list(b"[1,2]"), dtype=torch.uint8)) == {}


# --------------------------------------------------------------------------- bandwidth
def test_bandwidth_monitor():
    m = BandwidthMonitor(window_s=5.0)
    assert m.current_gbps() == 0.0 and m.peak_gbps() == 0.0
    m.record(1 << 30, now=100.0)
    assert m.current_gbps(now=100.0) == 0.0                 # one sample: no rate yet
    m.record(1 << 30, now=100.5)
    assert m.current_gbps(now=101.0) == pytest.approx(2.0)  # 2 GiB over 1 s
    assert m.peak_gbps() == pytest.approx(4.0)              # 2 GiB over 0.5 s at the record
    assert m.current_gbps(now=200.0) == 0.0                 # both samples left the window
    m.reset()
    assert m.peak_gbps() == 0.0 and m.bytes_in_window() == 0
    with pytest.raises(ValueError):
        BandwidthMonitor(0)


def test_bandwidth_monitor_wall_clock():
    """The reference's own checks (tests/test_transfer.py:152-190): two samples a moment
    apart give a positive rate, the peak stays at or above it, reset clears both."""
    m = BandwidthMonitor(window_s=5.0)
    m.record(1 << 30)
    time.sleep(0.01)
    m.record(1 << 30)
    assert m.current_gbps() > 0.0 and m.peak_gbps() >= m.current_gbps()
    m.reset()
    assert m.current_gbps() == 0.0 and m.peak_gbps() == 0.0


# --------------------------------------------------------------------------- scheduler
def sched(cm=None, **kw):
    cm = cm or FakeCM()
    return TransferScheduler(cm, bandwidth_gbps=24.0, max_concurrent=4, **kw), cm


def test_request_and_result_types():
    r = req(3, 7)
    with pytest.raises((AttributeError, TypeError)):
        r.layer_id = 1
    assert not hasattr(r, "tensor") and req().request_id != req().request_id
    res = TransferResult("x", False, 1.0, 0, "boom")
    assert (res.success, res.bytes_transferred, res.error) == (False, 0, "boom")
    with pytest.raises(ValueError):
        TransferScheduler(FakeCM(), 1.0, 0)


def test_submit_dedup():
    s, _ = sched()
    a = req(0, 1)
    assert s.submit(a) and s.pending_count() == 1
    assert not s.submit(req(0, 1))                          # same (layer, expert, direction)
    assert not s.submit(req(2, 2, rid=a.request_id))        # same id
    assert s.submit(req(0, 1, TransferDirection.GPU_TO_CPU))
    assert s.submit(req(0, 2)) and s.pending_count() == 3
    assert "pending=3" in repr(s)


def test_priority_then_fifo_order():
    s, cm = sched()
    t = time.monotonic()
    order = [req(0, 0, TransferDirection.GPU_TO_CPU, TransferPriority.LOW, issued=t),
             req(0, 1, TransferDirection.GPU_TO_CPU, TransferPriority.NORMAL, issued=t + 1),
             req(0, 2, TransferDirection.GPU_TO_CPU, TransferPriority.HIGH, issued=t + 2),
             req(0, 3, TransferDirection.GPU_TO_CPU, TransferPriority.NORMAL, issued=t + 3)]
    for r in order:
        cm.gpu[(0, r.expert_id)] = 10
        s.submit(r)
    results = s.drain()
    assert [r.request_id for r in results] == [order[i].request_id for i in (2, 1, 3, 0)]
    assert cm.demoted == [(0, 2), (0, 1), (0, 3), (0, 0)]
    assert all(r.success and r.bytes_transferred == 10 and r.elapsed_ms > 0 for r in results)
    assert s.pending_count() == 0 and s.execute_next() is None and s.drain() == []
    assert s.bandwidth_monitor.bytes_in_window() == 40


def test_cancel_keeps_heap_order():
    s, cm = sched()
    t = time.monotonic()
    rs = [req(0, i, TransferDirection.GPU_TO_CPU, TransferPriority(i % 3), issued=t + i)
          for i in range(7)]
    for r in rs:
        cm.gpu[(0, r.expert_id)] = 1
        s.submit(r)
    assert s.cancel(rs[3].request_id) and not s.cancel(rs[3].request_id)
    assert not s.cancel("nope") and s.pending_count() == 6
    got = [r.request_id for r in s.drain()]
    want = [r.request_id for r in sorted((r for r in rs if r is not rs[3]),
                                         key=lambda r: (r.priority.value, r.issued_at))]
    assert got == want


def test_failures_are_reported_in_the_result():
    s, cm = sched()
    s.submit(req(5, 5, TransferDirection.GPU_TO_CPU))       # not in the cache at all
    r = s.execute_next()
    assert not r.success and r.bytes_transferred == 0 and "layer=5" in r.error
    cm.cpu[(1, 1)] = 99
    s.submit(req(1, 1, TransferDirection.GPU_TO_CPU))       # present but not GPU-resident
    r = s.execute_next()
    assert not r.success and "Transfer failed" in r.error
    s.submit(req(1, 1, TransferDirection.CPU_TO_GPU))       # sized, but no CPU copy
    r = s.execute_next()
    assert not r.success and "CPU expert not found" in r.error
    cm.cpu_objs = {(1, 2): object()}
    cm.cpu[(1, 2)] = 99
    s.submit(req(1, 2, TransferDirection.CPU_TO_GPU))       # a CPU copy, but no stream
    r = s.execute_next()
    assert not r.success and "transfer_stream" in r.error
    assert EXECUTE_NEXT_PROFILE[-1]["success"] is False
    assert s.pending_count() == 0


def test_submit_async_rejections_without_gpu():
    s, cm = sched()
    with pytest.raises(ValueError):
        s.submit_async(req(0, 0, TransferDirection.GPU_TO_CPU))
    cm.gpu[(0, 0)] = 1
    assert s.submit_async(req(0, 0)).status.value == "ready"
    assert s.submit_async(req(0, 1)).status.value == "rejected"   # no CPU copy to send
    cm.cpu_objs = {(0, 1): object()}
    with pytest.raises(RuntimeError, match="transfer_stream"):
        s.submit_async(req(0, 1))
    assert s.poll_async(0, 1).value == "rejected"
