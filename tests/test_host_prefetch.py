"""PrefetchEngine scheduling and bookkeeping (the behaviours tests/test_engine.py:118-380 of
the reference checks), with a scheduler double: no GPU needed."""
from __future__ import annotations

import types

import torch

from moeinfra_amd.cache.manager import CacheManager
from moeinfra_amd.cache.types import EvictionPolicy
from moeinfra_amd.engine.prefetch import PrefetchEngine
from moeinfra_amd.engine.types import ForwardRequest, ForwardResult, PrefetchPolicy
from moeinfra_amd.transfer.types import TransferStatus


class FakeScheduler:
    def __init__(self, status=TransferStatus.IN_FLIGHT):
        self.submitted, self.cancelled, self.polled = [], [], []
        self.status = status

    def submit_async(self, request):
        self.submitted.append(request)
        return types.SimpleNamespace(request_id=request.request_id, layer_id=request.layer_id,
                                     expert_id=request.expert_id, status=self.status)

    def cancel(self, request_id):
        self.cancelled.append(request_id)
        return True

    def poll_async(self, layer_id, expert_id):
        self.polled.append((layer_id, expert_id))
        return TransferStatus.READY


def _engine(policy, depth=1, scheduler=None, cm=None):
    cm = cm or CacheManager(gpu_slots=4, cpu_slots=16, policy=EvictionPolicy.LRU)
    sch = scheduler or FakeScheduler()
    return PrefetchEngine(cm, sch, policy, depth), sch, cm


def test_none_policy_is_a_no_op():
    eng, sch, _ = _engine(PrefetchPolicy.NONE)
    assert eng.schedule_prefetch(0, torch.tensor([[0, 1]])) == []
    assert sch.submitted == []


def test_next_layer_one_request_per_distinct_expert():
    eng, sch, _ = _engine(PrefetchPolicy.NEXT_LAYER)
    out = eng.schedule_prefetch(5, torch.tensor([[0, 1], [2, 3], [1, 2]]))
    assert len(out) == 4
    assert {(r.layer_id, r.expert_id) for r in sch.submitted} == {(6, 0), (6, 1), (6, 2), (6, 3)}
    assert all(r.priority.name == "LOW" for r in sch.submitted)


def test_lookahead_targets_each_layer_up_to_depth():
    eng, sch, _ = _engine(PrefetchPolicy.LOOKAHEAD, depth=2)
    out = eng.schedule_prefetch(0, torch.tensor([[0, 1]]))
    assert len(out) == 4
    assert {(r.layer_id, r.expert_id) for r in sch.submitted} == {(1, 0), (1, 1), (2, 0), (2, 1)}


def test_duplicates_are_not_resubmitted():
    eng, sch, _ = _engine(PrefetchPolicy.NEXT_LAYER)
    assert len(eng.schedule_prefetch(3, torch.tensor([[0, 1]]))) == 2
    assert eng.schedule_prefetch(3, torch.tensor([[0, 1]])) == []
    assert len(sch.submitted) == 2


def test_gpu_resident_experts_are_skipped():
    eng, sch, cm = _engine(PrefetchPolicy.NEXT_LAYER)
    cm.put(6, 0, types.SimpleNamespace(device=torch.device("cpu"), size_bytes=1), device="cuda:0")
    out = eng.schedule_prefetch(5, torch.tensor([[0, 1]]))
    assert len(out) == 1
    assert (sch.submitted[0].layer_id, sch.submitted[0].expert_id) == (6, 1)


def test_rejected_submission_is_not_tracked():
    eng, sch, _ = _engine(PrefetchPolicy.NEXT_LAYER, scheduler=FakeScheduler(TransferStatus.REJECTED))
    assert eng.schedule_prefetch(0, torch.tensor([[0, 1]])) == []
    assert eng.cancel_stale(current_layer=10) == 0


def test_cancel_stale_past_layers_only():
    eng, sch, _ = _engine(PrefetchPolicy.LOOKAHEAD, depth=3)
    eng.schedule_prefetch(0, torch.tensor([[0, 1]]))            # layers 1, 2, 3
    assert eng.cancel_stale(current_layer=2) == 2                # layer 1's two requests
    assert len(sch.cancelled) == 2
    assert eng.cancel_stale(current_layer=2) == 0


def test_on_layer_complete_keeps_useful_work():
    eng, sch, _ = _engine(PrefetchPolicy.NEXT_LAYER)
    eng.schedule_prefetch(0, torch.tensor([[0, 1]]))
    eng.on_layer_complete(0, torch.tensor([[0, 1]]))             # layer 1 still ahead
    assert len(sch.submitted) == 2 and sch.cancelled == []
    eng.on_layer_complete(1, torch.tensor([[2, 3]]))             # layer 1 is now stale
    assert len(sch.cancelled) == 2
    assert {(r.layer_id, r.expert_id) for r in sch.submitted[2:]} == {(2, 2), (2, 3)}


def test_poll_retires_finished_prefetches():
    eng, sch, _ = _engine(PrefetchPolicy.NEXT_LAYER)
    eng.schedule_prefetch(0, torch.tensor([[4, 5]]))
    eng.poll()
    assert set(sch.polled) == {(1, 4), (1, 5)}
    assert eng.cancel_stale(current_layer=10) == 0               # nothing left in flight


def test_request_and_result_types():
    req = ForwardRequest(input_ids=torch.zeros((1, 4), dtype=torch.long))
    assert req.max_new_tokens == 128 and req.attention_mask is None
    res = ForwardResult(logits=torch.zeros(1), token_ids=[1, 2], ttft_ms=1.0, tps=2.0,
                        stage_timings={"prefill": 1.0})
    assert res.token_ids == [1, 2]
    assert [p.value for p in PrefetchPolicy] == ["none", "next_layer", "lookahead", "next_router"]


class PrefixScheduler(FakeScheduler):
    """Scheduler double for bounded prefixes: refuses expert 7, and a prefix counts as
    consumed once `consume` names it (the expert's transfer completed it)."""

    def __init__(self):
        super().__init__()
        self.prefixes = {}

    def start_prefix(self, layer_id, expert_id, nbytes):
        if expert_id == 7 or (layer_id, expert_id) in self.prefixes:
            return False
        self.prefixes[(layer_id, expert_id)] = nbytes
        return True

    def consume(self, layer_id, expert_id):
        self.prefixes.pop((layer_id, expert_id))

    def drop_prefix(self, layer_id, expert_id):
        return self.prefixes.pop((layer_id, expert_id), None) is not None


def test_prefix_prefetch_bookkeeping():
    eng, sch, _ = _engine(PrefetchPolicy.NEXT_ROUTER, scheduler=PrefixScheduler())
    assert eng.prefetch_prefix(3, [5, 1, 5, 7], 1 << 20) == [1, 5]   # ascending, once, 7 refused
    assert sch.prefixes == {(3, 1): 1 << 20, (3, 5): 1 << 20} and sch.submitted == []
    assert eng.prefetch_prefix(3, [1], 1 << 20) == []                # already started
    sch.consume(3, 5)                                                 # layer 3 routed to 5
    eng.cancel_stale(current_layer=3)                                 # layer 3 not passed yet
    assert eng.counts["prefixes_used"] == 0 and (3, 1) in sch.prefixes
    eng.cancel_stale(current_layer=4)
    assert eng.counts == {"started": 0, "refused": 0, "cancelled": 0, "prefixes": 2,
                          "prefixes_used": 1, "prefixes_dropped": 1}
    assert sch.prefixes == {}                                         # the unused slot is back
