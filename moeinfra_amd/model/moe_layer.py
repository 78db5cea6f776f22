"""One Mixtral MoE layer (mirrors model/moe_layer.py:20-237 of the reference).

``_forward_tokens`` keeps the reference's contract -- one routing pass, every routed expert
made GPU-resident, each expert run once on its tokens, weighted ascending-expert combine,
experts that were not resident before the layer demoted afterwards -- and runs it on the
HIP kernels:

* all-resident (every expert of the layer in the GPU tier): one library call routes,
  groups, runs the fused NF4 SwiGLU of every routed expert and combines, without any
  host synchronisation;
* offload: the routing runs on the device, the routed set is read back (the reference's
  ``unique().tolist()``), the copies of every missing routed expert are started at once on
  the transfer stream (``submit_async``; each expert is GPU-resident from then on, ordered
  behind its copy's event), ``_ensure_expert_on_gpu`` returns them (or runs the synchronous
  transfer for one that found no slot), and grouping / expert FFN / combine are enqueued
  behind stream waits on those events -- the host never waits for a copy.  Experts that
  were not resident before the layer are demoted after it, as in the reference
  (model/moe_layer.py:200-209), unless the layer was built with ``retain_transferred`` (the
  engine's offload mode with a per-layer GPU cache keeps them for the next token).

Expert objects that are not NF4 HIP experts (the fakes the reference's tests install by
monkeypatching ``_ensure_expert_on_gpu``) are called one by one, in the reference's order,
on the tokens routed to them.
"""
from __future__ import annotations

import logging
import time
from typing import Optional

import torch

from .. import ops
from ..engine.router import ExpertRouter
from ..transfer.types import TransferDirection, TransferPriority, TransferRequest


def _is_hip_expert(expert) -> bool:
    return hasattr(expert, "c_struct") and hasattr(expert, "intermediate_size")


class MoELayer:
    """Single Mixtral MoE layer with expert offloading."""

    def __init__(self, layer_id: int, router, cache_manager, model_loader, transfer_scheduler,
                 logger: Optional[logging.Logger] = None, *,
                 retain_transferred: bool = False) -> None:
        self.retain_transferred = retain_transferred
        self.layer_id = layer_id
        self.router = router
        self.cache_manager = cache_manager
        self.model_loader = model_loader
        self.transfer_scheduler = transfer_scheduler
        self._logger = logger or logging.getLogger(__name__)
        self._table_key = None
        self._table = None
        self._workspace: Optional[torch.Tensor] = None
        #: The expert indices [T, k] (device int64) of the last forward on the device path.
        self.last_expert_indices: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ residency
    def _ensure_expert_on_gpu(self, expert_id: int):
        """Return an expert that is resident on the GPU (model/moe_layer.py:39-115)."""
        expert = self.cache_manager.get(self.layer_id, expert_id)
        if expert is None:
            self._logger.debug("Expert miss: layer=%d expert=%d", self.layer_id, expert_id)
            expert = self.model_loader.load_expert(self.layer_id, expert_id)
            self.cache_manager.put(self.layer_id, expert_id, expert, device="cpu")
        if expert.device.type == "cuda":
            return expert
        request = TransferRequest(
            request_id=f"layer-{self.layer_id}-expert-{expert_id}-{id(self)}",
            layer_id=self.layer_id, expert_id=expert_id,
            direction=TransferDirection.CPU_TO_GPU, priority=TransferPriority.HIGH,
            issued_at=time.monotonic())
        if not self.transfer_scheduler.submit(request):
            raise RuntimeError(f"Failed to submit transfer for layer={self.layer_id}, "
                               f"expert={expert_id}")
        result = self.transfer_scheduler.execute_next()
        if result is None or not result.success:
            error = result.error if result is not None else "no transfer result"
            raise RuntimeError(f"Failed to transfer expert layer={self.layer_id}, "
                               f"expert={expert_id}: {error}")
        expert = self.cache_manager.get(self.layer_id, expert_id)
        if expert is None or expert.device.type != "cuda":
            raise RuntimeError(f"Expert layer={self.layer_id}, expert={expert_id} "
                               "was not resident on GPU after transfer")
        return expert

    def _start_async_transfers(self, unique: list, was_resident: dict) -> dict:
        """Start the copies of every routed expert that is not GPU-resident, back to back on
        the transfer stream, without waiting for any (submit_async publishes each expert in
        the GPU tier behind its copy's event).  Returns {expert id: the arriving expert} --
        held by the layer, so that an expert the GPU tier evicts again before the layer runs
        (more routed experts than the tier keeps for a layer) stays usable.  Experts that
        find no slot are left to the synchronous path of _ensure_expert_on_gpu."""
        sched = self.transfer_scheduler
        started = {}
        if not hasattr(sched, "submit_async"):
            return started
        for e in unique:
            if was_resident[e] or self.cache_manager.peek_cpu(self.layer_id, e) is None:
                continue
            h = sched.submit_async(TransferRequest(
                request_id=f"layer-{self.layer_id}-expert-{e}-{id(self)}-async",
                layer_id=self.layer_id, expert_id=e, direction=TransferDirection.CPU_TO_GPU,
                priority=TransferPriority.HIGH, issued_at=time.monotonic()))
            if getattr(h, "gpu_state", None) is not None:
                started[e] = h.gpu_state
        return started

    # ------------------------------------------------------------------ forward
    @torch.no_grad()
    def _forward_tokens(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.ndim != 2:
            raise ValueError("hidden_states must have shape (tokens, hidden_size)")
        if hidden_states.shape[-1] != self.router.hidden_size:
            raise ValueError(f"hidden size {hidden_states.shape[-1]} != "
                             f"router hidden size {self.router.hidden_size}")
        if self._device_path_ok(hidden_states):
            return self._forward_device(hidden_states)
        return self._forward_experts(hidden_states)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.ndim == 3:
            b, s, h = hidden_states.shape
            out = self._forward_tokens(hidden_states.reshape(b * s, h))
            return out.reshape(b, s, h)
        if hidden_states.ndim == 2:
            return self._forward_tokens(hidden_states)
        raise ValueError("hidden_states must have shape (tokens, hidden_size) or "
                         "(batch, sequence, hidden_size)")

    __call__ = forward

    # ------------------------------------------------------------------ device path
    def _device_path_ok(self, x: torch.Tensor) -> bool:
        return (isinstance(self.router, ExpertRouter) and x.device.type == "cuda"
                and x.dtype == torch.bfloat16 and self.cache_manager is not None
                and "_ensure_expert_on_gpu" not in self.__dict__)

    def _resident_table(self, experts: list):
        key = (getattr(self.cache_manager, "residency_epoch", None), tuple(map(id, experts)))
        if key[0] is None or key != self._table_key:
            self._table = ops.expert_table([None if e is None else e.c_struct() for e in experts])
            self._table_key = key if key[0] is not None else None
        return self._table

    def _forward_device(self, x: torch.Tensor) -> torch.Tensor:
        router = self.router
        E, k = router.num_experts, router.num_experts_per_tok
        x = x.contiguous()
        resident = [self.cache_manager.peek_gpu(self.layer_id, e) for e in range(E)]
        if all(r is not None and _is_hip_expert(r) for r in resident):
            for r in resident:                 # experts still arriving: order after their copies
                if getattr(r, "ready_event", None) is not None:
                    r.wait_ready()
            table = self._resident_table(resident)
            inter = resident[0].intermediate_size
            need = ops.lib().moe_layer_workspace_bytes(x.shape[0], k, E, x.shape[1], inter)
            if self._workspace is None or self._workspace.numel() < need or \
                    self._workspace.device != x.device:
                self._workspace = torch.empty((need,), dtype=torch.uint8, device=x.device)
            tl = getattr(self.transfer_scheduler, "timeline", None)
            if tl is not None:
                k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                k0.record()
            out, _, _, idx = ops.layer_forward(table, E, router.gate_weight.contiguous(), x, k,
                                               inter, bias=router.bias, workspace=self._workspace)
            if tl is not None:
                k1.record()
                tl.append(("moe", k0, k1, self.layer_id))
            self.last_expert_indices = idx
            return out
        return self._forward_offload(x)

    def _forward_offload(self, x: torch.Tensor) -> torch.Tensor:
        router = self.router
        E, k = router.num_experts, router.num_experts_per_tok
        T = x.shape[0]
        idx32 = torch.empty((T, k), dtype=torch.int32, device=x.device)
        _, w, idx = ops.router_topk(x, router.gate_weight.contiguous(), k, bias=router.bias,
                                    want_logits=False, idx32_out=idx32)
        self.last_expert_indices = idx
        unique = sorted(int(e) for e in idx.reshape(-1).unique().tolist())   # host sync
        was_resident = {e: self.cache_manager.is_gpu_resident(self.layer_id, e) for e in unique}
        experts = {}
        try:
            started = self._start_async_transfers(unique, was_resident)
            for e in unique:
                experts[e] = started[e] if e in started else self._ensure_expert_on_gpu(e)
            if not all(_is_hip_expert(ex) for ex in experts.values()):
                return self._combine_with_callables(x, idx, w, experts)
            first = next(iter(experts.values()))
            table = ops.expert_table([experts[e].c_struct() if e in experts else None
                                      for e in range(E)])
            tl = getattr(self.transfer_scheduler, "timeline", None)
            if tl is not None:           # the expert kernels start once the copies have landed
                k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                k0.record()
            route = ops.permute(idx32, E)
            _, ypart = ops.expert_ffn(table, E, x, k, x.shape[1], first.intermediate_size, route)
            out = ops.combine(ypart, w, idx32, route["slot_pos"])
            if tl is not None:
                k1.record()
                tl.append(("moe", k0, k1, self.layer_id))
            return out
        finally:
            if not self.retain_transferred:
                for e in unique:
                    if not was_resident[e]:
                        self.cache_manager.demote_to_cpu(self.layer_id, e)
            experts.clear()

    # ------------------------------------------------------------------ expert callables
    def _forward_experts(self, x: torch.Tensor) -> torch.Tensor:
        """The reference's per-expert loop for expert callables (model/moe_layer.py:142-211)."""
        idx, w = self.router.route(x)
        unique = sorted(int(e) for e in idx.reshape(-1).unique().tolist())
        was_resident = {e: (self.cache_manager.is_gpu_resident(self.layer_id, e)
                            if self.cache_manager is not None else True) for e in unique}
        experts = {}
        try:
            for e in unique:
                experts[e] = self._ensure_expert_on_gpu(e)
            return self._combine_with_callables(x, idx, w, experts)
        finally:
            if self.cache_manager is not None:
                for e in unique:
                    if not was_resident[e]:
                        self.cache_manager.demote_to_cpu(self.layer_id, e)
            experts.clear()

    @staticmethod
    def _combine_with_callables(x, idx, w, experts: dict) -> torch.Tensor:
        out = torch.zeros_like(x)
        for e in sorted(experts):
            matches = idx == e
            mask = matches.any(dim=-1)
            if not mask.any():
                continue
            tw = (w * matches.to(w.dtype)).sum(dim=-1)
            out[mask] += experts[e](x[mask]) * tw[mask].unsqueeze(-1)
        return out
