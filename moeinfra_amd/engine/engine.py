"""End-to-end inference engine (the generate() surface of engine/engine.py:440-627 of the
reference) over the native decoder (decoder.py) and the NF4 MoE layer.

generate(request): prefill the prompt (the last position's logits give the first token),
then greedy decode; ttft_ms is the prefill time, tps = (generated - 1) / decode seconds
(engine/engine.py:478-484).  Batch 1, like the reference's decode path.

Two expert modes, as in the reference:
* all-resident: every NF4 expert stays in HBM (288 GB holds all 23.6 GiB); the MoE block
  is one call of the layer entry point, and the whole decode step (embedding, 32 decoder
  layers, final norm, lm_head, argmax, position advance) is captured once as a HIP graph
  and replayed per token.  Generated ids stay on the device until the end.
* offload: the NF4 store is pinned once in host memory (CacheManager CPU tier) with a
  bounded GPU tier in a device-slot arena; each layer's MoE block is the reference's
  MoELayer (route, start the copies of the routed experts that are not resident as single
  hipMemcpyAsync calls on a side stream, run the kernels behind stream waits on their
  events, demote the ones that were not resident), optionally with a per-layer GPU tier
  that keeps transferred experts and with the PrefetchEngine starting later layers' copies
  (whole copies, or with NEXT_ROUTER bounded prefixes sized to the host link's idle gap).
"""
from __future__ import annotations

import logging
import time
from typing import Optional

import torch

from .decoder import DecoderWeights, NativeDecoder
from .prefetch import PrefetchEngine
from .types import ForwardRequest, ForwardResult, PrefetchPolicy


#: NEXT_ROUTER's bounded prefix per guessed expert: about the host link's idle time between
#: two layers' copies in the offload decode loop (8 MiB at ~54 GB/s is ~0.15 ms).
NEXT_ROUTER_PREFIX_BYTES = 8 << 20


class InferenceEngine:
    """Native Mixtral-shaped NF4 MoE inference engine on one GPU."""

    def __init__(self, weights: DecoderWeights, max_seq: int = 1024, device="cuda:0",
                 offload: bool = False, gpu_expert_slots: Optional[int] = None,
                 prefetch: PrefetchPolicy = PrefetchPolicy.NONE, prefetch_depth: int = 1,
                 use_graph: bool = True, logger: Optional[logging.Logger] = None,
                 gpu_slots_per_layer: Optional[int] = None, cache_policy="lru",
                 prefetch_prefix_bytes: Optional[int] = NEXT_ROUTER_PREFIX_BYTES) -> None:
        self._logger = logger or logging.getLogger(__name__)
        self.device = torch.device(device)
        self.weights = weights
        self.offload = offload
        self.use_graph = use_graph and not offload
        self._moe_layers = None
        self.cache_manager = None
        self.transfer_scheduler = None
        self.prefetch_engine = None
        self.pinned_store = None
        self._prefix_bytes = None            # None: NEXT_ROUTER copies whole experts ahead
        if prefetch_prefix_bytes and prefetch == PrefetchPolicy.NEXT_ROUTER:
            self._prefix_bytes = int(prefetch_prefix_bytes)
        moe = None
        if offload:
            moe = self._build_offload(gpu_expert_slots, prefetch, prefetch_depth,
                                      gpu_slots_per_layer, cache_policy)
        self.decoder = NativeDecoder(weights, max_seq, self.device, moe=moe)
        self._graph = None
        self._last_logits = None

    # ------------------------------------------------------------------ offload wiring
    def _build_offload(self, gpu_slots, policy, depth, slots_per_layer, cache_policy):
        """The host-authoritative offload mode: every expert pinned once in host memory
        (one arena per layer) as the CacheManager's CPU tier; a bounded GPU tier of
        `gpu_slots` experts (default: all) in a preallocated device-slot arena, filled by
        single-copy host-to-device transfers on a side stream that the compute stream waits
        for with events.  With `slots_per_layer` the GPU tier is partitioned by layer and
        layers keep the experts they transferred (otherwise they are demoted after the
        layer, the reference's contract).  `cache_policy` ("lru", "lfu", "arc" or an
        EvictionPolicy) picks the GPU tier's victims.  With NEXT_ROUTER bounded prefixes
        the arena holds one more slot per expert of a layer for the prefixes in flight."""
        from ..cache.manager import CacheManager
        from ..cache.types import EvictionPolicy
        from ..model.expert import PrequantizedNF4Expert
        from ..model.moe_layer import MoELayer
        from ..transfer.device_slots import DeviceExpertSlots
        from ..transfer.host_store import PinnedExpertStore
        from ..transfer.scheduler import TransferScheduler
        from .router import ExpertRouter

        s = self.weights.shape
        n_experts = s.layers * s.experts
        gpu_slots = n_experts if gpu_slots is None else max(1, int(gpu_slots))
        if slots_per_layer is not None:
            gpu_slots = min(gpu_slots, slots_per_layer * s.layers)
        cm = CacheManager(gpu_slots=gpu_slots, cpu_slots=n_experts,
                          policy=EvictionPolicy(cache_policy),
                          gpu_slots_per_layer=slots_per_layer)
        store = PinnedExpertStore()
        for l, lw in enumerate(self.weights.layers):
            src = [PrequantizedNF4Expert.from_nf4_tensors(st, s.hidden, s.ffn) for st in lw.experts]
            for e, ex in enumerate(store.add_layer(src)):
                cm.put(l, e, ex, device="cpu")
        self.pinned_store = store
        image_bytes = cm.peek_cpu(0, 0).image_layout.nbytes
        self._transfer_stream = torch.cuda.Stream(self.device)
        extra = s.experts if self._prefix_bytes else 0
        slots = DeviceExpertSlots(gpu_slots + extra, image_bytes, self.device)
        sched = TransferScheduler(cm, 24.0, max(2 * s.experts, 2 * s.top_k * max(depth, 1)),
                                  transfer_stream=self._transfer_stream, device_slots=slots)
        self.cache_manager, self.transfer_scheduler = cm, sched
        if policy != PrefetchPolicy.NONE:
            self.prefetch_engine = PrefetchEngine(cm, sched, policy, depth, logger=self._logger)
        retain = slots_per_layer is not None
        self._moe_layers = [MoELayer(l, ExpertRouter(lw.gate, s.top_k), cm, None, sched,
                                     logger=self._logger, retain_transferred=retain)
                            for l, lw in enumerate(self.weights.layers)]
        return self._moe_offload

    def _moe_offload(self, l: int, x: torch.Tensor) -> torch.Tensor:
        pe = self.prefetch_engine
        if pe is None:
            return self._moe_layers[l].forward(x)
        pe.poll()
        nxt = None
        if pe.policy == PrefetchPolicy.NEXT_ROUTER and l + 1 < len(self._moe_layers):
            # Enqueued before this layer's routing: the layer's own read-back of its routed
            # set covers it, so the guess costs no extra host synchronisation.
            nxt, _ = self._moe_layers[l + 1].router.route(x)
        out = self._moe_layers[l].forward(x)
        if pe.policy == PrefetchPolicy.NEXT_ROUTER:
            pe.poll()
            pe.cancel_stale(l + 1)           # also settles this layer's prefixes
            if nxt is not None:
                guess = nxt.reshape(-1).tolist()
                if self._prefix_bytes:
                    pe.prefetch_prefix(l + 1, guess, self._prefix_bytes)
                else:
                    pe.prefetch(l + 1, guess)
        else:
            pe.on_layer_complete(l, self._moe_layers[l].last_expert_indices)
        return out

    # ------------------------------------------------------------------ generate
    @torch.no_grad()
    def generate(self, request: ForwardRequest) -> ForwardResult:
        ids = request.input_ids
        if ids.ndim == 2 and ids.shape[1] + max(request.max_new_tokens - 1, 0) > self.decoder.max_seq:
            raise ValueError(f"prompt ({ids.shape[1]}) + new tokens ({request.max_new_tokens}) "
                             f"exceed max_seq {self.decoder.max_seq}")
        stage = {}
        t0 = time.perf_counter()
        logits = self._prefill(request.input_ids, request.attention_mask)
        torch.cuda.synchronize(self.device)
        ttft_ms = (time.perf_counter() - t0) * 1e3
        stage["prefill"] = ttft_ms
        t1 = time.perf_counter()
        tokens = self._decode(logits, request.max_new_tokens)
        torch.cuda.synchronize(self.device)
        decode_ms = (time.perf_counter() - t1) * 1e3
        stage["decode"] = decode_ms
        steps = max(len(tokens) - 1, 0)
        tps = steps / (decode_ms / 1e3) if steps > 0 and decode_ms > 0 else 0.0
        last = self._last_logits if self._last_logits is not None else logits
        return ForwardResult(logits=last, token_ids=tokens, ttft_ms=ttft_ms, tps=tps,
                             stage_timings=stage)

    @torch.no_grad()
    def _prefill(self, input_ids: torch.Tensor, attention_mask=None) -> torch.Tensor:
        """Encode the prompt [1, S] into the KV cache; logits [1, 1, V] of its last token."""
        if input_ids.ndim != 2:
            raise ValueError(f"input_ids must have shape (batch, seq_len), got {tuple(input_ids.shape)}")
        if input_ids.shape[0] != 1:
            raise ValueError("the decode path supports batch_size=1")
        if input_ids.shape[1] <= 0:
            raise ValueError("input_ids must contain at least one token")
        if attention_mask is not None and attention_mask.shape != input_ids.shape:
            raise ValueError("attention_mask must have the same shape as input_ids")
        if attention_mask is not None and not bool(attention_mask.all()):
            raise NotImplementedError("padded prompts are not supported (batch 1, causal mask)")
        if input_ids.shape[1] > self.decoder.max_seq:
            raise ValueError(f"prompt of {input_ids.shape[1]} tokens exceeds max_seq {self.decoder.max_seq}")
        self.decoder.reset()
        ids = input_ids[0].to(device=self.device, dtype=torch.long)
        logits = self.decoder.forward(ids).reshape(1, 1, -1)
        self._last_logits = logits
        return logits

    def prepare(self, max_new_tokens: int) -> None:
        """Capture the decode-step graph for up to ``max_new_tokens`` generated tokens now,
        so that no later generate() of that length captures inside its timed decode
        (all-resident graph mode; nothing to do in eager or offload mode)."""
        if self.use_graph and (self._graph is None or self._graph_n < max_new_tokens):
            with torch.no_grad():
                self._capture(max(max_new_tokens, 64))

    def _capture(self, n_max: int):
        """Graph of one decode step: token in -> logits, argmax, token out, position + 1,
        generated id stored at the step counter."""
        dec = self.decoder
        self._tok = torch.zeros((1,), dtype=torch.long, device=self.device)
        self._gen = torch.zeros((n_max,), dtype=torch.long, device=self.device)
        self._ctr = torch.zeros((1,), dtype=torch.long, device=self.device)
        pos_save = dec.pos.clone()
        kc, vc = dec.k_cache.clone(), dec.v_cache.clone()

        def body():
            return dec.decode_step(self._tok, self._gen, self._ctr)

        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):  # warm up allocations and library state outside the capture
                body()
        torch.cuda.current_stream(self.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._graph_logits = body()
        # The warm-up and the capture advanced the state: restore it.
        dec.pos.copy_(pos_save)
        dec.k_cache.copy_(kc)
        dec.v_cache.copy_(vc)
        self._graph = graph
        self._graph_n = n_max

    @torch.no_grad()
    def _decode(self, next_token_logits: torch.Tensor, max_new_tokens: int) -> list:
        """Greedy decode from the prompt's logits (engine/engine.py:568-627)."""
        if max_new_tokens < 0:
            raise ValueError("max_new_tokens must be non-negative")
        if max_new_tokens == 0:
            return []
        if next_token_logits.shape[0] != 1:
            raise ValueError("Current decode path supports batch_size=1")
        dec = self.decoder
        first = next_token_logits[:, -1, :].argmax(dim=-1)
        if max_new_tokens == 1:
            return [int(first.item())]
        if self.use_graph:
            if self._graph is None or self._graph_n < max_new_tokens:
                self._capture(max(max_new_tokens, 64))
            self._tok.copy_(first)
            self._ctr.zero_()
            self._gen[0:1].copy_(first)
            self._ctr.add_(1)
            for _ in range(1, max_new_tokens):
                self._graph.replay()
            self._last_logits = self._graph_logits.reshape(1, 1, -1).clone()
            return [int(v) for v in self._gen[:max_new_tokens].tolist()]
        # Eager steps: the same decode_step as the graph body, one launch sequence per token.
        tok = first.clone()
        gen = torch.zeros((max_new_tokens,), dtype=torch.long, device=self.device)
        ctr = torch.ones((1,), dtype=torch.long, device=self.device)
        gen[0:1].copy_(first)
        logits = next_token_logits
        for _ in range(1, max_new_tokens):
            logits = dec.decode_step(tok, gen, ctr)
        self._last_logits = logits.reshape(1, 1, -1).clone()
        return [int(v) for v in gen.tolist()]
