"""NF4 expert store pinned once in host memory (offload mode).

The reference stages every transfer: a pageable CPU expert is copied into a pinned slot,
then to the device (transfer/reusable_staging.py:235-284, transfer/nf4_transfer.py:8-40).
Here the whole store is pinned up front -- one pinned arena per layer, allocated through
torch's pinned allocator (hipHostMalloc), each expert's device tensors packed as one
contiguous image (expert_image.py) -- so a transfer is a single hipMemcpyAsync from the
arena and staging copies nothing.  About 24 GiB for the Mixtral-8x7B store.

The CPU-tier experts it returns are PrequantizedNF4Expert objects with the reference's
serialized keys, whose tensors are views into the arena; ``image`` / ``image_layout`` name
the contiguous bytes to copy.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch

from ..model.expert import PrequantizedNF4Expert
from .expert_image import ImageLayout, canonical_expert, pack_image

_BLOB = "weight.quant_state.bitsandbytes__nf4"


@dataclasses.dataclass
class PinnedNF4Expert(PrequantizedNF4Expert):
    """A CPU-authoritative NF4 expert whose device tensors sit contiguously in pinned host
    memory."""

    image: Optional[torch.Tensor] = None          # uint8 view of the pinned arena
    image_layout: Optional[ImageLayout] = None


def _serialized(src, v: dict, name: str, ex) -> dict:
    """The reference's serialized keys over the pinned views; the JSON blob is the
    source's own when it has one, else written from the projection's shape."""
    s = {"weight": v["weight"], "weight.absmax": v["absmax"], "weight.quant_map": v["code"]}
    if v.get("state2_absmax") is not None:
        s["weight.nested_absmax"] = v["state2_absmax"]
        s["weight.nested_quant_map"] = v["state2_code"]
    blob = src.get(_BLOB) if isinstance(src, dict) else None
    if blob is None:
        from ..model.expert import NF4QuantState

        H, F = ex.hidden_size, ex.intermediate_size
        shape = torch.Size((H, F) if name == "w2" else (F, H))
        blob = NF4QuantState(absmax=v["absmax"], code=v["code"], shape=shape).blob()
    s[_BLOB] = blob.detach().cpu()
    return s


class PinnedExpertStore:
    """Builds pinned, contiguous CPU-tier experts, one arena per layer."""

    def __init__(self) -> None:
        self.arenas: list[torch.Tensor] = []

    @property
    def pinned_bytes(self) -> int:
        return sum(a.numel() for a in self.arenas)

    def add_layer(self, experts: list) -> list:
        """Pin the experts of one layer (any form canonical_expert reads, on any device):
        returns PinnedNF4Expert objects in the same order."""
        states = [canonical_expert(e) for e in experts]
        layouts = [ImageLayout.of(s) for s in states]
        total = sum(l.nbytes for l in layouts)
        arena = torch.empty((max(total, 1),), dtype=torch.uint8, pin_memory=True)
        self.arenas.append(arena)
        out, off = [], 0
        for ex, st, lay in zip(experts, states, layouts):
            image = arena[off:off + lay.nbytes]
            off += lay.nbytes
            views = pack_image(st, image, lay)        # device-to-host into the pinned arena
            ser = {name: _serialized(getattr(ex, name), views[name], name, ex)
                   for name in ("w1", "w2", "w3")}
            out.append(PinnedNF4Expert(w1=ser["w1"], w2=ser["w2"], w3=ser["w3"],
                                       hidden_size=ex.hidden_size,
                                       intermediate_size=ex.intermediate_size,
                                       image=image, image_layout=lay))
        return out
