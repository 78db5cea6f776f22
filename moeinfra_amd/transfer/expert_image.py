"""The device-side tensors of one NF4 expert and their contiguous byte image.

A transfer moves, per projection (w1, w2, w3), the tensors the kernels read: the packed
weight, the block scales, the codebook, and for a nested (double-quantised) state its
second-level scales, codebook and offset -- the canonical staging keys of the reference's
transfer/reusable_staging.py:126-222 (``weight, absmax, code, offset[, state2_absmax,
state2_code, state2_offset]``).  The bitsandbytes JSON blob is host metadata and does not
travel.

An *image* lays those tensors out back to back at 256-byte offsets.  The offload store
keeps every expert's image in pinned host memory, the GPU tier keeps transferred experts
in device slots with the same layout, so one expert crosses the host link as a single
hipMemcpyAsync and its device tensors are views into the slot.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch

PROJECTIONS = ("w1", "w2", "w3")
IMAGE_ALIGN = 256

# serialized (bitsandbytes Linear4bit.state_dict) key -> canonical key
_SERIALIZED = {"weight": "weight", "weight.absmax": "absmax", "weight.quant_map": "code",
               "weight.nested_absmax": "state2_absmax", "weight.nested_quant_map": "state2_code"}
_BLOB = "weight.quant_state.bitsandbytes__nf4"
_CANONICAL_ORDER = ("weight", "absmax", "code", "offset", "state2_absmax", "state2_code",
                    "state2_offset")


def _from_quant_state(weight: torch.Tensor, qs) -> dict:
    out = {"weight": weight, "absmax": qs.absmax, "code": qs.code,
           "offset": getattr(qs, "offset", None)}
    s2 = getattr(qs, "state2", None)
    if s2 is not None:
        out.update(state2_absmax=s2.absmax, state2_code=s2.code,
                   state2_offset=getattr(s2, "offset", None))
    return out


def canonical_projection(expert, name: str) -> dict:
    """One projection of an expert as {canonical key: tensor or None}.  Accepts the forms a
    CPU-tier expert can hold: a dict in canonical or serialized (bitsandbytes) keys, an
    object with such a ``state`` dict or a ``serialized()`` method, or an NF4 linear with
    ``weight`` and ``quant_state``."""
    proj = getattr(expert, name)
    raw = proj if isinstance(proj, dict) else getattr(proj, "state", None)
    if not isinstance(raw, dict):
        if getattr(proj, "quant_state", None) is not None:
            return _from_quant_state(proj.weight, proj.quant_state)
        if hasattr(proj, "serialized"):
            raw = proj.serialized()
    if not isinstance(raw, dict):
        raise TypeError(f"Expert projection {name!r} does not expose serialized NF4 state")
    if "weight" not in raw:
        raise ValueError(f"Projection {name!r} is missing 'weight'")
    if "absmax" in raw:                                      # canonical already
        alias = {"code": "quant_map"}
        out = {k: raw.get(k, raw.get(alias.get(k, k))) for k in _CANONICAL_ORDER
               if k in _CANONICAL_ORDER[:4] or k in raw}
        if out["code"] is None:
            raise ValueError(f"Projection {name!r} is missing NF4 code/quant_map")
        return out
    missing = {"weight.absmax", "weight.quant_map", _BLOB} - raw.keys()
    if missing:
        raise ValueError(f"Projection {name!r} is missing serialized NF4 state tensors: "
                         f"{sorted(missing)}")
    out = {_SERIALIZED[k]: v for k, v in raw.items() if k in _SERIALIZED}
    out["offset"] = None
    if "state2_absmax" in out:
        from ..model.expert import parse_blob

        off = parse_blob(raw[_BLOB]).get("nested_offset")
        out["offset"] = None if off is None else torch.tensor(off, dtype=torch.float32)
        out["state2_offset"] = None
    return {k: out[k] for k in _CANONICAL_ORDER if k in out}


def canonical_expert(expert) -> dict:
    """{projection: canonical_projection(expert, projection)} for w1, w2, w3."""
    return {name: canonical_projection(expert, name) for name in PROJECTIONS}


@dataclasses.dataclass(frozen=True)
class ImageField:
    projection: str
    key: str
    offset: int
    nbytes: int
    dtype: torch.dtype
    shape: tuple


@dataclasses.dataclass(frozen=True)
class ImageLayout:
    fields: tuple
    nbytes: int

    @staticmethod
    def of(state: dict) -> "ImageLayout":
        """Back-to-back layout (256-byte aligned) of a canonical expert state's tensors."""
        fields, off = [], 0
        for name in PROJECTIONS:
            for key, t in state[name].items():
                if t is None:
                    continue
                n = t.numel() * t.element_size()
                fields.append(ImageField(name, key, off, n, t.dtype, tuple(t.shape)))
                off += -(-n // IMAGE_ALIGN) * IMAGE_ALIGN
        return ImageLayout(tuple(fields), off)

    def views(self, buf: torch.Tensor, template: Optional[dict] = None) -> dict:
        """Tensors of the layout as views into the uint8 buffer `buf` (an image-sized
        region); keys the template holds as None stay None."""
        out = {name: {} for name in PROJECTIONS}
        if template is not None:
            for name in PROJECTIONS:
                out[name] = {k: None for k, v in template[name].items() if v is None}
        for f in self.fields:
            v = buf[f.offset:f.offset + f.nbytes].view(f.dtype).reshape(f.shape)
            out[f.projection][f.key] = v
        return out


def pack_image(state: dict, buf: torch.Tensor, layout: ImageLayout) -> dict:
    """Copy a canonical state into `buf` at `layout`; returns the views (same device)."""
    views = layout.views(buf, state)
    for f in layout.fields:
        views[f.projection][f.key].copy_(state[f.projection][f.key])
    return views
