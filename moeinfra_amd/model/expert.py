"""NF4 expert containers (mirrors model/expert.py of the reference).

* ``QuantizedMixtralExpert(w1, w2, w3)`` (model/expert.py:8-87): bf16 weights, NF4-quantised
  (blocksize 64, fp32 absmax, no nested statistics) by the HIP quantiser when the expert
  moves to the GPU, as bitsandbytes' Params4bit does on ``.cuda()``; ``forward`` runs
  ``w2(silu(w1 x) * w3 x)`` on the HIP kernels.
* ``PrequantizedNF4Expert`` (model/expert.py:176-242): the CPU-authoritative serialized
  NF4 state dicts, with the bitsandbytes key names.

The serialized layout per projection is bitsandbytes' Linear4bit.state_dict():
``weight`` (packed uint8 [n/2, 1], high nibble first), ``weight.absmax`` (fp32),
``weight.quant_map`` (fp32[16]) and ``weight.quant_state.bitsandbytes__nf4`` (a uint8 tensor
holding a JSON dict with quant_type, blocksize, dtype, shape).
"""
from __future__ import annotations

import dataclasses
import json
from typing import Optional

import torch
import torch.nn as nn

from .. import ops
from .._lib import MoeNf4Expert
from ..nf4 import NF4_BLOCKSIZE, NF4_DTYPE, NF4_QUANT_STORAGE, NF4_QUANT_TYPE, nf4_code_tensor

_BLOB_KEY = "quant_state.bitsandbytes__" + NF4_QUANT_TYPE


# ----------------------------------------------------------------------------- quant state
@dataclasses.dataclass
class NF4QuantState:
    """Metadata of one NF4 weight (the fields of bitsandbytes' QuantState that the
    reference reads: absmax, code, offset, state2, blocksize, quant_type, shape, dtype)."""

    absmax: torch.Tensor
    code: torch.Tensor
    shape: torch.Size
    blocksize: int = NF4_BLOCKSIZE
    quant_type: Optional[str] = NF4_QUANT_TYPE
    dtype: torch.dtype = NF4_DTYPE
    offset: Optional[torch.Tensor] = None
    state2: Optional["NF4QuantState"] = None

    @property
    def nested(self) -> bool:
        return self.state2 is not None

    def to(self, device) -> "NF4QuantState":
        mv = lambda t: None if t is None else t.to(device)
        return dataclasses.replace(self, absmax=mv(self.absmax), code=mv(self.code),
                                   offset=mv(self.offset),
                                   state2=None if self.state2 is None else self.state2.to(device))

    def fp32_absmax(self) -> torch.Tensor:
        """The fp32 block scales the kernels take: ``absmax`` itself, or for a nested state
        its expansion on the GPU (moe_nf4_expand_absmax), computed once and kept."""
        if not self.nested:
            return self.absmax
        cached = self.__dict__.get("_absmax_f32")
        if cached is not None and cached.device == self.absmax.device:
            return cached
        if self.absmax.dtype != torch.uint8:
            raise ValueError(f"nested absmax must be uint8 indices, got {self.absmax.dtype}")
        out = ops.nf4_expand_absmax(self.absmax, self.state2.absmax, self.state2.code, self.offset,
                                    self.state2.blocksize)
        self.__dict__["_absmax_f32"] = out
        return out

    def blob(self) -> torch.Tensor:
        meta = {"quant_type": self.quant_type, "blocksize": self.blocksize,
                "dtype": str(self.dtype).replace("torch.", ""), "shape": list(self.shape)}
        if self.state2 is not None:
            meta.update({"nested_blocksize": self.state2.blocksize,
                         "nested_dtype": str(self.state2.dtype).replace("torch.", ""),
                         "nested_offset": None if self.offset is None else float(self.offset)})
        return torch.tensor(list(json.dumps(meta).encode()), dtype=torch.uint8)


def parse_blob(blob: Optional[torch.Tensor]) -> dict:
    """Decode a ``quant_state.bitsandbytes__nf4`` tensor; {} if it holds no JSON dict."""
    if blob is None:
        return {}
    try:
        meta = json.loads(bytes(blob.detach().cpu().reshape(-1).tolist()).decode())
    except (ValueError, UnicodeDecodeError):
        return {}
    return meta if isinstance(meta, dict) else {}


# ----------------------------------------------------------------------------- linear shell
class NF4Linear(nn.Module):
    """One NF4 projection: ``weight`` holds the packed uint8 nibbles once quantised (the
    bf16 matrix before), ``quant_state`` its absmax/codebook."""

    def __init__(self, weight: torch.Tensor, in_features: int, out_features: int,
                 quant_state: Optional[NF4QuantState] = None) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.bias = None
        self.compute_dtype = torch.bfloat16
        self.quant_storage = NF4_QUANT_STORAGE
        self.weight = weight
        self.quant_state = quant_state

    @property
    def quantized(self) -> bool:
        return self.quant_state is not None

    def quantize_(self) -> "NF4Linear":
        """Quantise the bf16 weight in place on its (GPU) device with the HIP quantiser."""
        if self.quantized:
            return self
        packed, absmax, code = ops.nf4_quantize(self.weight.contiguous(), NF4_BLOCKSIZE)
        self.quant_state = NF4QuantState(absmax=absmax, code=code.clone(),
                                          shape=torch.Size((self.out_features, self.in_features)))
        self.weight = packed
        return self

    def to_device(self, device) -> "NF4Linear":
        self.weight = self.weight.to(device)
        if self.quant_state is not None:
            self.quant_state = self.quant_state.to(device)
        return self

    def dequantize(self) -> torch.Tensor:
        """bf16 [out, in] via the HIP NF4 dequant kernel (bit-exact bitsandbytes semantics)."""
        if not self.quantized:
            return self.weight
        qs = self.quant_state
        return ops.nf4_dequant(self.weight, qs.fp32_absmax(), qs.code,
                               (self.out_features, self.in_features), qs.blocksize)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # A lone projection is not on the expert fast path: dequantise with the HIP kernel
        # and use the device GEMM.
        w = self.dequantize()
        return torch.nn.functional.linear(x.to(w.dtype), w).to(x.dtype)

    def serialized(self, prefix: str = "") -> dict[str, torch.Tensor]:
        if not self.quantized:
            raise ValueError("projection is not quantised yet (move the expert to the GPU)")
        qs = self.quant_state
        out = {f"{prefix}weight": self.weight, f"{prefix}weight.absmax": qs.absmax,
               f"{prefix}weight.quant_map": qs.code, f"{prefix}weight.{_BLOB_KEY}": qs.blob()}
        if qs.state2 is not None:
            out[f"{prefix}weight.nested_absmax"] = qs.state2.absmax
            out[f"{prefix}weight.nested_quant_map"] = qs.state2.code
        return out


def expert_struct(w1: NF4Linear, w2: NF4Linear, w3: NF4Linear) -> MoeNf4Expert:
    """moe_nf4_expert_t of three quantised device-resident projections."""
    for lin in (w1, w2, w3):
        if not lin.quantized or lin.weight.device.type != "cuda":
            raise ValueError("expert projections must be NF4-quantised and on the GPU")
        if lin.weight.dtype != NF4_QUANT_STORAGE:
            raise ValueError(f"Expected packed NF4 weight dtype {NF4_QUANT_STORAGE}, "
                             f"got {lin.weight.dtype}")
        if lin.quant_state.blocksize != NF4_BLOCKSIZE:
            raise ValueError(f"the fused expert kernels need blocksize {NF4_BLOCKSIZE}")
    p = lambda t: t.data_ptr()
    a = lambda lin: lin.quant_state.fp32_absmax().data_ptr()  # nested states: expanded once
    return MoeNf4Expert(p(w1.weight), a(w1), p(w1.quant_state.code),
                        p(w3.weight), a(w3), p(w3.quant_state.code),
                        p(w2.weight), a(w2), p(w2.quant_state.code))


def swiglu_forward(expert, x: torch.Tensor) -> torch.Tensor:
    """``w2(silu(w1 x) * w3 x)`` of an NF4 expert on the HIP kernels; any leading shape.
    Activations are computed in bf16 (other dtypes are converted and the result cast
    back)."""
    if x.device.type != "cuda":
        raise ValueError(f"expert input must be on the GPU (got {x.device})")
    lead = x.shape[:-1]
    xb = x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous()
    y = ops.expert_swiglu(expert.c_struct(), xb, expert.hidden_size, expert.intermediate_size)
    return y.reshape(*lead, expert.hidden_size).to(x.dtype)


# ----------------------------------------------------------------------------- experts
class QuantizedMixtralExpert(nn.Module):
    """A Mixtral SwiGLU expert with NF4 projections w1, w3: H -> F and w2: F -> H."""

    def __init__(self, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> None:
        super().__init__()
        self.w1 = self._quantize_linear(w1)
        self.w2 = self._quantize_linear(w2)
        self.w3 = self._quantize_linear(w3)
        self.intermediate_size, self.hidden_size = w1.shape
        self._struct: Optional[MoeNf4Expert] = None

    @staticmethod
    def _quantize_linear(weight: torch.Tensor) -> NF4Linear:
        if weight.ndim != 2:
            raise ValueError(f"Expected a 2D weight tensor, got shape {weight.shape}")
        if weight.dtype != torch.bfloat16:
            raise ValueError(f"Expected BF16 weights, got {weight.dtype}")
        lin = NF4Linear(weight, in_features=weight.shape[1], out_features=weight.shape[0])
        if weight.device.type == "cuda":
            lin.quantize_()
        return lin

    def cuda(self, device=None) -> "QuantizedMixtralExpert":
        dev = torch.device("cuda" if device is None else device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        for lin in (self.w1, self.w2, self.w3):
            lin.to_device(dev)
            lin.quantize_()
        self._struct = None
        return self

    def cpu(self) -> "QuantizedMixtralExpert":
        for lin in (self.w1, self.w2, self.w3):
            lin.to_device("cpu")
        self._struct = None
        return self

    def to(self, device) -> "QuantizedMixtralExpert":  # type: ignore[override]
        return self.cuda(device) if torch.device(device).type == "cuda" else self.cpu()

    def c_struct(self) -> MoeNf4Expert:
        if self._struct is None:
            self._struct = expert_struct(self.w1, self.w2, self.w3)
        return self._struct

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return swiglu_forward(self, x)

    @property
    def device(self) -> torch.device:
        return self.w1.weight.device

    @property
    def size_bytes(self) -> int:
        return sum(l.weight.numel() * l.weight.element_size() for l in (self.w1, self.w2, self.w3))

    def state_dict(self, *args, **kwargs):  # type: ignore[override]
        out = {}
        for name in ("w1", "w2", "w3"):
            out.update(getattr(self, name).serialized(prefix=f"{name}."))
        return out

    @classmethod
    def from_prequantized(cls, w1_state: dict, w2_state: dict, w3_state: dict, hidden_size: int,
                          intermediate_size: int) -> "QuantizedMixtralExpert":
        """Expert from Linear4bit.state_dict()-style NF4 tensors (kept on the CPU)."""
        expert = cls.__new__(cls)
        nn.Module.__init__(expert)
        expert.hidden_size = hidden_size
        expert.intermediate_size = intermediate_size
        expert._struct = None
        expert.w1 = _linear_from_serialized(w1_state, hidden_size, intermediate_size)
        expert.w2 = _linear_from_serialized(w2_state, intermediate_size, hidden_size)
        expert.w3 = _linear_from_serialized(w3_state, hidden_size, intermediate_size)
        return expert


_REQUIRED = {"weight", "weight.absmax", "weight.quant_map", "weight." + _BLOB_KEY}


def _linear_from_serialized(state: dict, in_features: int, out_features: int) -> NF4Linear:
    missing = _REQUIRED - state.keys()
    if missing:
        raise ValueError(f"Missing prequantized NF4 state tensors: {sorted(missing)}")
    meta = parse_blob(state["weight." + _BLOB_KEY])
    qs = NF4QuantState(absmax=state["weight.absmax"].cpu(), code=state["weight.quant_map"].cpu(),
                       shape=torch.Size((out_features, in_features)),
                       blocksize=int(meta.get("blocksize", NF4_BLOCKSIZE)))
    if "weight.nested_absmax" in state:
        qs.state2 = NF4QuantState(absmax=state["weight.nested_absmax"].cpu(),
                                  code=state["weight.nested_quant_map"].cpu(),
                                  shape=qs.absmax.shape,
                                  blocksize=int(meta.get("nested_blocksize", 256)),
                                  quant_type=None, dtype=torch.float32)
        off = meta.get("nested_offset")
        qs.offset = None if off is None else torch.tensor(off, dtype=torch.float32)
    return NF4Linear(state["weight"].cpu(), in_features, out_features, qs)


@dataclasses.dataclass
class PrequantizedNF4Expert:
    """CPU-resident serialized NF4 expert: the tensors exactly as stored."""

    w1: dict
    w2: dict
    w3: dict
    hidden_size: int
    intermediate_size: int

    _REQUIRED_KEYS = frozenset(_REQUIRED)

    @classmethod
    def from_serialized(cls, w1: dict, w2: dict, w3: dict, hidden_size: int,
                        intermediate_size: int) -> "PrequantizedNF4Expert":
        for name, state in (("w1", w1), ("w2", w2), ("w3", w3)):
            missing = cls._REQUIRED_KEYS - state.keys()
            if missing:
                raise ValueError(f"Missing serialized NF4 state for {name}: {sorted(missing)}")
        return cls(w1=dict(w1), w2=dict(w2), w3=dict(w3), hidden_size=hidden_size,
                   intermediate_size=intermediate_size)

    @classmethod
    def from_nf4_tensors(cls, states: dict, hidden_size: int,
                         intermediate_size: int) -> "PrequantizedNF4Expert":
        """Serialized expert from {"w1"|"w3"|"w2": (packed uint8, absmax fp32, code fp32)}
        (w1/w3 [intermediate, hidden], w2 [hidden, intermediate]), with the keys the
        reference's store uses (model/expert.py:193-198)."""
        shapes = {"w1": (intermediate_size, hidden_size), "w3": (intermediate_size, hidden_size),
                  "w2": (hidden_size, intermediate_size)}
        ser = {}
        for name, (packed, absmax, code) in states.items():
            qs = NF4QuantState(absmax=absmax, code=code, shape=torch.Size(shapes[name]))
            ser[name] = {"weight": packed.reshape(-1, 1), "weight.absmax": absmax,
                         "weight.quant_map": code, "weight." + _BLOB_KEY: qs.blob()}
        return cls.from_serialized(ser["w1"], ser["w2"], ser["w3"], hidden_size, intermediate_size)

    @property
    def device(self) -> torch.device:
        return self.w1["weight"].device

    @property
    def size_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for st in (self.w1, self.w2, self.w3)
                   for t in st.values())
