"""On-disk NF4 expert store: one safetensors file per (layer, expert) with the reference's
file and key scheme, so that a store written by either side reads on the other.

* File ``layer_{LL:02d}_expert_{EE:02d}.safetensors`` under one of several store
  directories, searched in order (model/loader.py:303-316 ``_resolve_expert_path``).
* Keys ``w1.`` / ``w2.`` / ``w3.`` + the serialized projection keys (model/expert.py:193-198):
  ``weight`` (packed uint8), ``weight.absmax``, ``weight.quant_map``,
  ``weight.quant_state.bitsandbytes__nf4`` (the JSON metadata blob), and for a nested
  (double-quantised) state ``weight.nested_absmax`` and ``weight.nested_quant_map``.
* ``load_expert`` follows the store branch of ``ModelLoader.load_expert``
  (model/loader.py:318-381): the tensors are read on the CPU with safetensors (no code
  runs from the file) and become a CPU-authoritative ``PrequantizedNF4Expert``.

The model loader's checkpoint side (HF safetensors index, dense layers, quantising from
bf16) is not here: the decoder takes synthetic or caller-provided weights.
"""
from __future__ import annotations

from pathlib import Path
from typing import Iterable, Optional, Union


from .expert import PrequantizedNF4Expert

PROJECTIONS = ("w1", "w2", "w3")


def expert_filename(layer_id: int, expert_id: int) -> str:
    return f"layer_{int(layer_id):02d}_expert_{int(expert_id):02d}.safetensors"


def expert_state_dict(expert: PrequantizedNF4Expert) -> dict:
    """The file's tensors: ``<projection>.<serialized key>`` -> contiguous CPU tensor."""
    out = {}
    for name in PROJECTIONS:
        for key, t in getattr(expert, name).items():
            out[f"{name}.{key}"] = t.detach().to("cpu").contiguous()
    return out


def save_expert(store_path: Union[str, Path], layer_id: int, expert_id: int,
                expert: PrequantizedNF4Expert) -> Path:
    """Write one expert as ``store_path/layer_LL_expert_EE.safetensors``."""
    from safetensors.torch import save_file

    d = Path(store_path)
    d.mkdir(parents=True, exist_ok=True)
    path = d / expert_filename(layer_id, expert_id)
    save_file(expert_state_dict(expert), str(path))
    return path


class NF4ExpertStore:
    """Reader of the per-expert NF4 files of one or more store directories."""

    def __init__(self, store_paths: Iterable[Union[str, Path]], hidden_size: int,
                 intermediate_size: int, num_layers: Optional[int] = None,
                 num_experts: Optional[int] = None) -> None:
        self._expert_store_paths = [Path(p) for p in store_paths]
        self.hidden_size = int(hidden_size)
        self.intermediate_size = int(intermediate_size)
        self.num_layers = num_layers
        self.num_experts = num_experts

    def _resolve_expert_path(self, layer_id: int, expert_id: int) -> Path:
        filename = expert_filename(layer_id, expert_id)
        for store_path in self._expert_store_paths:
            expert_path = store_path / filename
            if expert_path.is_file():
                return expert_path
        searched = ", ".join(str(p) for p in self._expert_store_paths)
        raise FileNotFoundError(f"Pre-quantized expert not found: {filename}. "
                                f"Searched stores: {searched}")

    def load_expert(self, layer_id: int, expert_id: int) -> PrequantizedNF4Expert:
        from safetensors import safe_open

        if self.num_layers is not None and not (0 <= layer_id < self.num_layers):
            raise IndexError(f"layer_id {layer_id} out of range [0, {self.num_layers})")
        if self.num_experts is not None and not (0 <= expert_id < self.num_experts):
            raise IndexError(f"expert_id {expert_id} out of range [0, {self.num_experts})")
        path = self._resolve_expert_path(layer_id, expert_id)
        with safe_open(str(path), framework="pt", device="cpu") as f:
            state = {key: f.get_tensor(key) for key in f.keys()}

        def extract(prefix: str) -> dict:
            return {key[len(prefix):]: value for key, value in state.items()
                    if key.startswith(prefix)}

        return PrequantizedNF4Expert.from_serialized(extract("w1."), extract("w2."), extract("w3."),
                                                     hidden_size=self.hidden_size,
                                                     intermediate_size=self.intermediate_size)
