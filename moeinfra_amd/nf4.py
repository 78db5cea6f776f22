"""NF4 constants of the expert path.

The codebook is the 16-level NormalFloat4 table (QLoRA, Dettmers et al. 2023), which is
what bitsandbytes stores as ``quant_map`` for ``quant_type="nf4"``; the reference fixes
blocksize 64 and bf16 as the dequantised dtype (transfer/nf4_reconstruct.py:9-14).
"""
from __future__ import annotations

import torch

NF4_BLOCKSIZE = 64
NF4_NESTED_BLOCKSIZE = 256
NF4_QUANT_TYPE = "nf4"
NF4_DTYPE = torch.bfloat16
NF4_QUANT_STORAGE = torch.uint8

NF4_CODE_VALUES = (
    -1.0,
    -0.6961928009986877,
    -0.5250730514526367,
    -0.39491748809814453,
    -0.28444138169288635,
    -0.18477343022823334,
    -0.09105003625154495,
    0.0,
    0.07958029955625534,
    0.16093020141124725,
    0.24611230194568634,
    0.33791524242401123,
    0.44070982933044434,
    0.5626170039176941,
    0.7229568362236023,
    1.0,
)

_code_cache: dict = {}


def nf4_code_tensor(device="cpu") -> torch.Tensor:
    """The NF4 codebook as fp32[16] on ``device`` (cached; do not modify in place)."""
    dev = torch.device(device)
    t = _code_cache.get(dev)
    if t is None:
        t = torch.tensor(NF4_CODE_VALUES, dtype=torch.float32, device=dev)
        _code_cache[dev] = t
    return t
