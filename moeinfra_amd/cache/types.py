"""Cache entry / statistics / policy types (mirrors cache/types.py:17-101 of the reference)."""
from __future__ import annotations

import dataclasses
import enum
import time
from typing import Any, Optional


class EvictionPolicy(enum.Enum):
    LRU = "lru"
    LFU = "lfu"
    ARC = "arc"


@dataclasses.dataclass
class CacheEntry:
    """One cached expert in the GPU or the CPU tier."""

    expert_id: int
    layer_id: int
    device: str
    expert: Optional[Any]
    last_access: float
    access_count: int
    size_bytes: int

    @property
    def is_on_gpu(self) -> bool:
        return self.device.startswith("cuda")

    @property
    def age(self) -> float:
        return time.monotonic() - self.last_access


@dataclasses.dataclass
class CacheStats:
    hits: int = 0
    misses: int = 0
    evictions: int = 0
    gpu_slots_used: int = 0
    cpu_slots_used: int = 0

    @property
    def hit_rate(self) -> float:
        total = self.hits + self.misses
        return self.hits / total if total > 0 else 0.0
