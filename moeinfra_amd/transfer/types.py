"""Transfer request/result types (mirrors transfer/types.py:13-70 of the reference).

Requests name an expert by (layer_id, expert_id); the CacheManager owns the expert
objects and their residency, the scheduler only moves them.
"""
from __future__ import annotations

import dataclasses
import enum


class TransferDirection(enum.Enum):
    """Direction of an expert residency change."""

    CPU_TO_GPU = "cpu_to_gpu"
    GPU_TO_CPU = "gpu_to_cpu"


class TransferPriority(enum.Enum):
    """Scheduling priority (lower value runs first)."""

    HIGH = 0
    NORMAL = 1
    LOW = 2


@dataclasses.dataclass(frozen=True)
class TransferRequest:
    request_id: str
    layer_id: int
    expert_id: int
    direction: TransferDirection
    priority: TransferPriority
    issued_at: float


@dataclasses.dataclass(frozen=True)
class TransferResult:
    request_id: str
    success: bool
    elapsed_ms: float
    bytes_transferred: int
    error: str | None = None


class TransferStatus(enum.Enum):
    IN_FLIGHT = "in_flight"
    READY = "ready"
    REJECTED = "rejected"
    CANCELLED = "cancelled"


@dataclasses.dataclass
class TransferHandle:
    request_id: str
    layer_id: int
    expert_id: int
    slot: object
    event: object
    status: TransferStatus = TransferStatus.IN_FLIGHT
    gpu_state: object = None
    cpu_expert: object = None
    #: Bytes the transfer moves host -> device (recorded by the bandwidth monitor when the
    #: copy is seen complete).
    nbytes: int = 0
