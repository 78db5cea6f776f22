"""Host-to-device hand-off of NF4 experts: pinned staging, async copies, reconstruction,
and the transfer scheduler."""
from .nf4_reconstruct import ReconstructedNF4Expert
from .nf4_transfer import transfer_staged_expert_to_gpu
from .pinned_memory import PinnedMemoryBudget
from .reusable_staging import ReusablePinnedStagingPool, StagingSlot
from .scheduler import EXECUTE_NEXT_PROFILE, TransferScheduler
from .types import (TransferDirection, TransferHandle, TransferPriority, TransferRequest,
                    TransferResult, TransferStatus)

__all__ = [
    "EXECUTE_NEXT_PROFILE", "PinnedMemoryBudget", "ReconstructedNF4Expert",
    "ReusablePinnedStagingPool", "StagingSlot", "TransferDirection", "TransferHandle",
    "TransferPriority", "TransferRequest", "TransferResult", "TransferScheduler",
    "TransferStatus", "transfer_staged_expert_to_gpu",
]
