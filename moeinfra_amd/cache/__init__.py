"""Two-tier expert residency cache."""
from .manager import CacheManager
from .types import CacheEntry, CacheStats, EvictionPolicy

__all__ = ["CacheEntry", "CacheManager", "CacheStats", "EvictionPolicy"]
