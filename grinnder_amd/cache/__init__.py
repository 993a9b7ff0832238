"""Host-memory cache policy of the storage tier."""

from grinnder_amd.cache.partition_cache import CacheMemoryPlan, PartitionCache

__all__ = ["CacheMemoryPlan", "PartitionCache"]
