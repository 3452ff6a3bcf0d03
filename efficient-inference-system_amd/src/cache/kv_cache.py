"""Legacy aliases, as src/cache/kv_cache.py:1-6 of the reference."""
from src.cache.paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState

KVCache = PagedKVCacheState
BatchedKVCache = BatchedPagedKVCache

__all__ = ["KVCache", "BatchedKVCache", "LayerBlockPool", "PagedKVCacheState"]
