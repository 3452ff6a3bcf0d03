from .paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState
