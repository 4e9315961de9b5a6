"""nanoslg_amd — the KV-cache hot path of nanoslg, built for MI355X (gfx950).

Drop-in for nanoslg/kv_cache.py: ``create_cache_manager``, ``KVCacheConfig``,
``CacheContext``, ``KVCacheManager`` and the paged / contiguous backends, on
hand-written HIP kernels in libnslg_kv.so (C ABI: include/nslg_kv.h).
"""
__version__ = "0.1.0"

from .kv_cache import (  # noqa: F401
    CacheContext,
    ContiguousCacheContext,
    ContiguousKVCache,
    KVCacheConfig,
    KVCacheManager,
    PagedCacheContext,
    PagedKVCache,
    PagePool,
    RadixTree,
    attention_forward,
    create_cache_manager,
)
