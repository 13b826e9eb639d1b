"""engine.cache (reference: engine/cache.py:4-57) -> the paged KV block allocator."""
from mycustomcudaengine_amd.engine.cache import KVCacheManager  # noqa: F401

__all__ = ["KVCacheManager"]
