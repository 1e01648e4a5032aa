from radeon_kernels.ops.kv_cache.api import kv_cache_append, kv_cache_copy

__all__ = ["kv_cache_append", "kv_cache_copy"]
