from radeon_kernels.ops.kv_cache.api import kv_cache_append

__all__ = ["kv_cache_append"]
