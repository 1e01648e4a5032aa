"""Operators with a static-dispatch native path and a declared torch fallback."""

from radeon_kernels.ops.kv_cache import kv_cache_append
from radeon_kernels.ops.paged_attention import paged_attention_decode

__all__ = ["kv_cache_append", "paged_attention_decode"]
