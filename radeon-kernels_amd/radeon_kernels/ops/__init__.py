"""Operators with a static-dispatch native path and a declared torch fallback."""

from radeon_kernels.ops.kv_cache import kv_cache_append, kv_cache_copy
from radeon_kernels.ops.paged_attention import paged_attention_decode
from radeon_kernels.ops.sdpa import sdpa

__all__ = ["kv_cache_append", "kv_cache_copy", "paged_attention_decode", "sdpa"]
