"""Operators with a static-dispatch native path and a declared torch fallback."""

from radeon_kernels.ops.paged_attention import paged_attention_decode

__all__ = ["paged_attention_decode"]
