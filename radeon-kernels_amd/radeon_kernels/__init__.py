"""MI355X (gfx950) paged-attention decode behind radeon-kernels' static-dispatch API.

``import radeon_kernels as rk`` exposes the same names the reference exports for this path
(src/radeon_kernels/__init__.py:3-34): ``paged_attention_decode``, the paged-cache operators around
it, ``kv_cache_append`` and ``kv_cache_copy``, the prefill step before it, ``sdpa``, and
``explain_last_dispatch`` / ``get_last_dispatch``.  Importing the package does not import torch.
"""

from radeon_kernels import ops
from radeon_kernels.ops.kv_cache import kv_cache_append, kv_cache_copy
from radeon_kernels.ops.paged_attention import paged_attention_decode
from radeon_kernels.ops.sdpa import sdpa
from radeon_kernels.runtime.explain import explain_last_dispatch, get_last_dispatch

__version__ = "1.0.0"

__all__ = [
    "__version__",
    "explain_last_dispatch",
    "get_last_dispatch",
    "kv_cache_append",
    "kv_cache_copy",
    "ops",
    "paged_attention_decode",
    "sdpa",
]
