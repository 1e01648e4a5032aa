"""Declared torch fallback of the paged KV-cache append.

Restates the reference fallback (src/radeon_kernels/ops/kv_cache/reference.py:6-20): the caches
are viewed as ``[num_blocks * block_size, kv_heads, head_dim]`` physical slots and token ``t``'s
K and V rows are written to slot ``slot_mapping[t]`` with ``index_copy_`` (slot = block *
block_size + offset).  The caches are updated in place and returned.

Slots must be in range and unique (contracts/kv_cache_append-1.0.json:19): ``index_copy_``
raises on an out-of-range slot.  The native kernel instead skips such tokens (as the reference's
own native kernel does, benchmarks/kv_cache/native_kv_cache.hip:42-45), because it cannot report an
error without a host synchronisation.
"""

from __future__ import annotations

from typing import Any


def kv_cache_append_reference(
    torch_module: Any,
    key: Any,
    value: Any,
    key_cache: Any,
    value_cache: Any,
    slot_mapping: Any,
) -> tuple[Any, Any]:
    slots = slot_mapping.to(dtype=torch_module.int64)
    rows = (-1, int(key_cache.shape[2]), int(key_cache.shape[3]))
    key_cache.view(rows).index_copy_(0, slots, key)
    value_cache.view(rows).index_copy_(0, slots, value)
    return key_cache, value_cache
