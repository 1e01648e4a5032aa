"""Declared torch fallbacks of the paged KV-cache operators.

``kv_cache_append_reference`` restates src/radeon_kernels/ops/kv_cache/reference.py:6-20: the caches
are viewed as ``[num_blocks * block_size, kv_heads, head_dim]`` physical slots and token ``t``'s
K and V rows are written to slot ``slot_mapping[t]`` with ``index_copy_`` (slot = block *
block_size + offset).

``kv_cache_copy_reference`` restates reference.py:23-38: every source block of ``block_mapping``
(column 0) is first gathered with ``index_select`` (a snapshot), then written to its destination
block (column 1) with ``index_copy_``.

Both update the caches in place and return them.  Indices must be in range (and destinations unique
and, for the copy, disjoint from the sources: contracts/kv_cache_append-1.0.json:19,
contracts/kv_cache_copy-1.0.json:17); torch raises on an out-of-range index.  The native kernels
instead skip such tokens or pairs (as the reference's own kernels do,
benchmarks/kv_cache/native_kv_cache.hip:44-46,72-74), because they cannot report an error without a
host synchronisation.
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


def kv_cache_copy_reference(
    torch_module: Any,
    key_cache: Any,
    value_cache: Any,
    block_mapping: Any,
) -> tuple[Any, Any]:
    pairs = block_mapping.to(dtype=torch_module.int64)
    sources, destinations = pairs[:, 0], pairs[:, 1]
    key_snapshot = key_cache.index_select(0, sources)
    value_snapshot = value_cache.index_select(0, sources)
    key_cache.index_copy_(0, destinations, key_snapshot)
    value_cache.index_copy_(0, destinations, value_snapshot)
    return key_cache, value_cache
