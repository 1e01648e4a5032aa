"""CPU oracle for the paged KV-cache append and block copy -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only as
the checker (or the timed CPU baseline).  The product path (``radeon_kernels``) never imports it.

Restates the reference fallback (src/radeon_kernels/ops/kv_cache/reference.py:6-20): the caches
viewed as ``[num_blocks * block_size, kv_heads, head_dim]`` slots; token ``t``'s K and V rows are
written to slot ``slot_mapping[t]`` (block ``slot // block_size``, offset ``slot % block_size``).

``append_numpy``       numpy on copies of the caches, any element type, whole-row assignment.
``append_bruteforce``  pure-Python loops element by element (tiny shapes only).

Both skip a slot outside ``[0, num_blocks * block_size)`` instead of raising as ``index_copy_``
does: that is the native kernel's documented behaviour (the reference's own kernel does the same,
benchmarks/kv_cache/native_kv_cache.hip:44-46), and the contract requires in-range slots anyway
(contracts/kv_cache_append-1.0.json:19).  With duplicate slots (outside the contract) the last
token wins here; the kernel gives no order guarantee.

``copy_numpy`` restates the block copy (reference.py:23-38): a snapshot of every source block is
taken first, then written to its destination, so overlapping mappings (outside the contract) still
read pre-call contents; a pair with a block id outside ``[0, num_blocks)`` is skipped, as the
native kernels do (native_kv_cache.hip:72-74).

Pinning (``tests/test_kv_oracle.py``): against torch's ``index_copy_`` on every reference case,
against the brute force on small shapes, and by invariants (untouched slots unchanged, gathering
the written slots returns the input rows, block/offset addressing), with planted mistakes that
each fail one of these checks.
"""

from __future__ import annotations

from typing import Any

import numpy as np


def append_numpy(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                 slot_mapping: Any) -> tuple[np.ndarray, np.ndarray]:
    """New (key_cache, value_cache) arrays with each token's rows written to its slot."""

    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    capacity = num_blocks * block_size
    k_out = key_cache.copy().reshape(capacity, kv_heads, head_dim)
    v_out = value_cache.copy().reshape(capacity, kv_heads, head_dim)
    for token, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64).tolist()):
        if 0 <= slot < capacity:
            k_out[slot] = key[token]
            v_out[slot] = value[token]
    return k_out.reshape(key_cache.shape), v_out.reshape(value_cache.shape)


def append_bruteforce(key, value, key_cache, value_cache, slot_mapping):
    """Element-by-element restatement with explicit block/offset addressing (tiny shapes)."""

    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    k_out, v_out = key_cache.copy(), value_cache.copy()
    for token in range(key.shape[0]):
        slot = int(slot_mapping[token])
        if not 0 <= slot < num_blocks * block_size:
            continue
        block, offset = slot // block_size, slot % block_size
        for h in range(kv_heads):
            for d in range(head_dim):
                k_out[block, offset, h, d] = key[token, h, d]
                v_out[block, offset, h, d] = value[token, h, d]
    return k_out, v_out


def as_bits(tensor: Any) -> np.ndarray:
    """The 16-bit patterns of an fp16/bf16 torch tensor (exact comparison without conversion)."""

    import torch

    return tensor.detach().cpu().contiguous().view(torch.int16).numpy()


def append_inplace_torch(torch: Any, key: Any, value: Any, key_cache: Any, value_cache: Any,
                         slot_mapping: Any) -> None:
    """The reference fallback's own steps (reference.py:16-19) on CPU tensors, in place: the CPU
    path the gfx950 kernel is timed beside.  In-range unique slots only (``index_copy_`` raises
    otherwise)."""

    slots = slot_mapping.to(dtype=torch.int64)
    rows = (-1, int(key_cache.shape[2]), int(key_cache.shape[3]))
    key_cache.view(rows).index_copy_(0, slots, key)
    value_cache.view(rows).index_copy_(0, slots, value)


def copy_numpy(key_cache: np.ndarray, value_cache: np.ndarray, block_mapping: Any) -> tuple[np.ndarray, np.ndarray]:
    """New (key_cache, value_cache) arrays with each source block copied to its destination block."""

    num_blocks = key_cache.shape[0]
    pairs = [(int(s), int(d)) for s, d in np.asarray(block_mapping, dtype=np.int64).tolist()]
    pairs = [(s, d) for s, d in pairs if 0 <= s < num_blocks and 0 <= d < num_blocks]
    k_out, v_out = key_cache.copy(), value_cache.copy()
    k_snap = [key_cache[s].copy() for s, _ in pairs]
    v_snap = [value_cache[s].copy() for s, _ in pairs]
    for (_, d), k_block, v_block in zip(pairs, k_snap, v_snap):
        k_out[d] = k_block
        v_out[d] = v_block
    return k_out, v_out


def copy_inplace_torch(torch: Any, key_cache: Any, value_cache: Any, block_mapping: Any) -> None:
    """The reference fallback's own steps (reference.py:30-37) on CPU tensors, in place: the CPU path
    the gfx950 copy kernel is timed beside."""

    mapping = block_mapping.to(dtype=torch.int64)
    k = key_cache.index_select(0, mapping[:, 0])
    v = value_cache.index_select(0, mapping[:, 0])
    key_cache.index_copy_(0, mapping[:, 1], k)
    value_cache.index_copy_(0, mapping[:, 1], v)
