"""Declared torch fallback of paged-attention decode (runs wherever the tensors live).

This is the operator's general path for requests no dispatch entry covers, and the behaviour the
native kernels are held to.  It restates the reference fallback
(src/radeon_kernels/ops/paged_attention/reference.py:7-47) step for step, with the same torch
operations in the same order, so that on the same torch build it returns bit-identical results:

1. positions ``0 .. max_blocks*block_size - 1``; logical block ``pos // block_size`` and offset
   ``pos % block_size``; physical slot ``block_tables[b, pos // BS] * BS + pos % BS``;
2. gather K and V rows of every slot into ``[B, max_ctx, Hkv, D]``;
3. expand KV heads to query heads with ``index_select`` on ``h // (Hq / Hkv)``, convert to fp32;
4. scores ``einsum("bhd,bthd->bht")`` times ``scale``; positions ``>= context_length`` -> ``-inf``;
5. fp32 softmax over positions; output ``einsum("bht,bthd->bhd")``; cast to the query dtype.

It is not the oracle the kernels are tested against (that lives in ``oracle/``, outside the
package); it is the product's own fallback.
"""

from __future__ import annotations

import math
from typing import Any


def paged_attention_decode_reference(
    torch_module: Any,
    query: Any,
    key_cache: Any,
    value_cache: Any,
    block_tables: Any,
    context_lengths: Any,
    scale: float | None = None,
) -> Any:
    """Evaluate one decode query per sequence against a paged K/V cache."""

    torch = torch_module
    batch, query_heads, head_dim = (int(size) for size in query.shape)
    _, block_size, kv_heads, _ = (int(size) for size in key_cache.shape)
    max_context = int(block_tables.shape[1]) * block_size
    device = query.device

    positions = torch.arange(max_context, device=device)
    logical = positions // block_size
    offsets = positions % block_size
    slots = block_tables.to(dtype=torch.int64).index_select(1, logical) * block_size + offsets.unsqueeze(0)
    flat_slots = slots.reshape(-1)

    rows = (-1, kv_heads, head_dim)
    keys = key_cache.view(rows).index_select(0, flat_slots).view(batch, max_context, kv_heads, head_dim)
    values = value_cache.view(rows).index_select(0, flat_slots).view(batch, max_context, kv_heads, head_dim)

    head_map = torch.arange(query_heads, device=device) // (query_heads // kv_heads)
    keys = keys.index_select(2, head_map).float()
    values = values.index_select(2, head_map).float()

    factor = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
    scores = torch.einsum("bhd,bthd->bht", query.float(), keys) * factor
    valid = positions.unsqueeze(0) < context_lengths.to(dtype=torch.int64).unsqueeze(1)
    scores = scores.masked_fill(~valid.unsqueeze(1), float("-inf"))
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32)
    return torch.einsum("bht,bthd->bhd", weights, values).to(dtype=query.dtype)
