"""Public paged-attention decode operator.

Contract of src/radeon_kernels/ops/paged_attention/api.py:27-157 in the reference, kept exactly so
this package is a drop-in for ``rk.paged_attention_decode``: the same validation order and
messages, the same 13-key dispatch signature, the same native argument tuple
``(query, key_cache, value_cache, block_tables, context_lengths, scale: float)`` and the same
fallback label ``"torch/paged_attention"``.  On gfx950 the signature selects an entry of
``radeon_kernels/dispatch/paged_attention_decode-1.0.json`` whose winner is the HIP library's
``decode_mfma`` entrypoint; elsewhere (or for shapes outside every entry) the declared torch
fallback runs.
"""

from __future__ import annotations

import math
from typing import Any

from radeon_kernels.ops._common import (
    call_key,
    index_dtype_name,
    tensor_context,
    torch_runtime,
    validate_index_tensor,
    validate_same,
    validate_tensor,
)
from radeon_kernels.ops._runtime import OperatorRuntime, default_operator_runtime
from radeon_kernels.ops.paged_attention.reference import paged_attention_decode_reference

OPERATOR = "paged_attention_decode"
SEMANTIC_VERSION = "1.0"
CACHE_LAYOUT = "block_slot_head_dim"
SUPPORTED_HEAD_DIMS = (64, 128, 256)
FALLBACK_SELECTED = "torch/paged_attention"


def _torch() -> Any:
    return torch_runtime(OPERATOR)


def _normalize_scale(scale: float | None, head_dim: int) -> tuple[float, str]:
    """``None`` -> (1/sqrt(head_dim), "default"); a finite positive number -> (float, "explicit")."""

    if scale is None:
        return 1.0 / math.sqrt(head_dim), "default"
    if isinstance(scale, bool) or not isinstance(scale, (int, float)):
        raise TypeError(f"{OPERATOR} scale must be a number")
    value = float(scale)
    if not (math.isfinite(value) and value > 0):
        raise ValueError(f"{OPERATOR} scale must be positive and finite")
    return value, "explicit"


def _execute(
    query: Any,
    key_cache: Any,
    value_cache: Any,
    block_tables: Any,
    context_lengths: Any,
    scale: float | None = None,
    *,
    torch_module: Any,
    runtime: OperatorRuntime,
    plan_key: Any = None,
) -> Any:
    op = OPERATOR
    validate_tensor(torch_module, query, name="query", rank=3, operator=op)
    validate_tensor(torch_module, key_cache, name="key_cache", rank=4, operator=op)
    validate_tensor(torch_module, value_cache, name="value_cache", rank=4, operator=op)
    validate_same(op, query, key_cache, first_name="query", second_name="key_cache")
    validate_same(op, key_cache, value_cache, first_name="key_cache", second_name="value_cache")
    if tuple(key_cache.shape) != tuple(value_cache.shape):
        raise ValueError(f"{op} key_cache and value_cache must have the same shape")
    validate_index_tensor(torch_module, block_tables, name="block_tables", rank=2, operator=op)
    validate_index_tensor(torch_module, context_lengths, name="context_lengths", rank=1, operator=op)
    if block_tables.device != query.device or context_lengths.device != query.device:
        raise ValueError(f"{op} index tensors must use the same device as query")
    if block_tables.dtype != context_lengths.dtype:
        raise TypeError(f"{op} block_tables and context_lengths must use the same dtype")

    batch, query_heads, head_dim = (int(size) for size in query.shape)
    num_blocks, block_size, kv_heads, cache_head_dim = (int(size) for size in key_cache.shape)
    if min(batch, query_heads, num_blocks, block_size, kv_heads) <= 0:
        raise ValueError(f"{op} tensor dimensions must be positive")
    if head_dim != cache_head_dim or head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{op} head_dim must match cache and be one of 64, 128, 256")
    if query_heads % kv_heads != 0:
        raise ValueError(f"{op} query_heads must be divisible by kv_heads")
    max_blocks = int(block_tables.shape[1])
    if int(block_tables.shape[0]) != batch or max_blocks <= 0:
        raise ValueError(f"{op} block_tables must have shape [batch, max_blocks]")
    if tuple(context_lengths.shape) != (batch,):
        raise ValueError(f"{op} context_lengths must contain one length per sequence")
    context = tensor_context(torch_module, op, query, key_cache, value_cache, block_tables, context_lengths)
    if not context.contiguous:
        raise ValueError(f"{op} inputs must be contiguous")
    if context.requires_grad:
        raise ValueError(f"{op} is inference-only and does not support autograd")
    normalized_scale, scale_mode = _normalize_scale(scale, head_dim)
    signature = {
        "dtype": context.dtype,
        "batch": batch,
        "query_heads": query_heads,
        "kv_heads": kv_heads,
        "head_dim": head_dim,
        "num_blocks": num_blocks,
        "block_size": block_size,
        "max_blocks_per_sequence": max_blocks,
        "index_dtype": index_dtype_name(torch_module, block_tables.dtype, op),
        "cache_layout": CACHE_LAYOUT,
        "scale_mode": scale_mode,
        "contiguous": True,
        "requires_grad": False,
    }
    arguments = (query, key_cache, value_cache, block_tables, context_lengths, normalized_scale)
    return runtime.execute(
        operator=op,
        semantic_version=SEMANTIC_VERSION,
        signature=signature,
        device_index=context.device_index,
        torch_module=torch_module,
        native_arguments=arguments,
        fallback=lambda: paged_attention_decode_reference(torch_module, *arguments),
        fallback_selected=FALLBACK_SELECTED,
        plan_key=plan_key,
    )


def _dispatch(
    query: Any,
    key_cache: Any,
    value_cache: Any,
    block_tables: Any,
    context_lengths: Any,
    scale: float | None,
    *,
    torch_module: Any,
    runtime: OperatorRuntime,
) -> Any:
    """A call shape validated before runs its kept plan; any other call takes ``_execute``."""

    # Only None and plain floats join the key: any other scale (int, bool, numpy) is validated.
    key = call_key(torch_module, OPERATOR, (query, key_cache, value_cache, block_tables, context_lengths),
                   scale) if scale is None or type(scale) is float else None
    plan = runtime.plan_for(key)
    if plan is not None:  # an equal call passed validation, so query is [B, Hq, D] and scale is valid
        normalized = 1.0 / math.sqrt(query.shape[2]) if scale is None else scale
        arguments = (query, key_cache, value_cache, block_tables, context_lengths, normalized)
        return runtime.run_plan(plan, arguments, lambda: paged_attention_decode_reference(torch_module, *arguments),
                                FALLBACK_SELECTED)
    return _execute(query, key_cache, value_cache, block_tables, context_lengths, scale,
                    torch_module=torch_module, runtime=runtime, plan_key=key)


def paged_attention_decode(
    query: Any,
    key_cache: Any,
    value_cache: Any,
    block_tables: Any,
    context_lengths: Any,
    scale: float | None = None,
) -> Any:
    """Attend one query token per sequence over a paged K/V cache.

    Shapes: query ``[B, Hq, D]``; key/value cache ``[num_blocks, block_size, Hkv, D]``;
    block_tables ``[B, max_blocks]``; context_lengths ``[B]``.  Returns a new ``[B, Hq, D]`` tensor
    in the query dtype.  ``scale`` defaults to ``1/sqrt(D)``.
    """

    return _dispatch(
        query,
        key_cache,
        value_cache,
        block_tables,
        context_lengths,
        scale,
        torch_module=_torch(),
        runtime=default_operator_runtime(),
    )
