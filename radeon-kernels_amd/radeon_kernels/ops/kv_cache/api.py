"""Public paged KV-cache operators.

``kv_cache_append`` writes each new token's K/V rows into its cache slot; ``kv_cache_copy`` copies
whole cache blocks (a beam fork).  Mirrors src/radeon_kernels/ops/kv_cache/api.py:25-215 in the
reference: the same checks in the same order with the same messages, the same 10-key dispatch
signatures, ``native_arguments`` = (key, value, key_cache, value_cache, slot_mapping) and
(key_cache, value_cache, block_mapping), the fallback label ``torch/index_copy``, and the rule that
an implementation must hand back the very cache tensors it was given (it writes them in place).
"""

from __future__ import annotations

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
from radeon_kernels.ops.kv_cache.reference import kv_cache_append_reference, kv_cache_copy_reference

APPEND = "kv_cache_append"
COPY = "kv_cache_copy"
SEMANTIC_VERSION = "1.0"
LAYOUT = "block_slot_head_dim"
FALLBACK_SELECTED = "torch/index_copy"


def _torch() -> Any:
    return torch_runtime("kv_cache")


def _cache_shape(torch_module: Any, key_cache: Any, value_cache: Any, operator: str) -> tuple[int, int, int, int]:
    """Validate a K/V cache pair; returns (num_blocks, block_size, kv_heads, head_dim)."""

    validate_tensor(torch_module, key_cache, name="key_cache", rank=4, operator=operator)
    validate_tensor(torch_module, value_cache, name="value_cache", rank=4, operator=operator)
    validate_same(operator, key_cache, value_cache, first_name="key_cache", second_name="value_cache")
    if tuple(key_cache.shape) != tuple(value_cache.shape):
        raise ValueError(f"{operator} key_cache and value_cache must have the same shape")
    shape = tuple(int(size) for size in key_cache.shape)
    if min(shape) <= 0:
        raise ValueError(f"{operator} cache dimensions must be positive")
    return shape


def _returned_caches(operator: str, result: Any, key_cache: Any, value_cache: Any) -> tuple[Any, Any]:
    """An implementation returns (key_cache, value_cache): the same storage it was given."""

    if not isinstance(result, (tuple, list)) or len(result) != 2:
        raise RuntimeError(f"{operator} implementation must return key_cache and value_cache")
    for returned, given in zip(result, (key_cache, value_cache)):
        if hasattr(returned, "data_ptr") and returned.data_ptr() != given.data_ptr():
            raise RuntimeError(f"{operator} implementation must return the input cache tensors")
    return result[0], result[1]


def _execute_append(
    key: Any,
    value: Any,
    key_cache: Any,
    value_cache: Any,
    slot_mapping: Any,
    *,
    torch_module: Any,
    runtime: OperatorRuntime,
    plan_key: Any = None,
) -> tuple[Any, Any]:
    op = APPEND
    validate_tensor(torch_module, key, name="key", rank=3, operator=op)
    validate_tensor(torch_module, value, name="value", rank=3, operator=op)
    validate_same(op, key, value, first_name="key", second_name="value")
    if tuple(key.shape) != tuple(value.shape):
        raise ValueError(f"{op} key and value must have the same shape")
    num_blocks, block_size, kv_heads, head_dim = _cache_shape(torch_module, key_cache, value_cache, op)
    validate_same(op, key, key_cache, first_name="key", second_name="key_cache")
    validate_index_tensor(torch_module, slot_mapping, name="slot_mapping", rank=1, operator=op)
    if slot_mapping.device != key.device:
        raise ValueError(f"{op} slot_mapping must use the same device as key")
    tokens = int(key.shape[0])
    if tokens <= 0 or int(key.shape[1]) != kv_heads or int(key.shape[2]) != head_dim:
        raise ValueError(f"{op} key/value shape must be [tokens, kv_heads, head_dim]")
    if tuple(slot_mapping.shape) != (tokens,):
        raise ValueError(f"{op} slot_mapping must contain one slot per token")
    context = tensor_context(torch_module, op, key, value, key_cache, value_cache, slot_mapping)
    if not context.contiguous:
        raise ValueError(f"{op} paged-layout tensors must be contiguous")
    if context.requires_grad:
        raise ValueError(f"{op} is inference-only and does not support autograd")
    signature = {
        "dtype": context.dtype,
        "tokens": tokens,
        "num_blocks": num_blocks,
        "block_size": block_size,
        "kv_heads": kv_heads,
        "head_dim": head_dim,
        "index_dtype": index_dtype_name(torch_module, slot_mapping.dtype, op),
        "layout": LAYOUT,
        "contiguous": context.contiguous,
        "requires_grad": False,
    }
    result = runtime.execute(
        operator=op,
        semantic_version=SEMANTIC_VERSION,
        signature=signature,
        device_index=context.device_index,
        torch_module=torch_module,
        native_arguments=(key, value, key_cache, value_cache, slot_mapping),
        fallback=lambda: kv_cache_append_reference(torch_module, key, value, key_cache, value_cache, slot_mapping),
        fallback_selected=FALLBACK_SELECTED,
        plan_key=plan_key,
    )
    return _returned_caches(op, result, key_cache, value_cache)


def _dispatch_append(key: Any, value: Any, key_cache: Any, value_cache: Any, slot_mapping: Any, *,
                     torch_module: Any, runtime: OperatorRuntime) -> tuple[Any, Any]:
    """A call shape validated before runs its kept plan; any other call takes ``_execute_append``."""

    plan_key = call_key(torch_module, APPEND, (key, value, key_cache, value_cache, slot_mapping))
    plan = runtime.plan_for(plan_key)
    if plan is None:
        return _execute_append(key, value, key_cache, value_cache, slot_mapping, torch_module=torch_module,
                               runtime=runtime, plan_key=plan_key)
    result = runtime.run_plan(
        plan, (key, value, key_cache, value_cache, slot_mapping),
        lambda: kv_cache_append_reference(torch_module, key, value, key_cache, value_cache, slot_mapping),
        FALLBACK_SELECTED,
    )
    return _returned_caches(APPEND, result, key_cache, value_cache)


def kv_cache_append(key: Any, value: Any, key_cache: Any, value_cache: Any, slot_mapping: Any) -> tuple[Any, Any]:
    """Write token ``t``'s K/V rows ``[kv_heads, head_dim]`` into physical slot ``slot_mapping[t]``.

    Shapes: key/value ``[tokens, kv_heads, head_dim]``; caches ``[num_blocks, block_size, kv_heads,
    head_dim]``; slot_mapping ``[tokens]`` (slot = block * block_size + offset, in range and
    unique).  Updates the caches in place and returns them.
    """

    return _dispatch_append(key, value, key_cache, value_cache, slot_mapping, torch_module=_torch(),
                            runtime=default_operator_runtime())


def _execute_copy(
    key_cache: Any,
    value_cache: Any,
    block_mapping: Any,
    *,
    torch_module: Any,
    runtime: OperatorRuntime,
    plan_key: Any = None,
) -> tuple[Any, Any]:
    op = COPY
    num_blocks, block_size, kv_heads, head_dim = _cache_shape(torch_module, key_cache, value_cache, op)
    validate_index_tensor(torch_module, block_mapping, name="block_mapping", rank=2, operator=op)
    if block_mapping.device != key_cache.device:
        raise ValueError(f"{op} block_mapping must use the same device as key_cache")
    if int(block_mapping.shape[1]) != 2 or int(block_mapping.shape[0]) <= 0:
        raise ValueError(f"{op} block_mapping must have shape [pairs, 2]")
    context = tensor_context(torch_module, op, key_cache, value_cache, block_mapping)
    if not context.contiguous:
        raise ValueError(f"{op} paged-layout tensors must be contiguous")
    if context.requires_grad:
        raise ValueError(f"{op} is inference-only and does not support autograd")
    signature = {
        "dtype": context.dtype,
        "pairs": int(block_mapping.shape[0]),
        "num_blocks": num_blocks,
        "block_size": block_size,
        "kv_heads": kv_heads,
        "head_dim": head_dim,
        "index_dtype": index_dtype_name(torch_module, block_mapping.dtype, op),
        "layout": LAYOUT,
        "contiguous": context.contiguous,
        "requires_grad": False,
    }
    result = runtime.execute(
        operator=op,
        semantic_version=SEMANTIC_VERSION,
        signature=signature,
        device_index=context.device_index,
        torch_module=torch_module,
        native_arguments=(key_cache, value_cache, block_mapping),
        fallback=lambda: kv_cache_copy_reference(torch_module, key_cache, value_cache, block_mapping),
        fallback_selected=FALLBACK_SELECTED,
        plan_key=plan_key,
    )
    return _returned_caches(op, result, key_cache, value_cache)


def _dispatch_copy(key_cache: Any, value_cache: Any, block_mapping: Any, *, torch_module: Any,
                   runtime: OperatorRuntime) -> tuple[Any, Any]:
    """A call shape validated before runs its kept plan; any other call takes ``_execute_copy``."""

    plan_key = call_key(torch_module, COPY, (key_cache, value_cache, block_mapping))
    plan = runtime.plan_for(plan_key)
    if plan is None:
        return _execute_copy(key_cache, value_cache, block_mapping, torch_module=torch_module, runtime=runtime,
                             plan_key=plan_key)
    result = runtime.run_plan(
        plan, (key_cache, value_cache, block_mapping),
        lambda: kv_cache_copy_reference(torch_module, key_cache, value_cache, block_mapping),
        FALLBACK_SELECTED,
    )
    return _returned_caches(COPY, result, key_cache, value_cache)


def kv_cache_copy(key_cache: Any, value_cache: Any, block_mapping: Any) -> tuple[Any, Any]:
    """Copy whole cache blocks: block ``block_mapping[i, 0]`` to block ``block_mapping[i, 1]``.

    ``block_mapping`` is ``[pairs, 2]`` (source, destination); destinations must be in range, unique
    and disjoint from the sources, so every copy reads the pre-call contents.  Updates the caches in
    place and returns them.
    """

    return _dispatch_copy(key_cache, value_cache, block_mapping, torch_module=_torch(),
                          runtime=default_operator_runtime())
