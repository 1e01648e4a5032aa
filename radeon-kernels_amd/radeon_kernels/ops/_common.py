"""Tensor validation shared by operators.

Names, order of checks and messages follow src/radeon_kernels/ops/_common.py:16-109 in the
reference (callers pin the messages).  Torch is imported lazily so ``import radeon_kernels`` never
imports it; tests pass duck-typed fakes as ``torch_module``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True)
class TensorContext:
    dtype: str
    device_index: int
    contiguous: bool
    requires_grad: bool


def torch_runtime(operator: str) -> Any:
    try:
        import torch
    except ImportError as error:
        raise RuntimeError(f"{operator} requires a ROCm PyTorch installation") from error
    return torch


def dtype_name(torch_module: Any, dtype: Any, operator: str) -> str:
    names = ((torch_module.float16, "fp16"), (torch_module.bfloat16, "bf16"))
    for candidate, name in names:
        if dtype == candidate:
            return name
    raise TypeError(f"{operator} supports torch.float16 and torch.bfloat16 tensors")


def index_dtype_name(torch_module: Any, dtype: Any, operator: str) -> str:
    names = ((torch_module.int32, "int32"), (torch_module.int64, "int64"))
    for candidate, name in names:
        if dtype == candidate:
            return name
    raise TypeError(f"{operator} index tensors must use torch.int32 or torch.int64")


def _check_tensor_common(torch_module: Any, tensor: Any, name: str, rank: int, operator: str) -> None:
    if not isinstance(tensor, getattr(torch_module, "Tensor", ())):
        raise TypeError(f"{operator} {name} must be a PyTorch tensor")
    if tensor.dim() != rank:
        raise ValueError(f"{operator} {name} must be rank {rank}")
    if not tensor.is_cuda:
        raise ValueError(f"{operator} {name} must be on a visible ROCm GPU")


def validate_tensor(torch_module: Any, tensor: Any, *, name: str, rank: int, operator: str) -> None:
    _check_tensor_common(torch_module, tensor, name, rank, operator)
    dtype_name(torch_module, tensor.dtype, operator)


def validate_index_tensor(torch_module: Any, tensor: Any, *, name: str, rank: int, operator: str) -> None:
    _check_tensor_common(torch_module, tensor, name, rank, operator)
    index_dtype_name(torch_module, tensor.dtype, operator)


def validate_same(operator: str, first: Any, second: Any, *, first_name: str, second_name: str) -> None:
    if first.device != second.device:
        raise ValueError(f"{operator} {first_name} and {second_name} must use the same device")
    if first.dtype != second.dtype:
        raise TypeError(f"{operator} {first_name} and {second_name} must use the same dtype")


def tensor_context(torch_module: Any, operator: str, *tensors: Any) -> TensorContext:
    head = tensors[0]
    index = getattr(head.device, "index", None)
    if index is None:
        index = int(torch_module.cuda.current_device())
    return TensorContext(
        dtype=dtype_name(torch_module, head.dtype, operator),
        device_index=int(index),
        contiguous=all(bool(item.is_contiguous()) for item in tensors),
        requires_grad=any(bool(item.requires_grad) for item in tensors),
    )


def call_key(torch_module: Any, operator: str, tensors: tuple[Any, ...], extra: Any = None) -> tuple | None:
    """Exact, hashable description of everything validation reads from a call, or None.

    Per tensor: its type (the ``isinstance`` check), dtype, device, ``is_cuda``, shape (which fixes
    ``dim()``), contiguity and ``requires_grad``; plus the operator, the torch module the dtypes are
    compared with, and ``extra`` (the call's non-tensor arguments).  Two calls with equal keys pass
    or fail every check identically and build the same dispatch signature, which is what lets the
    operator runtime reuse a call plan.  Anything unusual about the inputs (a missing attribute, a
    raising property) gives None, and the call then takes the fully validated path.
    """

    try:
        key = [operator, torch_module, extra]
        for tensor in tensors:
            key += (type(tensor), tensor.dtype, tensor.device, tensor.is_cuda, tensor.shape,
                    tensor.is_contiguous(), tensor.requires_grad)
        return tuple(key)
    except Exception:
        return None
