"""CPU tests of the public ``kv_cache_append`` contract with duck-typed tensors (no torch, no GPU).

Pins what the reference's unit tests pin for this operator (tests/test_llm_ops.py:193-224,357-383):
the 10-key dispatch signature, the native argument tuple, the ``torch/index_copy`` fallback label,
the validation messages, and that an implementation must return the cache tensors it was given.
"""

from __future__ import annotations

import pytest

from radeon_kernels.ops.kv_cache.api import _execute_append
from test_api import FakeTensor, FakeTorch


class Runtime:
    def __init__(self, result=None):
        self.result = result
        self.call = None

    def execute(self, **values):
        self.call = values
        return self.result


def append(key=(32, 8, 128), cache=(256, 16, 8, 128), slots=(32,), *, result=None, **overrides):
    key_cache = overrides.pop("key_cache", FakeTensor(cache))
    value_cache = overrides.pop("value_cache", FakeTensor(cache))
    runtime = Runtime((key_cache, value_cache) if result is None else result)
    key_tensor = key if isinstance(key, FakeTensor) else FakeTensor(key)
    tensors = dict(key=key_tensor, value=FakeTensor(key_tensor.shape), slot_mapping=FakeTensor(slots, dtype="int64"))
    tensors.update(overrides)
    out = _execute_append(tensors["key"], tensors["value"], key_cache, value_cache, tensors["slot_mapping"],
                          torch_module=FakeTorch(), runtime=runtime)
    return out, runtime.call, (key_cache, value_cache)


def test_signature_arguments_and_fallback_label():
    out, call, caches = append()
    assert out == caches
    assert call["operator"] == "kv_cache_append" and call["semantic_version"] == "1.0"
    assert call["signature"] == {
        "dtype": "fp16", "tokens": 32, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128,
        "index_dtype": "int64", "layout": "block_slot_head_dim", "contiguous": True, "requires_grad": False,
    }
    assert len(call["native_arguments"]) == 5 and call["native_arguments"][2] is caches[0]
    assert call["fallback_selected"] == "torch/index_copy"


@pytest.mark.parametrize(
    "kwargs, error, message",
    [
        (dict(slots=(1,)), ValueError, "one slot per token"),
        (dict(key=FakeTensor((2, 8, 128), contiguous=False), slots=(2,)), ValueError, "must be contiguous"),
        (dict(key=(32, 4, 128)), ValueError, r"\[tokens, kv_heads, head_dim\]"),
        (dict(value=FakeTensor((32, 8, 64))), ValueError, "key and value must have the same shape"),
        (dict(value_cache=FakeTensor((256, 16, 8, 64))), ValueError, "same shape"),
        (dict(slot_mapping=FakeTensor((32,), dtype="float16")), TypeError, "index tensors"),
        (dict(key=FakeTensor((32, 8, 128), dtype="float32")), TypeError, "torch.float16 and torch.bfloat16"),
        (dict(key_cache=FakeTensor((256, 16, 8, 128), dtype="bfloat16")), TypeError, "same dtype"),
        (dict(key=FakeTensor((32, 8, 128), requires_grad=True)), ValueError, "inference-only"),
        (dict(key=FakeTensor((32, 8, 128), is_cuda=False)), ValueError, "visible ROCm GPU"),
    ],
)
def test_validation_messages(kwargs, error, message):
    with pytest.raises(error, match=message):
        append(**kwargs)


def test_implementation_must_return_the_given_caches():
    with pytest.raises(RuntimeError, match="must return key_cache and value_cache"):
        append(result="not a pair")

    class Other(FakeTensor):
        def data_ptr(self):
            return 1

    class Same(FakeTensor):
        def data_ptr(self):
            return 2

    with pytest.raises(RuntimeError, match="must return the input cache tensors"):
        append(result=(Other((256, 16, 8, 128)), Other((256, 16, 8, 128))),
               key_cache=Same((256, 16, 8, 128)), value_cache=Same((256, 16, 8, 128)))


# ---------------------------------------------------------------------------------------------
from radeon_kernels.ops.kv_cache.api import _execute_copy  # noqa: E402


def copy(cache=(128, 32, 32, 128), mapping=(8, 2), *, dtype="bfloat16", index="int32", **overrides):
    key_cache = overrides.pop("key_cache", FakeTensor(cache, dtype=dtype))
    value_cache = overrides.pop("value_cache", FakeTensor(cache, dtype=dtype))
    block_mapping = overrides.pop("block_mapping", FakeTensor(mapping, dtype=index))
    runtime = Runtime((key_cache, value_cache))
    out = _execute_copy(key_cache, value_cache, block_mapping, torch_module=FakeTorch(), runtime=runtime)
    return out, runtime.call


def test_copy_signature_matches_the_reference_unit_test():
    _, call = copy()
    assert call["operator"] == "kv_cache_copy"
    assert call["signature"] == {
        "dtype": "bf16", "pairs": 8, "num_blocks": 128, "block_size": 32, "kv_heads": 32, "head_dim": 128,
        "index_dtype": "int32", "layout": "block_slot_head_dim", "contiguous": True, "requires_grad": False,
    }
    assert len(call["native_arguments"]) == 3 and call["fallback_selected"] == "torch/index_copy"


@pytest.mark.parametrize(
    "kwargs, error, message",
    [
        (dict(block_mapping=FakeTensor((1, 2))), TypeError, "index tensors"),
        (dict(mapping=(4, 3)), ValueError, r"shape \[pairs, 2\]"),
        (dict(block_mapping=FakeTensor((4,), dtype="int64")), ValueError, "rank 2"),
        (dict(value_cache=FakeTensor((128, 32, 32, 64), dtype="bfloat16")), ValueError, "same shape"),
        (dict(key_cache=FakeTensor((128, 32, 32, 128), dtype="bfloat16", contiguous=False)), ValueError,
         "must be contiguous"),
    ],
)
def test_copy_validation_messages(kwargs, error, message):
    with pytest.raises(error, match=message):
        copy(**kwargs)
