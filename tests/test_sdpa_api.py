"""CPU tests of the public ``sdpa`` contract with duck-typed tensors (no torch, no GPU).

Pins what the reference's unit tests pin for this operator (tests/test_llm_ops.py:280-307,404-411):
the 11-key dispatch signature of a causal GQA call, the native argument tuple with the default
scale, the ``torch/scaled_dot_product_attention`` fallback label, and the validation messages of
src/radeon_kernels/ops/sdpa/api.py:37-77 in their order.
"""

from __future__ import annotations

import pytest

import radeon_kernels as rk
from radeon_kernels.ops.sdpa.api import _execute
from test_api import CaptureRuntime, FakeTensor, FakeTorch


def run(q=(2, 32, 256, 128), k=(2, 8, 256, 128), v=None, causal=True, scale=None, **overrides):
    tensors = {"query": q if isinstance(q, FakeTensor) else FakeTensor(q),
               "key": k if isinstance(k, FakeTensor) else FakeTensor(k)}
    tensors["value"] = v if isinstance(v, FakeTensor) else FakeTensor(v or tensors["key"].shape)
    tensors.update(overrides)
    runtime = CaptureRuntime("attended")
    result = _execute(tensors["query"], tensors["key"], tensors["value"], causal, scale, torch_module=FakeTorch(),
                      runtime=runtime)
    return result, runtime.call


def test_causal_gqa_signature_native_arguments_and_fallback_label():
    result, call = run()
    assert result == "attended" and call["operator"] == "sdpa" and call["semantic_version"] == "1.0"
    assert call["signature"] == {
        "dtype": "fp16", "batch": 2, "query_heads": 32, "kv_heads": 8, "sequence": 256, "head_dim": 128,
        "layout": "batch_head_sequence_dim", "attention_mode": "causal", "scale_mode": "default",
        "contiguous": True, "requires_grad": False,
    }
    assert len(call["native_arguments"]) == 5 and call["native_arguments"][3] is True
    assert call["native_arguments"][4] == pytest.approx(128 ** -0.5)
    assert call["fallback_selected"] == "torch/scaled_dot_product_attention"
    _, call = run(causal=False, scale=0.25)
    assert call["signature"]["attention_mode"] == "noncausal" and call["signature"]["scale_mode"] == "explicit"
    assert call["native_arguments"][4] == 0.25


@pytest.mark.parametrize("kwargs, error, message", [
    (dict(q=(1, 8, 64, 128), k=(1, 2, 128, 128)), ValueError, "equal query and KV sequence"),
    (dict(q=(1, 8, 64)), ValueError, "query must be rank 4"),
    (dict(q=FakeTensor((1, 8, 64, 128), dtype="float32")), TypeError, "float16 and torch.bfloat16"),
    (dict(k=FakeTensor((2, 8, 256, 128), dtype="bfloat16")), TypeError, "same dtype"),
    (dict(causal=1), TypeError, "is_causal must be bool"),
    (dict(v=FakeTensor((2, 8, 256, 64))), ValueError, "key and value must have the same shape"),
    (dict(q=(2, 32, 0, 128), k=(2, 8, 0, 128)), ValueError, "dimensions must be positive"),
    (dict(k=(1, 8, 256, 128)), ValueError, "share the batch dimension"),
    (dict(q=(2, 32, 256, 96), k=(2, 8, 256, 96)), ValueError, "one of 64, 128, 256"),
    (dict(k=(2, 6, 256, 128)), ValueError, "divisible by kv_heads"),
    (dict(q=FakeTensor((2, 32, 256, 128), contiguous=False)), ValueError, "must be contiguous"),
    (dict(q=FakeTensor((2, 32, 256, 128), requires_grad=True)), ValueError, "inference-only"),
    (dict(scale=0.0), ValueError, "positive and finite"),
    (dict(scale=True), TypeError, "scale must be a number"),
])
def test_validation_messages(kwargs, error, message):
    with pytest.raises(error, match=message):
        run(**kwargs)


def test_public_export_without_torch_import():
    assert callable(rk.sdpa) and "sdpa" in rk.__all__
