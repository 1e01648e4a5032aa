"""CPU tests of call plans: a call shape that ran natively once skips re-validation and dispatch.

The plan is an optimisation only, so every test checks that behaviour is unchanged: the same
entrypoint arguments, launch parameters and explain record as the validated path; every input that
differs from the planned call in anything validation reads still gets the reference's error; errors
from the planned winner still demote (or raise in strict mode); the kv operators still check that
the caches they get back are the ones they passed.
"""

from __future__ import annotations

import math
import warnings
from pathlib import Path
from types import SimpleNamespace

import pytest

from radeon_kernels.ops import _runtime
from radeon_kernels.ops._common import call_key
from radeon_kernels.ops._runtime import NativeDemotionWarning, OperatorDispatchError, OperatorRuntime
from radeon_kernels.ops.kv_cache import api as kv_api
from radeon_kernels.ops.paged_attention import api as pa_api
from radeon_kernels.ops.sdpa import api as sdpa_api
from radeon_kernels.runtime.dispatcher import Dispatcher
from radeon_kernels.runtime.explain import clear_last_dispatch, get_last_dispatch
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.registry import DispatchManifest, DispatchRegistry
from test_api import FakeDevice, FakeTensor, FakeTorch

DEFAULT_SCALE = 1.0 / math.sqrt(128)  # the reference's default, api.py:27-29
ENV = {"architecture": "gfx950", "wavefront_size": 64, "rocm_abi": "7.0", "python_abi": "cp310",
       "pytorch_version": "2.10.0+rocm7.0"}


def manifest(operator, entrypoint, workload, launch):
    return DispatchManifest.from_mapping({
        "schema_version": "1.0", "operator": operator, "semantic_version": "1.0", "default_fallbacks": ["torch"],
        "entries": [{
            "id": f"{operator}-test", "priority": 100, "environment": dict(ENV), "workload": workload,
            "winner": {"provider": "native", "artifact": "lib/x.so", "entrypoint": entrypoint, "sha256": "a" * 64,
                       "format": "python_extension"},
            "launch": launch, "fallbacks": ["torch"], "evidence_id": f"evidence-{operator}",
        }],
    })


class Packs:
    def __init__(self):
        self.calls = 0

    def resolve(self, **_):
        self.calls += 1
        return SimpleNamespace(pack=SimpleNamespace(root=Path("."), pack_id="pack", pack_version="1.0.0"))


class Native:
    """Loader factory whose entrypoint records its calls; ``mode`` switches it to failing."""

    mode = "ok"
    calls: list = []
    loads = 0
    result = None

    def __init__(self, _root):
        pass

    def load_entrypoint(self, _artifact):
        Native.loads += 1

        def entry(*args, **launch):
            Native.calls.append((args, launch))
            if Native.mode == "raise":
                raise RuntimeError("launch failed")
            if Native.mode == "none":
                return None
            return Native.result if Native.result is not None else ("native", len(Native.calls))

        return SimpleNamespace(callable=entry)


@pytest.fixture
def runtime_factory():
    def make(*manifests, strict=False):
        clear_last_dispatch()
        Native.mode, Native.calls, Native.loads, Native.result = "ok", [], 0, None
        packs = Packs()
        runtime = OperatorRuntime(registry=DispatchRegistry(list(manifests)), pack_registry=packs,
                                  loader_factory=Native, strict_native=strict,
                                  fingerprint_detector=lambda **_: EnvironmentFingerprint(**ENV))
        return runtime, packs

    return make


PA = manifest("paged_attention_decode", "decode_mfma", {"dtype": "bf16", "batch": [8, 8], "head_dim": 128},
              {"partition_tokens": 256, "merge": "fused"})


def pa_inputs(**changes):
    spec = dict(q=((8, 32, 128), "bfloat16"), k=((1024, 16, 8, 128), "bfloat16"), v=((1024, 16, 8, 128), "bfloat16"),
                bt=((8, 64), "int32"), cl=((8,), "int32"))
    tensors = {name: FakeTensor(shape, dtype=dtype) for name, (shape, dtype) in spec.items()}
    tensors.update(changes)
    return tensors["q"], tensors["k"], tensors["v"], tensors["bt"], tensors["cl"]


def pa_call(runtime, torch_module, tensors, scale=None):
    return pa_api._dispatch(*tensors, scale, torch_module=torch_module, runtime=runtime)


def test_second_call_runs_the_plan_with_identical_arguments_and_record(runtime_factory):
    runtime, packs = runtime_factory(PA)
    torch_module = FakeTorch()
    tensors = pa_inputs()
    first = pa_call(runtime, torch_module, tensors)
    first_record = get_last_dispatch()
    clear_last_dispatch()
    second = pa_call(runtime, torch_module, tensors)
    assert first == ("native", 1) and second == ("native", 2)
    assert packs.calls == 1 and Native.loads == 1  # no second resolution or load
    assert Native.calls[0] == Native.calls[1]
    args, launch = Native.calls[1]
    assert args == (*tensors, DEFAULT_SCALE) and launch == {"partition_tokens": 256, "merge": "fused"}
    assert get_last_dispatch() == first_record
    assert first_record["selected"] == "native/decode_mfma"


def test_plan_is_reused_for_new_tensors_of_the_same_shape(runtime_factory, monkeypatch):
    runtime, packs = runtime_factory(PA)
    torch_module = FakeTorch()
    pa_call(runtime, torch_module, pa_inputs())
    monkeypatch.setattr(pa_api, "_execute", lambda *a, **k: pytest.fail("validated path taken"))
    fresh = pa_inputs()
    pa_call(runtime, torch_module, fresh)
    assert Native.calls[-1][0][:5] == fresh


def test_explicit_scale_plans_per_value(runtime_factory):
    runtime, packs = runtime_factory(PA)
    torch_module = FakeTorch()
    tensors = pa_inputs()
    for scale, resolutions in ((0.25, 1), (0.25, 1), (0.5, 2), (None, 3), (None, 3)):
        pa_call(runtime, torch_module, tensors, scale)
        assert packs.calls == resolutions
        assert Native.calls[-1][0][5] == (0.25 if scale == 0.25 else 0.5 if scale == 0.5 else DEFAULT_SCALE)
    # Non-float scales are never keyed: they take the validated path every time.
    pa_call(runtime, torch_module, tensors, 1)
    pa_call(runtime, torch_module, tensors, 1)
    assert packs.calls == 5 and Native.calls[-1][0][5] == 1.0


@pytest.mark.parametrize("change, error, message", [
    (dict(q=FakeTensor((8, 32, 128), dtype="bfloat16", contiguous=False)), ValueError, "inputs must be contiguous"),
    (dict(k=FakeTensor((1024, 16, 8, 128), dtype="bfloat16", requires_grad=True)), ValueError, "inference-only"),
    (dict(v=FakeTensor((1024, 16, 8, 128), dtype="float16")), TypeError, "must use the same dtype"),
    (dict(bt=FakeTensor((8, 64), dtype="int32", is_cuda=False)), ValueError, "visible ROCm GPU"),
    (dict(cl=FakeTensor((8,), dtype="int32", device=FakeDevice(1))), ValueError, "same device as query"),
    (dict(cl=FakeTensor((8,), dtype="int64")), TypeError, "same dtype"),
    (dict(q=FakeTensor((8, 32, 100), dtype="bfloat16")), ValueError, "head_dim must match"),
    (dict(bt=FakeTensor((7, 64), dtype="int32")), ValueError, "block_tables must have shape"),
    (dict(q=object()), TypeError, "query must be a PyTorch tensor"),
])
def test_calls_that_differ_from_a_plan_are_validated(runtime_factory, change, error, message):
    runtime, _ = runtime_factory(PA)
    torch_module = FakeTorch()
    pa_call(runtime, torch_module, pa_inputs())
    with pytest.raises(error, match=message):
        pa_call(runtime, torch_module, pa_inputs(**change))


@pytest.mark.parametrize("scale, error", [(float("nan"), ValueError), (-1.0, ValueError), (0.0, ValueError),
                                          (True, TypeError), ("0.1", TypeError)])
def test_invalid_scales_after_a_plan_still_raise(runtime_factory, scale, error):
    runtime, _ = runtime_factory(PA)
    torch_module = FakeTorch()
    pa_call(runtime, torch_module, pa_inputs())
    pa_call(runtime, torch_module, pa_inputs(), 0.5)
    with pytest.raises(error, match="scale"):
        pa_call(runtime, torch_module, pa_inputs(), scale)


def test_planned_winner_failure_demotes_like_the_validated_path(runtime_factory, monkeypatch):
    runtime, _ = runtime_factory(PA)
    torch_module = FakeTorch()
    monkeypatch.setattr(pa_api, "paged_attention_decode_reference", lambda *args: "torch-result")
    pa_call(runtime, torch_module, pa_inputs())
    for mode, text in (("raise", "launch failed"), ("none", "native entrypoint returned no output")):
        Native.mode = mode
        with pytest.warns(NativeDemotionWarning, match="decode_mfma unavailable"):
            assert pa_call(runtime, torch_module, pa_inputs()) == "torch-result"
        record = get_last_dispatch()
        assert record["selected"] == "torch/paged_attention"
        assert f"winner unavailable: {text}; executed declared torch fallback" in record["reason"]
    # The plan survives a demotion: the next good call runs natively again.
    Native.mode = "ok"
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert pa_call(runtime, torch_module, pa_inputs())[0] == "native"
    assert get_last_dispatch()["selected"] == "native/decode_mfma"


def test_planned_winner_failure_raises_in_strict_mode(runtime_factory):
    runtime, _ = runtime_factory(PA, strict=True)
    torch_module = FakeTorch()
    pa_call(runtime, torch_module, pa_inputs())
    Native.mode = "raise"
    with pytest.raises(OperatorDispatchError, match="native winner"):
        pa_call(runtime, torch_module, pa_inputs())
    record = get_last_dispatch()
    assert record["selected"] == "none" and record["reason"].endswith("strict native mode")


def test_failed_native_calls_leave_no_plan(runtime_factory, monkeypatch):
    runtime, packs = runtime_factory(PA)
    torch_module = FakeTorch()
    monkeypatch.setattr(pa_api, "paged_attention_decode_reference", lambda *args: "torch-result")
    Native.mode = "raise"
    with pytest.warns(NativeDemotionWarning):
        pa_call(runtime, torch_module, pa_inputs())
    Native.mode = "ok"
    pa_call(runtime, torch_module, pa_inputs())
    assert packs.calls == 2  # resolved again: the failed call kept nothing


def test_unmatched_shapes_keep_no_plan(runtime_factory, monkeypatch):
    runtime, _ = runtime_factory(PA)
    torch_module = FakeTorch()
    monkeypatch.setattr(pa_api, "paged_attention_decode_reference", lambda *args: "torch-result")
    q = FakeTensor((4, 32, 128), dtype="bfloat16")
    tensors = pa_inputs(q=q, bt=FakeTensor((4, 64), dtype="int32"), cl=FakeTensor((4,), dtype="int32"))
    for _ in range(2):
        assert pa_call(runtime, torch_module, tensors) == "torch-result"
        assert get_last_dispatch()["selected"] == "torch/paged_attention"
    assert runtime._plans == {}


def test_plan_table_is_bounded(runtime_factory, monkeypatch):
    runtime, _ = runtime_factory(PA)
    monkeypatch.setattr(OperatorRuntime, "_PLAN_LIMIT", 3)
    torch_module = FakeTorch()
    for scale in (0.1, 0.2, 0.3, 0.4, 0.5):
        pa_call(runtime, torch_module, pa_inputs(), scale)
        assert len(runtime._plans) <= 3
    assert runtime.plan_for(None) is None


def test_call_key_covers_what_validation_reads():
    torch_module = FakeTorch()
    base = call_key(torch_module, "op", pa_inputs())
    assert base is not None and hash(base) == hash(call_key(torch_module, "op", pa_inputs()))
    variants = [
        pa_inputs(q=FakeTensor((8, 32, 128), dtype="float16")),
        pa_inputs(q=FakeTensor((8, 32, 128), dtype="bfloat16", device=FakeDevice(1))),
        pa_inputs(q=FakeTensor((8, 32, 128), dtype="bfloat16", is_cuda=False)),
        pa_inputs(q=FakeTensor((8, 16, 128), dtype="bfloat16")),
        pa_inputs(q=FakeTensor((8, 32, 128), dtype="bfloat16", contiguous=False)),
        pa_inputs(q=FakeTensor((8, 32, 128), dtype="bfloat16", requires_grad=True)),
    ]
    for tensors in variants:
        assert call_key(torch_module, "op", tensors) != base
    assert call_key(torch_module, "other", pa_inputs()) != base
    assert call_key(FakeTorch(), "op", pa_inputs()) != base  # another module's dtypes
    assert call_key(torch_module, "op", pa_inputs(), 0.5) != base
    assert call_key(torch_module, "op", (object(),)) is None


class PtrTensor(FakeTensor):
    def __init__(self, shape, ptr, **kwargs):
        super().__init__(shape, **kwargs)
        self._ptr = ptr

    def data_ptr(self):
        return self._ptr


def test_kv_append_plan_still_checks_returned_caches(runtime_factory):
    runtime, packs = runtime_factory(manifest("kv_cache_append", "append", {"dtype": "bf16", "tokens": [8, 8]}, {}))
    torch_module = FakeTorch()
    key, value = (FakeTensor((8, 8, 128), dtype="bfloat16") for _ in range(2))
    k_cache, v_cache = PtrTensor((64, 16, 8, 128), 1, dtype="bfloat16"), PtrTensor((64, 16, 8, 128), 2, dtype="bfloat16")
    slots = FakeTensor((8,), dtype="int32")
    Native.result = (k_cache, v_cache)
    for _ in range(2):
        assert kv_api._dispatch_append(key, value, k_cache, v_cache, slots, torch_module=torch_module,
                                       runtime=runtime) == (k_cache, v_cache)
    assert packs.calls == 1 and len(Native.calls) == 2
    Native.result = (PtrTensor((64, 16, 8, 128), 9, dtype="bfloat16"), v_cache)
    with pytest.raises(RuntimeError, match="must return the input cache tensors"):
        kv_api._dispatch_append(key, value, k_cache, v_cache, slots, torch_module=torch_module, runtime=runtime)
    assert packs.calls == 1


def test_kv_copy_plan(runtime_factory):
    runtime, packs = runtime_factory(manifest("kv_cache_copy", "copy_blocks", {"dtype": "fp16", "pairs": [4, 4]}, {}))
    torch_module = FakeTorch()
    k_cache, v_cache = PtrTensor((64, 16, 8, 128), 1), PtrTensor((64, 16, 8, 128), 2)
    mapping = FakeTensor((4, 2), dtype="int64")
    Native.result = (k_cache, v_cache)
    for _ in range(3):
        kv_api._dispatch_copy(k_cache, v_cache, mapping, torch_module=torch_module, runtime=runtime)
    assert packs.calls == 1 and Native.calls[-1] == ((k_cache, v_cache, mapping), {})
    with pytest.raises(ValueError, match=r"block_mapping must have shape \[pairs, 2\]"):
        kv_api._dispatch_copy(k_cache, v_cache, FakeTensor((4, 3), dtype="int64"), torch_module=torch_module,
                              runtime=runtime)


def test_sdpa_plan_keys_causality_and_scale(runtime_factory):
    runtime, packs = runtime_factory(manifest("sdpa", "forward", {"dtype": "fp16", "batch": [1, 1]}, {}))
    torch_module = FakeTorch()
    q = FakeTensor((1, 32, 128, 128))
    k, v = FakeTensor((1, 8, 128, 128)), FakeTensor((1, 8, 128, 128))
    for causal in (True, True, False, False):
        sdpa_api._dispatch(q, k, v, causal, None, torch_module=torch_module, runtime=runtime)
        assert Native.calls[-1][0] == (q, k, v, causal, DEFAULT_SCALE)
    assert packs.calls == 2
    with pytest.raises(TypeError, match="is_causal must be bool"):
        sdpa_api._dispatch(q, k, v, 1, None, torch_module=torch_module, runtime=runtime)
    sdpa_api._dispatch(q, k, v, True, 0.1, torch_module=torch_module, runtime=runtime)
    sdpa_api._dispatch(q, k, v, True, 0.1, torch_module=torch_module, runtime=runtime)
    assert packs.calls == 3 and Native.calls[-1][0][-1] == 0.1


def test_public_functions_use_the_plan_path():
    import inspect

    assert "_dispatch(" in inspect.getsource(pa_api.paged_attention_decode)
    assert "_dispatch(" in inspect.getsource(sdpa_api.sdpa)
    assert "_dispatch_append(" in inspect.getsource(kv_api.kv_cache_append)
    assert "_dispatch_copy(" in inspect.getsource(kv_api.kv_cache_copy)
    assert isinstance(_runtime.OperatorRuntime._PLAN_LIMIT, int) and Dispatcher._CACHE_LIMIT > 0
