"""GPU acceptance through the public API: ``rk.paged_attention_decode`` must select the gfx950 winner.

Mirrors the reference's release acceptance (developer/promotion/verify_paged_attention_release.py:
26-150): compilation is never triggered, the explain record names the exact entry and
``native/<entrypoint>``, uncovered shapes run the declared torch fallback with an exact match, and
(contracts/paged_attention_decode-1.0.json:23) the call is graph-capturable and deterministic.
"""

from __future__ import annotations

import pytest

from _helpers import announce, assert_within, make_case, oracle64, to_device

pytestmark = pytest.mark.gpu

ENTRY_IDS = {
    "c1": "paged_attention_decode-gfx950-b1-gqa32x8-c128-d128-p16-fp16",
    "c2": "paged_attention_decode-gfx950-b8-gqa32x8-c1024-d128-p16-bf16",
    "c3": "paged_attention_decode-gfx950-b4-mha16-c2048-d64-p32-bf16",
    "c4": "paged_attention_decode-gfx950-b4-gqa32x8-c1024-d256-p16-fp16",
}


@pytest.fixture(autouse=True)
def _no_compilation(monkeypatch):
    import torch.utils.cpp_extension as cpp_extension

    def forbidden(*_, **__):
        raise RuntimeError("compilation is forbidden during acceptance")

    monkeypatch.setattr(cpp_extension, "load", forbidden)


@pytest.mark.parametrize("key", sorted(ENTRY_IDS))
def test_public_api_selects_gfx950_entry(gpu, key):
    import radeon_kernels as rk
    from benchmarks.workloads import make_inputs

    data = make_inputs(key)
    dev = to_device(data, gpu)
    announce(f"rk.paged_attention_decode {key}")
    out = rk.paged_attention_decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                                    dev["context_lengths"])
    record = rk.get_last_dispatch()
    assert record["selected"] == "native/decode_mfma", rk.explain_last_dispatch()
    assert record["entry_id"] == ENTRY_IDS[key]
    assert record["architecture"] == "gfx950"
    assert "selected: native/decode_mfma" in rk.explain_last_dispatch()
    assert_within(out, oracle64(data), data["workload"].dtype, key)


def test_public_api_ragged_b128_selects_exact_entry(gpu, c5_case):
    import radeon_kernels as rk

    announce("rk.paged_attention_decode c5")
    data = c5_case["gpu"]
    out = rk.paged_attention_decode(data["query"], data["key_cache"], data["value_cache"], data["block_tables"],
                                    data["context_lengths"])
    record = rk.get_last_dispatch()
    assert record["selected"] == "native/decode_mfma"
    assert record["entry_id"] == "paged_attention_decode-gfx950-b128-gqa32x8-ragged-d128-p16-bf16"
    assert record["launch"] == {"partition_tokens": 8192, "merge": "fused"}
    assert_within(out, c5_case["expected"], "bf16", "public c5 call, all 128 rows")


def test_other_shapes_use_the_broad_gfx950_region(gpu):
    import torch

    import radeon_kernels as rk

    case = make_case(torch, batch=3, query_heads=12, kv_heads=4, head_dim=128, block_size=32,
                     contexts=[100, 1, 999], dtype="fp16", index_dtype="int64", seed=21)
    dev = to_device(case, gpu)
    announce("broad region")
    out = rk.paged_attention_decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                                    dev["context_lengths"], 0.1)
    record = rk.get_last_dispatch()
    assert record["entry_id"] == "paged_attention_decode-gfx950-region"
    assert record["selected"] == "native/decode_mfma"
    assert_within(out, oracle64(case, scale=0.1), "fp16", "broad region")


def test_uncovered_shape_runs_declared_fallback_exactly(gpu):
    """block_size 48 is outside every gfx950 entry: the torch fallback runs, bit-exact to itself."""

    import torch

    import radeon_kernels as rk
    from radeon_kernels.ops.paged_attention.reference import paged_attention_decode_reference

    case = make_case(torch, batch=2, query_heads=8, kv_heads=2, head_dim=64, block_size=48,
                     contexts=[57, 41], dtype="bf16", seed=8)
    dev = to_device(case, gpu)
    announce("uncovered shape -> fallback")
    out = rk.paged_attention_decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                                    dev["context_lengths"])
    expected = paged_attention_decode_reference(torch, dev["query"], dev["key_cache"], dev["value_cache"],
                                                dev["block_tables"], dev["context_lengths"])
    assert rk.get_last_dispatch()["selected"] == "torch/paged_attention"
    assert torch.equal(out, expected)
    assert_within(out, oracle64(case), "bf16", "fallback")


def test_graph_capture_replays_match_eager(gpu):
    import torch

    import radeon_kernels as rk
    from benchmarks.workloads import make_inputs

    data = to_device(make_inputs("c2"), gpu)
    args = (data["query"], data["key_cache"], data["value_cache"], data["block_tables"], data["context_lengths"])
    announce("graph capture c2")
    eager = rk.paged_attention_decode(*args)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            rk.paged_attention_decode(*args)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = rk.paged_attention_decode(*args)
    for _ in range(3):
        scratch = torch.randn(1 << 20, device=gpu)  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        del scratch


def _binding():
    import importlib.util

    from radeon_kernels.cabi import LIBRARY_PATH

    path = LIBRARY_PATH.parent / "rk_pa_gfx950.so"
    spec = importlib.util.spec_from_file_location("rk_pa_gfx950", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_binding_merge_forms_agree_bit_for_bit(gpu):
    """The binding's ``merge`` launch parameter: fused, reduce and auto give identical outputs."""

    import torch

    binding = _binding()
    case = make_case(torch, batch=6, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                     contexts=[1, 300, 1024, 2047, 4000, 77], dtype="bf16", seed=31)
    dev = to_device(case, gpu)
    args = (dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"], dev["context_lengths"], 0.088)
    announce("binding merge forms")
    outs = {merge: binding.decode_mfma(*args, partition_tokens=256, merge=merge) for merge in ("reduce", "fused", "auto")}
    outs["valu-fused"] = binding.decode_valu(*args, partition_tokens=256, merge="fused")
    outs["valu-reduce"] = binding.decode_valu(*args, partition_tokens=256, merge="reduce")
    torch.cuda.synchronize()
    assert torch.equal(outs["fused"], outs["reduce"]) and torch.equal(outs["auto"], outs["reduce"])
    assert torch.equal(outs["valu-fused"], outs["valu-reduce"])
    assert_within(outs["fused"], oracle64(case, scale=0.088), "bf16", "binding fused")
    with pytest.raises(ValueError, match="merge must be"):
        binding.decode_mfma(*args, partition_tokens=256, merge="tree")


def test_fused_calls_on_two_streams_use_separate_counters(gpu):
    """Fused calls in flight on two streams at once: each stream has its own counter buffer, so
    both match their single-stream results on every repetition."""

    import torch

    binding = _binding()
    cases = [make_case(torch, batch=8, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                       contexts=[900 + 150 * i for i in range(8)], dtype="bf16", seed=40 + s) for s in range(2)]
    devs = [to_device(c, gpu) for c in cases]
    argss = [(d["query"], d["key_cache"], d["value_cache"], d["block_tables"], d["context_lengths"], 0.088) for d in devs]
    announce("fused on two streams")
    expected = [binding.decode_mfma(*a, partition_tokens=128, merge="reduce") for a in argss]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    results = [[], []]
    for _ in range(20):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                results[i].append(binding.decode_mfma(*argss[i], partition_tokens=128, merge="fused"))
    torch.cuda.synchronize()
    for i in range(2):
        assert all(torch.equal(r, expected[i]) for r in results[i]), f"stream {i}"


# ---------------------------------------------------------------------------------------------
# The reference's eight workload cases in both dtypes (benchmarks/workloads/paged_attention_decode-1.0.yaml:
# 13-22), drawn as its benchmark draws them, on its three seeds: each selects its exact gfx950 entry
# through the public operator and matches the float64 oracle; the entry's launch in the other merge
# form gives the same bits.
def _reference_keys():
    from benchmarks.workloads import REFERENCE_KEYS

    return list(REFERENCE_KEYS)


@pytest.mark.parametrize("key", _reference_keys())
def test_reference_case_selects_its_entry_and_matches_oracle(gpu, palib, key):
    import torch

    import radeon_kernels as rk
    from benchmarks.workloads import REFERENCE_SEEDS, WORKLOADS, make_inputs

    w = WORKLOADS[key]
    for seed in REFERENCE_SEEDS:
        data = make_inputs(key, seed=seed)
        dev = to_device(data, gpu)
        announce(f"rk.paged_attention_decode reference case {key} seed {seed}")
        args = (dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"], dev["context_lengths"])
        out = rk.paged_attention_decode(*args)
        record = rk.get_last_dispatch()
        assert record["selected"] == "native/decode_mfma", rk.explain_last_dispatch()
        assert record["entry_id"] == f"paged_attention_decode-gfx950-{key}"
        assert_within(out, oracle64(data), w.dtype, f"{key} seed {seed}")
        partition = record["launch"]["partition_tokens"]
        fused = palib.decode(*args, partition_tokens=partition, phase="fused")
        two = palib.decode(*args, partition_tokens=partition)
        torch.cuda.synchronize()
        assert torch.equal(fused.view(torch.int16), out.view(torch.int16))
        assert torch.equal(two.view(torch.int16), out.view(torch.int16))
