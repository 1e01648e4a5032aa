"""GPU parity of the gfx950 paged KV-cache append and block copy (bit-exact: contracts/kv_cache_append-1.0.json:21,
contracts/kv_cache_copy-1.0.json:21).

* every case of the reference's workload file (benchmarks/workloads/kv_cache_append-1.0.yaml:12-18),
  both dtypes, both index types, through the C ABI and through ``rk.kv_cache_append`` (which must
  select the gfx950 native winner), against the oracle;
* out-of-range and negative slots are skipped and nothing else changes;
* HIP graph capture: every replay (with new token data each time) matches the oracle;
* append then decode: tokens written by the append are read by the decode exactly where the block
  tables put them (the two halves of a decode step, on the same cache layout);
* block copy: every case of kv_cache_copy-1.0.yaml, both dtypes and index types, through the C ABI;
  ``rk.kv_cache_copy`` selects the gfx950 winner; pairs with an out-of-range block are skipped;
* both operators on layouts beyond the reference's cases: blocks of 1 to 256 tokens, one and three KV
  heads, head_dim 64, 96 and 256.
"""

from __future__ import annotations

import numpy as np
import pytest

from _helpers import announce, assert_within, make_case, oracle64, to_device
from oracle import kv_oracle
from benchmarks.workloads import APPEND_CASES, AppendCase, make_append_inputs

pytestmark = pytest.mark.gpu


def expected_bits(data):
    b = kv_oracle.as_bits
    return kv_oracle.append_numpy(b(data["key"]), b(data["value"]), b(data["key_cache"]), b(data["value_cache"]),
                                  data["slot_mapping"].cpu().numpy())


def assert_caches(kc, vc, expected, label):
    got_k, got_v = kv_oracle.as_bits(kc), kv_oracle.as_bits(vc)
    bad_k, bad_v = int((got_k != expected[0]).sum()), int((got_v != expected[1]).sum())
    assert bad_k == 0 and bad_v == 0, f"{label}: {bad_k} key and {bad_v} value elements differ from the oracle"


@pytest.mark.parametrize("case", sorted(APPEND_CASES))
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_append_cases_bit_exact_through_the_c_abi(gpu, kvlib, case, dtype, index_dtype):
    import torch

    data = make_append_inputs(case, dtype=dtype, index_dtype=index_dtype)
    expected = expected_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce(f"kv append {case} {dtype} {index_dtype}")
    kc, vc = kvlib.append(dev["key"], dev["value"], dev["key_cache"], dev["value_cache"], dev["slot_mapping"])
    torch.cuda.synchronize()
    assert kc is dev["key_cache"] and vc is dev["value_cache"]
    assert_caches(kc, vc, expected, f"{case}/{dtype}/{index_dtype}")


@pytest.mark.parametrize("case", ["decode-t1-gqa8-d128-p16", "prefill-t128-mha32-d128-p32"])
def test_public_api_selects_the_gfx950_append(gpu, case):
    import torch

    import radeon_kernels as rk

    data = make_append_inputs(case, dtype="bf16", index_dtype="int64")
    expected = expected_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce(f"rk.kv_cache_append {case}")
    kc, vc = rk.kv_cache_append(dev["key"], dev["value"], dev["key_cache"], dev["value_cache"], dev["slot_mapping"])
    torch.cuda.synchronize()
    record = rk.get_last_dispatch()
    assert record["selected"] == "native/append", rk.explain_last_dispatch()
    assert record["entry_id"] == f"kv_cache_append-gfx950-{case}"
    assert kc.data_ptr() == dev["key_cache"].data_ptr()
    assert_caches(kc, vc, expected, case)


def test_out_of_range_slots_are_skipped(gpu, kvlib):
    import torch

    case = AppendCase("edge", 6, 8, 16, 2, 64)
    data = make_append_inputs(case, dtype="fp16", index_dtype="int64", seed=11)
    cap = case.num_blocks * case.block_size
    data["slot_mapping"] = torch.tensor([5, -1, cap, 17, -(1 << 40), 1 << 40], dtype=torch.int64)
    expected = expected_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce("kv append out-of-range slots")
    kvlib.append(dev["key"], dev["value"], dev["key_cache"], dev["value_cache"], dev["slot_mapping"])
    torch.cuda.synchronize()
    assert_caches(dev["key_cache"], dev["value_cache"], expected, "out-of-range slots")
    # int32 negatives too
    data32 = dict(data, slot_mapping=torch.tensor([5, -1, -7, 17, 3, 0], dtype=torch.int32))
    expected32 = expected_bits(data32)
    dev32 = {k: v.to(gpu) for k, v in data32.items() if hasattr(v, "to")}
    kvlib.append(dev32["key"], dev32["value"], dev32["key_cache"], dev32["value_cache"], dev32["slot_mapping"])
    torch.cuda.synchronize()
    assert_caches(dev32["key_cache"], dev32["value_cache"], expected32, "negative int32 slots")


def test_graph_capture_replays_match_the_oracle(gpu, kvlib):
    import torch

    case = APPEND_CASES["decode-t32-gqa8-d128-p16"]
    base = make_append_inputs(case, dtype="bf16", index_dtype="int64", seed=21)
    dev = {k: v.to(gpu) for k, v in base.items() if hasattr(v, "to")}
    announce("kv append graph capture")
    kvlib.append(dev["key"], dev["value"], dev["key_cache"], dev["value_cache"], dev["slot_mapping"])  # warm up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            kvlib.append(dev["key"], dev["value"], dev["key_cache"], dev["value_cache"], dev["slot_mapping"])
    torch.cuda.synchronize()
    for replay in range(3):
        fresh = make_append_inputs(case, dtype="bf16", index_dtype="int64", seed=100 + replay)
        dev["key"].copy_(fresh["key"].to(gpu))
        dev["value"].copy_(fresh["value"].to(gpu))
        dev["slot_mapping"].copy_(fresh["slot_mapping"].to(gpu))
        before = {name: dev[name].cpu() for name in ("key_cache", "value_cache")}
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = expected_bits({"key": fresh["key"], "value": fresh["value"], "key_cache": before["key_cache"],
                                  "value_cache": before["value_cache"], "slot_mapping": fresh["slot_mapping"]})
        assert_caches(dev["key_cache"], dev["value_cache"], expected, f"replay {replay}")


def test_append_then_decode_reads_the_new_tokens(gpu, kvlib, palib):
    import torch

    # Sequences of 37 and 70 tokens; append 5 new tokens to each through the block tables, then
    # decode over the grown contexts and compare with the oracle on the updated cache.
    case = make_case(torch, batch=2, query_heads=16, kv_heads=4, head_dim=128, block_size=16, contexts=[42, 75],
                     dtype="bf16", index_dtype="int64", seed=31)
    old = [37, 70]
    tables = case["block_tables"]
    slots = []
    for b, start in enumerate(old):
        for t in range(start, start + 5):
            slots.append(int(tables[b, t // 16]) * 16 + t % 16)
    gen = torch.Generator().manual_seed(32)
    new_k = torch.randn((10, 4, 128), generator=gen).to(torch.bfloat16)
    new_v = torch.randn((10, 4, 128), generator=gen).to(torch.bfloat16)
    slot_mapping = torch.tensor(slots, dtype=torch.int64)
    updated = dict(case)
    k_bits, v_bits = kv_oracle.append_numpy(kv_oracle.as_bits(new_k), kv_oracle.as_bits(new_v),
                                            kv_oracle.as_bits(case["key_cache"]), kv_oracle.as_bits(case["value_cache"]),
                                            slot_mapping.numpy())
    updated["key_cache"] = torch.from_numpy(k_bits).view(torch.bfloat16)
    updated["value_cache"] = torch.from_numpy(v_bits).view(torch.bfloat16)
    dev = to_device(case, gpu)
    announce("append then decode")
    kvlib.append(new_k.to(gpu), new_v.to(gpu), dev["key_cache"], dev["value_cache"], slot_mapping.to(gpu))
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                       dev["context_lengths"], partition_tokens=32)
    torch.cuda.synchronize()
    assert_within(out, oracle64(updated), "bf16", "append then decode")


# ---------------------------------------------------------------------------------------------
# Block copy (contracts/kv_cache_copy-1.0.json: bit-exact, snapshot semantics)
from benchmarks.workloads import COPY_CASES, CopyCase, make_copy_inputs  # noqa: E402


def expected_copy_bits(data):
    b = kv_oracle.as_bits
    return kv_oracle.copy_numpy(b(data["key_cache"]), b(data["value_cache"]), data["block_mapping"].cpu().numpy())


@pytest.mark.parametrize("case", sorted(COPY_CASES))
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_copy_cases_bit_exact_through_the_c_abi(gpu, kvlib, case, dtype, index_dtype):
    import torch

    data = make_copy_inputs(case, dtype=dtype, index_dtype=index_dtype)
    expected = expected_copy_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce(f"kv copy {case} {dtype} {index_dtype}")
    kc, vc = kvlib.copy(dev["key_cache"], dev["value_cache"], dev["block_mapping"])
    torch.cuda.synchronize()
    assert_caches(kc, vc, expected, f"copy {case}/{dtype}/{index_dtype}")


def test_public_copy_selects_the_gfx950_kernel_and_skips_out_of_range_pairs(gpu, kvlib):
    import torch

    import radeon_kernels as rk

    data = make_copy_inputs("beam-pairs32-mha32-d128-p32", dtype="bf16", index_dtype="int64")
    expected = expected_copy_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce("rk.kv_cache_copy beam-pairs32-mha32")
    kc, vc = rk.kv_cache_copy(dev["key_cache"], dev["value_cache"], dev["block_mapping"])
    torch.cuda.synchronize()
    record = rk.get_last_dispatch()
    assert record["selected"] == "native/copy", rk.explain_last_dispatch()
    assert record["entry_id"] == "kv_cache_copy-gfx950-beam-pairs32-mha32-d128-p32"
    assert_caches(kc, vc, expected, "public copy")

    small = make_copy_inputs(CopyCase("edge", 3, 12, 16, 2, 64), dtype="fp16", index_dtype="int32", seed=8)
    small["block_mapping"] = torch.tensor([[1, 5], [2, 12], [-1, 6], [3, 0], [11, -4]], dtype=torch.int32)
    expected = expected_copy_bits(small)
    dev = {k: v.to(gpu) for k, v in small.items() if hasattr(v, "to")}
    announce("kv copy out-of-range pairs")
    kvlib.copy(dev["key_cache"], dev["value_cache"], dev["block_mapping"])
    torch.cuda.synchronize()
    assert_caches(dev["key_cache"], dev["value_cache"], expected, "out-of-range pairs")


# Layouts beyond the reference's cases: one-token and 256-token blocks, one and three KV heads, head_dim
# 64, 96 and 256 (cache rows of any multiple of 16 bytes).
OTHER_APPEND = [
    AppendCase("bs1-kv1-d64", 37, 64, 1, 1, 64),
    AppendCase("bs256-kv2-d128", 50, 12, 256, 2, 128),
    AppendCase("bs8-kv3-d96", 19, 40, 8, 3, 96),
    AppendCase("bs128-kv1-d256", 7, 16, 128, 1, 256),
]
OTHER_COPY = [
    CopyCase("bs1-kv1-d64", 5, 32, 1, 1, 64),
    CopyCase("bs256-kv2-d128", 3, 8, 256, 2, 128),
    CopyCase("bs8-kv3-d96", 4, 20, 8, 3, 96),
]


@pytest.mark.parametrize("case", OTHER_APPEND, ids=lambda c: c.key)
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_append_on_other_layouts(gpu, kvlib, case, dtype):
    import torch

    data = make_append_inputs(case, dtype=dtype, index_dtype="int32", seed=case.tokens)
    expected = expected_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce(f"kv append {case.key} {dtype}")
    kc, vc = kvlib.append(dev["key"], dev["value"], dev["key_cache"], dev["value_cache"], dev["slot_mapping"])
    torch.cuda.synchronize()
    assert_caches(kc, vc, expected, f"append {case.key}/{dtype}")


@pytest.mark.parametrize("case", OTHER_COPY, ids=lambda c: c.key)
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_copy_on_other_layouts(gpu, kvlib, case, dtype):
    import torch

    data = make_copy_inputs(case, dtype=dtype, index_dtype="int64", seed=case.pairs)
    expected = expected_copy_bits(data)
    dev = {k: v.to(gpu) for k, v in data.items() if hasattr(v, "to")}
    announce(f"kv copy {case.key} {dtype}")
    kc, vc = kvlib.copy(dev["key_cache"], dev["value_cache"], dev["block_mapping"])
    torch.cuda.synchronize()
    assert_caches(kc, vc, expected, f"copy {case.key}/{dtype}")
