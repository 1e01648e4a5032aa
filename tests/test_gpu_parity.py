"""GPU parity: the gfx950 HIP path (through the C ABI) against the CPU oracle.

Bars (max abs error against the float64 oracle on the same quantised inputs): fp16 <= 2e-3,
bf16 <= 1.6e-2.  Every case also asserts the NaN pattern matches.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from _helpers import TOLERANCE, announce, assert_within, make_case, max_abs_error, oracle64, to_device
from oracle import pa_oracle

pytestmark = pytest.mark.gpu

WORKLOAD_PARTITIONS = {"c1": 128, "c2": 64, "c3": 128, "c4": 64, "c5": 2048}


@pytest.mark.parametrize("variant", ["mfma", "valu", "mfma_qk"])
@pytest.mark.parametrize("key", ["c1", "c2", "c3", "c4"])
def test_measured_workloads_match_oracle(gpu, palib, key, variant):
    import torch
    from benchmarks.workloads import make_inputs

    data = make_inputs(key)  # CPU generator: bit-identical inputs everywhere
    w = data["workload"]
    dev = to_device(data, gpu)
    announce(f"{key} {w.name} variant={variant}")
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                       dev["context_lengths"], partition_tokens=WORKLOAD_PARTITIONS[key], variant=variant)
    torch.cuda.synchronize()
    expected = oracle64(data)
    assert_within(out, expected, w.dtype, f"{key}/{variant} vs float64 oracle")
    # The repo's own fallback algorithm in fp32 (before its final cast), evaluated on the CPU.
    fp32 = pa_oracle.fallback_restated(torch, data["query"], data["key_cache"], data["value_cache"],
                                       data["block_tables"], data["context_lengths"], out_dtype=torch.float32)
    assert_within(out, fp32.numpy().astype(np.float64), w.dtype, f"{key}/{variant} vs fp32 fallback")


@pytest.mark.parametrize("variant", ["mfma", "valu", "mfma_qk"])
def test_ragged_b128_workload(gpu, palib, c5_case, variant):
    """All 128 sequences of the headline workload against the float64 oracle."""

    import torch

    data = c5_case["gpu"]
    announce(f"c5 ragged b128, all 128 rows, variant={variant}")
    out = palib.decode(data["query"], data["key_cache"], data["value_cache"], data["block_tables"],
                       data["context_lengths"], partition_tokens=2048, variant=variant)
    torch.cuda.synchronize()
    err = assert_within(out, c5_case["expected"], "bf16", f"c5/{variant} all 128 rows")
    announce(f"c5/{variant} max abs error {err:.3e} over 128 rows")


@pytest.mark.parametrize("partition", [16, 64, 256, 1024, 4096])
@pytest.mark.parametrize("variant", ["mfma", "valu", "mfma_qk"])
def test_partition_sizes_agree(gpu, palib, partition, variant):
    case = make_case(__import__("torch"), batch=4, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                     contexts=[1, 17, 1000, 3333], dtype="bf16", seed=11)
    dev = to_device(case, gpu)
    announce(f"partition={partition} variant={variant}")
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                       dev["context_lengths"], partition_tokens=partition, variant=variant)
    assert_within(out, oracle64(case), "bf16", f"partition {partition}")


@pytest.mark.parametrize("block_size, partition, contexts, table", [
    (16, 8192, [16384, 12000, 8191, 8192, 8193, 100, 0], 16384),  # the b128 entry's partitions
    (8, 4096, [8192, 5000, 4095, 4097, 1], 8192),                 # per-lane table reads (blocks < 16)
    (1, 512, [1024, 700, 511, 513, 2], 1024),
])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_slices_of_512_blocks(gpu, palib, block_size, partition, contexts, table, dtype):
    """Partitions of 512 table entries, the widest slice the library takes: every schedule and merge
    form of the MFMA variant, and the two-launch form of the others, against the float64 oracle.  The
    MFMA forms must agree bit for bit."""

    import torch
    from test_gpu_partition_growth import device_case

    d = device_case(gpu, batch=len(contexts), contexts=contexts, table_tokens=table, dtype=dtype,
                    seed=block_size + partition, block_size=block_size)
    args = [d[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    expected = oracle64(d)
    live = torch.tensor(contexts) > 0
    outs = {}
    for variant, phase, schedule in (("mfma", "all", "grid"), ("mfma", "all", "queue"), ("mfma", "fused", "grid"),
                                     ("mfma", "fused", "queue"), ("mfma_qk", "all", "grid"), ("valu", "all", "grid")):
        tag = f"bs{block_size} P{partition} {dtype} {variant} {phase} {schedule}"
        announce(tag)
        counters = torch.zeros(palib.counter_words(len(contexts), 32, 8), dtype=torch.int32, device=gpu)
        out = palib.decode(*args, partition_tokens=partition, variant=variant, phase=phase, schedule=schedule,
                           counters=counters if phase == "fused" else None).cpu()
        assert torch.isnan(out[~live]).all(), tag
        assert_within(out[live], expected[live.numpy()], dtype, tag)
        outs[variant, phase, schedule] = out
    reference = outs["mfma", "all", "grid"].view(torch.int16)
    for key, out in outs.items():
        if key[0] == "mfma":
            assert torch.equal(out.view(torch.int16), reference), key


SHAPES = [
    # (Hq, Hkv, D, BS, dtype)
    (8, 8, 64, 16, "fp16"),
    (16, 8, 64, 32, "bf16"),
    (12, 4, 128, 16, "bf16"),   # group 3: one padded head slot
    (64, 8, 128, 16, "fp16"),   # group 8: one 8-head chunk (8-lane probability broadcast)
    (128, 8, 64, 16, "bf16"),   # group 16: two 8-head chunks
    (24, 2, 128, 32, "fp16"),   # group 12: an 8-head chunk, then 4 heads in an 8-head chunk
    (64, 8, 256, 16, "bf16"),   # group 8 at head_dim 256: one 8-head chunk (mfma), two chunks of 4 (others)
    (128, 8, 256, 16, "fp16"),  # group 16 at head_dim 256: two 8-head chunks (mfma), four chunks of 4
    (32, 8, 256, 16, "bf16"),
    (4, 4, 256, 8, "fp16"),
    (32, 4, 128, 64, "bf16"),
    (8, 2, 128, 1, "fp16"),     # one token per block
    (6, 2, 64, 128, "bf16"),
    (8, 2, 128, 256, "bf16"),   # the largest block the C ABI takes
    (16, 16, 64, 256, "fp16"),
    (32, 1, 128, 16, "fp16"),   # multi-query: one KV head, group 32 (four 8-head chunks)
    (64, 1, 64, 32, "bf16"),    # multi-query, group 64
]


@pytest.mark.parametrize("variant", ["mfma", "valu", "mfma_qk"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_shape_sweep(gpu, palib, shape, variant):
    import torch

    hq, hkv, d, bs, dtype = shape
    case = make_case(torch, batch=3, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=bs,
                     contexts=[5, bs * 3 + 1, 700], dtype=dtype, seed=hq * 7 + d + bs)
    dev = to_device(case, gpu)
    announce(f"shape {shape} variant={variant}")
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                       dev["context_lengths"], partition_tokens=128, variant=variant)
    assert_within(out, oracle64(case), dtype, f"shape {shape}")


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
def test_context_edges(gpu, palib, variant):
    """ctx=1 (output is that V row), block boundaries, full table, over-long and empty contexts."""

    import torch

    bs, mb = 16, 6
    contexts = [1, bs, bs + 1, mb * bs, mb * bs + 40, 0, -3]
    case = make_case(torch, batch=len(contexts), query_heads=8, kv_heads=2, head_dim=128, block_size=bs,
                     contexts=contexts, max_blocks=mb, dtype="fp16", seed=5)
    dev = to_device(case, gpu)
    announce(f"context edges variant={variant}")
    for partition in (16, 64, 4096):
        out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                           dev["context_lengths"], partition_tokens=partition, variant=variant).cpu()
        assert_within(out, oracle64(case), "fp16", f"edges partition {partition}")
        assert torch.isnan(out[5]).all() and torch.isnan(out[6]).all()
        # ctx = 1: softmax weight 1 on token 0, so the output is exactly token 0's V row.
        block0 = int(case["block_tables"][0, 0])
        for h in range(8):
            assert torch.equal(out[0, h], case["value_cache"][block0, 0, h // 4])


def test_int64_indices_and_explicit_scale(gpu, palib):
    import torch

    case = make_case(torch, batch=2, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                     contexts=[300, 77], dtype="bf16", index_dtype="int64", seed=9)
    dev = to_device(case, gpu)
    announce("int64 indices, scale 0.05")
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                       dev["context_lengths"], 0.05, partition_tokens=64)
    assert_within(out, oracle64(case, scale=0.05), "bf16", "int64/explicit scale")


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
def test_out_of_range_block_ids_are_skipped(gpu, palib, variant):
    import torch

    case = make_case(torch, batch=1, query_heads=8, kv_heads=2, head_dim=64, block_size=16,
                     contexts=[64], dtype="fp16", seed=3)
    num_blocks = case["key_cache"].shape[0]
    bad = case["block_tables"].clone()
    bad[0, 1] = num_blocks + 1000   # tokens 16..31 point outside the cache
    bad[0, 2] = -1                  # tokens 32..47 likewise
    dev = to_device(case, gpu)
    announce(f"out-of-range block ids variant={variant}")
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], bad.to(gpu),
                       dev["context_lengths"], partition_tokens=16, variant=variant)
    # Same as attending only over the valid tokens: blocks 0 and 3 (tokens 0-15, 48-63).
    keep = case["block_tables"][0, [0, 3]]
    compact = dict(case)
    compact["block_tables"] = keep.view(1, 2).to(case["block_tables"].dtype)
    compact["context_lengths"] = torch.tensor([32], dtype=case["context_lengths"].dtype)
    assert_within(out, oracle64(compact), "fp16", "skipped blocks")


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
def test_non_finite_propagates(gpu, palib, variant):
    import torch

    case = make_case(torch, batch=2, query_heads=8, kv_heads=2, head_dim=128, block_size=16,
                     contexts=[40, 40], dtype="bf16", seed=4)
    block = int(case["block_tables"][0, 1])
    case["key_cache"][block, 3, 1, 7] = float("nan")  # sequence 0, token 19, KV head 1
    dev = to_device(case, gpu)
    announce(f"NaN in K variant={variant}")
    out = palib.decode(dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"],
                       dev["context_lengths"], partition_tokens=16, variant=variant).cpu()
    assert torch.isnan(out[0, 4:8]).all()          # query heads of KV head 1
    assert torch.isfinite(out[0, 0:4]).all() and torch.isfinite(out[1]).all()


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
def test_deterministic(gpu, palib, variant):
    import torch
    from benchmarks.workloads import make_inputs

    data = to_device(make_inputs("c2"), gpu)
    announce(f"determinism c2 variant={variant}")
    runs = [palib.decode(data["query"], data["key_cache"], data["value_cache"], data["block_tables"],
                         data["context_lengths"], partition_tokens=64, variant=variant) for _ in range(3)]
    assert all(torch.equal(runs[0], r) for r in runs[1:])


# ---------------------------------------------------------------------------------------------
# Single-launch form (rk_pa_decode_fused): the partition kernel's last workgroup per (sequence,
# head slot) merges the records with the reduce kernel's own merge code, so it must agree with
# the two-launch form bit for bit, and leave its arrival counters zero after every call.
def _fused_vs_two_launch(palib, dev, partition, counters, variant="mfma"):
    import torch

    args = (dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"], dev["context_lengths"])
    two = palib.decode(*args, partition_tokens=partition, variant=variant)
    fused = palib.decode(*args, partition_tokens=partition, variant=variant, phase="fused", counters=counters)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16)), "fused and two-launch outputs differ"
    assert int(counters.abs().sum().item()) == 0, "arrival counters not left zero"
    return fused


@pytest.mark.parametrize("variant", ["mfma", "valu", "mfma_qk"])
@pytest.mark.parametrize("key", ["c1", "c2", "c3", "c4"])
def test_fused_matches_two_launch_on_measured_workloads(gpu, palib, key, variant):
    import torch
    from benchmarks.workloads import make_inputs

    data = make_inputs(key)
    dev = to_device(data, gpu)
    announce(f"fused {key} variant={variant}")
    counters = torch.zeros(1 << 16, dtype=torch.int32, device=gpu)
    out = _fused_vs_two_launch(palib, dev, WORKLOAD_PARTITIONS[key], counters, variant)
    assert_within(out, oracle64(data), data["workload"].dtype, f"fused {key}/{variant} vs float64 oracle")


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
@pytest.mark.parametrize("partition", [16, 64, 1024])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fused_shape_sweep(gpu, palib, shape, partition, variant):
    import torch

    hq, hkv, d, bs, dtype = shape
    if partition // bs > 512:
        pytest.skip("partition_tokens / block_size must be <= 512")
    case = make_case(torch, batch=3, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=bs,
                     contexts=[5, bs * 3 + 1, 1500], dtype=dtype, seed=hq * 5 + d + bs)
    dev = to_device(case, gpu)
    announce(f"fused shape {shape} partition={partition} variant={variant}")
    counters = torch.zeros(palib.counter_words(3, hq, hkv), dtype=torch.int32, device=gpu)
    out = _fused_vs_two_launch(palib, dev, partition, counters, variant)
    assert_within(out, oracle64(case), dtype, f"fused shape {shape}")


def test_fused_counters_serve_consecutive_calls_of_different_shapes(gpu, palib):
    """One counter buffer, stream-ordered calls: a large batch, then a smaller one, then empty and
    over-long contexts, then the large batch again.  Each must match the two-launch form."""

    import torch

    counters = torch.zeros(4096, dtype=torch.int32, device=gpu)
    cases = [
        make_case(torch, batch=16, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                  contexts=[37 * i + 900 for i in range(16)], dtype="bf16", seed=21),
        make_case(torch, batch=3, query_heads=8, kv_heads=2, head_dim=64, block_size=16,
                  contexts=[700, 12, 333], dtype="fp16", seed=22),
        make_case(torch, batch=4, query_heads=8, kv_heads=2, head_dim=128, block_size=16,
                  contexts=[0, 90, -1, 200], max_blocks=8, dtype="fp16", seed=23),
    ]
    for round_ in range(2):
        for i, case in enumerate(cases):
            dev = to_device(case, gpu)
            announce(f"fused consecutive round {round_} case {i}")
            out = _fused_vs_two_launch(palib, dev, 64, counters)
            assert_within(out, oracle64(case), case["dtype"], f"consecutive case {i}")


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
def test_fused_ragged_b128_matches_two_launch(gpu, palib, c5_case, variant):
    import torch

    announce(f"fused c5 ragged b128 variant={variant}")
    data = c5_case["gpu"]
    counters = torch.zeros(palib.counter_words(128, 32, 8), dtype=torch.int32, device=gpu)
    for _ in range(2):
        out = _fused_vs_two_launch(palib, data, 2048, counters, variant)
    assert_within(out, c5_case["expected"], "bf16", "fused c5 all 128 rows")
