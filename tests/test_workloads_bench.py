"""CPU tests of the seeded workloads and of bench.py's contract pieces that need no GPU."""

from __future__ import annotations

import dataclasses
import json
import math
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from benchmarks.workloads import WORKLOADS, aux_bytes, kv_bytes, make_inputs

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("key", ["c1", "c2", "c3", "c4"])
def test_fixed_workloads_shapes_tables_and_bytes(key):
    data = make_inputs(key)
    w = data["workload"]
    assert tuple(data["query"].shape) == (w.batch, w.query_heads, w.head_dim)
    assert tuple(data["key_cache"].shape) == (w.num_blocks, w.block_size, w.kv_heads, w.head_dim)
    assert data["key_cache"].dtype == {"fp16": torch.float16, "bf16": torch.bfloat16}[w.dtype]
    tables = data["block_tables"]
    assert tables.dtype == torch.int32 and tuple(tables.shape) == (w.batch, w.max_blocks)
    assert len(set(tables.flatten().tolist())) == w.batch * w.max_blocks  # disjoint, no padding
    assert int(tables.max()) < w.num_blocks
    assert data["context_lengths"].tolist() == [w.context] * w.batch
    # The KV bytes the bench divides by (4 fixed workloads of the scale table in the brief).
    expected = {"c1": 524_288, "c2": 33_554_432, "c3": 33_554_432, "c4": 33_554_432}[key]
    assert data["kv_bytes"] == expected


def test_generation_is_deterministic_and_seed_dependent():
    a, b = make_inputs("c1"), make_inputs("c1")
    for field in ("query", "key_cache", "value_cache", "block_tables", "context_lengths"):
        assert torch.equal(a[field], b[field])
    c = make_inputs("c1", seed=123)
    assert not torch.equal(a["query"], c["query"])
    assert make_inputs("c1", index_dtype="int64")["block_tables"].dtype == torch.int64


def test_c4_uses_half_standard_deviation():
    data = make_inputs("c4")
    std = data["key_cache"].float().std().item()
    assert 0.45 < std < 0.55


def test_ragged_workload_structure_on_a_scaled_copy():
    w = dataclasses.replace(WORKLOADS["c5"], batch=6)
    data = make_inputs(w)
    ctx = data["context_lengths"].long()
    assert ((ctx >= 1024) & (ctx <= 16384)).all()
    need = [math.ceil(int(c) / 16) for c in ctx]
    assert data["num_blocks"] == sum(need)
    tables = data["block_tables"].long()
    used = torch.cat([tables[b, :n] for b, n in enumerate(need)])
    assert sorted(used.tolist()) == list(range(data["num_blocks"]))  # a permutation of all blocks
    for b, n in enumerate(need):
        assert (tables[b, n:] == 0).all()  # padding with block 0
    assert data["kv_bytes"] == int(ctx.sum()) * 8 * 128 * 2 * 2


def test_byte_accounting_caps_and_ignores_padding():
    w = WORKLOADS["c2"]
    assert kv_bytes(w, [2000, 0, -5, 10]) == (1024 + 0 + 0 + 10) * 8 * 128 * 4
    assert aux_bytes(w, [1024] * 8) == 2 * 8 * 32 * 128 * 2 + 8 * 64 * 4 + 8 * 4


def test_bench_refuses_more_than_one_gpu():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert result.returncode == 2
    message = json.loads(result.stdout.strip().splitlines()[-1])
    assert message["n_gpus"] == 2 and "one GPU" in message["error"]


def test_bench_reads_traffic_only_for_its_exact_configuration(tmp_path, monkeypatch):
    import bench

    summary = tmp_path / "traffic.txt"
    summary.write_text("# measured\nworkload = b128-x\nvariant = mfma\npartition_tokens = 2048\n"
                       "kv_bytes_per_call = 4237918208\nhbm_bytes_per_launch = 4867000000\n")
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARIES", (tmp_path / "absent.txt", summary))
    kv = 4_237_918_208
    assert bench.read_traffic("b128-x", "mfma", 2048, "reduce", "grid", kv) == 4_867_000_000
    assert bench.read_traffic("b128-x", "mfma", 1024, "reduce", "grid", kv) is None
    assert bench.read_traffic("other", "mfma", 2048, "reduce", "grid", kv) is None
    assert bench.read_traffic("b128-x", "mfma", 2048, "reduce", "grid", kv + 1) is None  # another input draw
    assert bench.read_traffic("b128-x", "mfma", 2048, "fused", "grid", kv) is None  # measured in the reduce form
    assert bench.read_traffic("b128-x", "mfma", 2048, "reduce", "queue", kv) is None  # and on the grid schedule
    summary.write_text(summary.read_text() + "merge = fused\nschedule = queue\n")
    assert bench.read_traffic("b128-x", "mfma", 2048, "fused", "queue", kv) == 4_867_000_000
    assert bench.read_traffic("b128-x", "mfma", 2048, "fused", "grid", kv) is None
    assert bench.read_traffic("b128-x", "mfma", 2048, "reduce", "queue", kv) is None
    # A summary that records its draw's seed matches that seed only (same shape and KV bytes, other values).
    summary.write_text(summary.read_text() + "seed = 7\n")
    assert bench.read_traffic("b128-x", "mfma", 2048, "fused", "queue", kv, seed=7) == 4_867_000_000
    assert bench.read_traffic("b128-x", "mfma", 2048, "fused", "queue", kv, seed=8) is None
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARIES", (tmp_path / "absent.txt",))
    assert bench.read_traffic("b128-x", "mfma", 2048, "fused", "queue", kv) is None


def test_case_traffic_matches_operator_case_and_dtype(tmp_path):
    import bench

    summary = tmp_path / "kv.txt"
    summary.write_text("# measured\nworkload = kv_cache_copy-beam-pairs64-gqa8-d256-p16-bf16\n"
                       "hbm_bytes_per_launch = 16839687\n")
    assert bench.read_case_traffic(summary, "kv_cache_copy-beam-pairs64-gqa8-d256-p16-bf16") == 16_839_687
    assert bench.read_case_traffic(summary, "kv_cache_copy-beam-pairs64-gqa8-d256-p16-fp16") is None
    assert bench.read_case_traffic(tmp_path / "absent.txt", "anything") is None


def test_committed_case_summaries_name_their_bench_workloads():
    import bench

    profiles = bench.ROOT / "profiles"
    assert bench.read_case_traffic(profiles / "kv_append_kernel_prefill-t128-mha32-d128-p32.txt",
                                   "kv_cache_append-prefill-t128-mha32-d128-p32-bf16") == 4_220_936
    assert bench.read_case_traffic(profiles / "kv_copy_kernel_beam-pairs64-gqa8-d256-p16.txt",
                                   "kv_cache_copy-beam-pairs64-gqa8-d256-p16-bf16") == 16_839_687


def test_bench_accepts_every_workload_and_defaults_to_b128():
    import bench

    args = bench.parse_args([])
    assert (args.gpus, args.workload) == (1, "c5")
    for key in WORKLOADS:
        assert bench.parse_args(["--workload", key]).workload == key


def test_cpu_baseline_thread_count_respects_affinity_and_share(monkeypatch):
    import bench

    monkeypatch.setattr(bench.os, "sched_getaffinity", lambda pid: set(range(64)))
    monkeypatch.setenv("OMP_NUM_THREADS", "16")
    assert bench.cpu_threads() == (16, 64)
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.cpu_threads() == (64, 64)
    monkeypatch.setattr(bench.os, "sched_getaffinity", lambda pid: set(range(8)))
    monkeypatch.setenv("OMP_NUM_THREADS", "16")
    assert bench.cpu_threads() == (8, 8)


def test_cpu_baseline_protocol_on_a_small_workload():
    """The CPU leg on CPU tensors: one warmup pass, at least three timed passes, the thread count set
    and recorded with torch's parallel_info."""

    import torch

    import bench
    from benchmarks.workloads import make_inputs

    data = make_inputs("b1-gqa32x8-c128-d128-p16-fp16")
    before = torch.get_num_threads()
    try:
        result = bench.cpu_baseline(torch, data, seconds=0.5)
        assert result["cores"] == bench.cpu_threads()[0] == torch.get_num_threads()
    finally:
        torch.set_num_threads(before)
    assert 3 <= result["pass_seconds"]["passes"] <= 30 and result["value"] > 0
    assert result["kind"] == "port" and "1 warmup pass" in result["sample"]
    assert any("ATen" in line or "OpenMP" in line for line in result["parallel_info"])
