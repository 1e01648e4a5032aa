"""Partition growth (RK_PA_PARTITION_GROW): on the work-queue schedule the kernel runs partitions of
partition_tokens * 2^k tokens, k chosen from the live context lengths.

Parity: a growing call is bit-identical to a call without growth at the size it ran (read from
workspace header word 1 in the two-launch form), in both merge forms, through the phase entries,
the no-allocation entry and append-and-decode, and matches the float64 oracle
(src/radeon_kernels/ops/paged_attention/reference.py:7-47 restated in oracle/).  The size itself is
checked against the rule the kernel documents (resident workgroups = 2 per CU for the head_dim-128
GQA-4 queue kernel) and, on the long-context shapes, against the fastest fixed size measured.
"""

from __future__ import annotations

import random

import pytest

from _helpers import announce, assert_within, make_case, oracle64_rows, to_device

pytestmark = pytest.mark.gpu

GROW_BALANCE = 1440
GROW_MAX_TOKENS = 4096


def _args(d):
    return d["query"], d["key_cache"], d["value_cache"], d["block_tables"], d["context_lengths"]


def _grown_size(workspace) -> int:
    import torch

    return int(workspace[4:8].view(torch.int32).item())


def _workspace(palib, d, partition):
    import torch

    q, k, _, bt, _ = _args(d)
    need = palib.workspace_bytes(q.shape[0], q.shape[1], q.shape[2], k.shape[1], bt.shape[1], partition)
    return torch.zeros(need, dtype=torch.uint8, device=q.device)


def expected_size(contexts, table_tokens, heads_per_seq, base, block_size, capacity):
    """The rule: the largest base * 2^k within the host limit with (base * 2^k)^2 <= GROW_BALANCE * W,
    W = clamped context tokens x head slots per workgroup of the grid, which holds min(items at the
    base size, resident workgroups)."""

    grid = min(len(contexts) * heads_per_seq * -(-table_tokens // base), capacity)
    work = min(sum(max(0, min(c, table_tokens)) for c in contexts) * heads_per_seq // grid, 1 << 40)
    limit = base
    while 2 * limit <= GROW_MAX_TOKENS and 2 * limit // block_size <= 256 and 2 * limit < table_tokens:
        limit *= 2
    size = base
    while 2 * size <= limit and (2 * size) ** 2 <= GROW_BALANCE * work:
        size *= 2
    return size


def _capacity(gpu):
    import torch

    return 2 * torch.cuda.get_device_properties(gpu).multi_processor_count


def device_case(gpu, *, batch, contexts, table_tokens, dtype="bf16", seed=0, kv_heads=8, query_heads=32,
                head_dim=128, block_size=16):
    """Inputs built on the GPU (caches of several GB would take minutes on the host): disjoint
    random blocks per sequence, padding entries 0."""

    import torch

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    gen = torch.Generator(device=gpu).manual_seed(seed)
    max_blocks = table_tokens // block_size
    needed = [max(1, -(-c // block_size)) for c in contexts]
    num_blocks = sum(needed) + 3
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    rows, cursor = [], 0
    for n in needed:
        rows.append(perm[cursor:cursor + n] + [0] * (max_blocks - n))
        cursor += n
    shape = (num_blocks, block_size, kv_heads, head_dim)
    return {
        "query": torch.randn(batch, query_heads, head_dim, generator=gen, device=gpu).to(tdt),
        "key_cache": torch.randn(shape, generator=gen, device=gpu).to(tdt),
        "value_cache": torch.randn(shape, generator=gen, device=gpu).to(tdt),
        "block_tables": torch.tensor(rows, dtype=torch.int32, device=gpu),
        "context_lengths": torch.tensor(contexts, dtype=torch.int32, device=gpu),
    }


def _check_against_fixed(palib, d, base, what):
    """Two-launch and fused growing calls against calls without growth at the size that ran."""

    import torch

    ws = _workspace(palib, d, base)
    grown = palib.decode(*_args(d), partition_tokens=base, workspace=ws, grow=True)
    size = _grown_size(ws)
    grown_fused = palib.decode(*_args(d), partition_tokens=base, phase="fused", grow=True)
    fixed = palib.decode(*_args(d), partition_tokens=size)
    fixed_fused = palib.decode(*_args(d), partition_tokens=size, phase="fused")
    torch.cuda.synchronize()
    for name, out in (("grown fused", grown_fused), ("fixed", fixed), ("fixed fused", fixed_fused)):
        assert torch.equal(out.view(torch.int16), grown.view(torch.int16)), f"{what}: {name} differs"
    return grown, size


@pytest.fixture(scope="module")
def ragged96(gpu):
    """96 sequences of 1-4096 tokens (a 4096-token table), GQA 32x8, head_dim 128, bf16."""

    import torch

    rng = random.Random(96)
    contexts = [rng.randint(1, 4096) for _ in range(96)]
    contexts[:3] = [1, 4096, 4095]
    case = make_case(torch, batch=96, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                     contexts=contexts, max_blocks=256, dtype="bf16", seed=96)
    return case, to_device(case, gpu), oracle64_rows(case)


def test_growth_matches_fixed_size_and_oracle(gpu, palib, ragged96):
    case, d, expected = ragged96
    announce("partition growth: 96 ragged sequences, base 256")
    assert palib.schedule(96, 32, 8, 128, 16, 256, "bf16", 256) == "queue"
    out, size = _check_against_fixed(palib, d, 256, "ragged96")
    assert size == expected_size(case["context_lengths"].tolist(), 4096, 8, 256, 16, _capacity(gpu)) > 256
    assert_within(out, expected, "bf16", "ragged96 grown")


@pytest.mark.parametrize("batch, lo, hi, best", [(64, 4096, 16384, 2048), (32, 8192, 32768, 2048),
                                                 (256, 1024, 8192, 4096)])
def test_long_contexts_grow_to_the_measured_fastest_size(gpu, palib, batch, lo, hi, best):
    rng = random.Random(batch + hi)
    contexts = [rng.randint(lo, hi) for _ in range(batch)]
    announce(f"partition growth: b{batch} {lo}-{hi} tokens")
    d = device_case(gpu, batch=batch, contexts=contexts, table_tokens=hi, seed=batch)
    _, size = _check_against_fixed(palib, d, 256, f"b{batch}")
    assert size == expected_size(contexts, hi, 8, 256, 16, _capacity(gpu)) == best


def test_wide_table_with_short_contexts_keeps_the_base_size(gpu, palib):
    """A table sized for 64k tokens (256 partitions of the base size, the queue's limit) holding
    1k-3k-token sequences: the size follows the live contexts (1024 tokens, measured fastest on
    such a batch), not the table (which would allow 4096)."""

    rng = random.Random(7)
    contexts = [rng.randint(1024, 3072) for _ in range(32)]
    announce("partition growth: 64k-token table, short contexts")
    d = device_case(gpu, batch=32, contexts=contexts, table_tokens=65536, seed=7)
    assert palib.schedule(32, 32, 8, 128, 16, 4096, "bf16", 256) == "queue"
    _, size = _check_against_fixed(palib, d, 256, "wide table")
    assert size == expected_size(contexts, 65536, 8, 256, 16, _capacity(gpu)) == 1024


@pytest.mark.parametrize("batch, lo, hi", [(32, 1024, 3072), (8, 32768, 131072)])
def test_table_too_wide_for_the_queue_starts_from_a_larger_size(gpu, palib, batch, lo, hi):
    """A 128k-token table has 512 partitions of 256 tokens, more than the queue's item map holds:
    without growth the call takes the grid schedule at 256; with growth it starts from 512 (256
    partitions) on the work queue and grows from there."""

    rng = random.Random(batch + lo)
    contexts = [rng.randint(lo, hi) for _ in range(batch)]
    announce(f"partition growth: 128k-token table, b{batch} {lo}-{hi} tokens")
    assert palib.schedule(batch, 32, 8, 128, 16, 8192, "bf16", 256) == "grid"
    assert palib.schedule(batch, 32, 8, 128, 16, 8192, "bf16", 256, grow=True) == "queue"
    assert palib.schedule(batch, 32, 8, 128, 16, 8192, "bf16", 256, schedule="grid", grow=True) == "grid"
    d = device_case(gpu, batch=batch, contexts=contexts, table_tokens=131072, seed=batch)
    _, size = _check_against_fixed(palib, d, 256, f"128k table b{batch}")
    assert size == expected_size(contexts, 131072, 8, 512, 16, _capacity(gpu)) > 512


def test_growth_off_the_queue_changes_nothing(gpu, palib):
    """A grid-schedule shape: the bit changes nothing and header word 1 is not written."""

    import torch

    case = make_case(torch, batch=4, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                     contexts=[3000, 1, 1500, 2048], dtype="fp16", seed=4)
    d = to_device(case, gpu)
    announce("partition growth: grid schedule")
    assert palib.schedule(4, 32, 8, 128, 16, int(d["block_tables"].shape[1]), "fp16", 256) == "grid"
    ws = _workspace(palib, d, 256)
    grown = palib.decode(*_args(d), partition_tokens=256, workspace=ws, grow=True)
    fixed = palib.decode(*_args(d), partition_tokens=256)
    torch.cuda.synchronize()
    assert _grown_size(ws) == 0
    assert torch.equal(grown.view(torch.int16), fixed.view(torch.int16))


def test_growth_through_phase_entries_and_noalloc(gpu, palib, ragged96):
    import torch

    _, d, _ = ragged96
    announce("partition growth: phase entries and no-allocation entry")
    ws = _workspace(palib, d, 256)
    whole = palib.decode(*_args(d), partition_tokens=256, workspace=ws, grow=True)
    out = torch.empty_like(d["query"])
    ws2 = _workspace(palib, d, 256)
    palib.decode(*_args(d), partition_tokens=256, out=out, workspace=ws2, phase="partitions", grow=True)
    palib.decode(*_args(d), partition_tokens=256, out=out, workspace=ws2, phase="reduce", grow=True)
    noalloc = palib.decode_noalloc(*_args(d), out=torch.empty_like(d["query"]), partition_tokens=256, grow=True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), whole.view(torch.int16))
    assert torch.equal(noalloc.view(torch.int16), whole.view(torch.int16))


def test_growth_with_append_and_decode(gpu, palib, ragged96):
    """Append-and-decode grows like a plain decode (the caches receive the same rows each call)."""

    import torch

    case, d, _ = ragged96
    gen = torch.Generator(device=gpu).manual_seed(11)
    k = d["key_cache"].clone()
    v = d["value_cache"].clone()
    new_k = torch.randn(96, 8, 128, generator=gen, device=gpu).to(torch.bfloat16)
    new_v = torch.randn(96, 8, 128, generator=gen, device=gpu).to(torch.bfloat16)
    args = (d["query"], k, v, d["block_tables"], d["context_lengths"])
    announce("partition growth: append-and-decode")
    ws = _workspace(palib, d, 256)
    grown = palib.decode(*args, partition_tokens=256, workspace=ws, new_key=new_k, new_value=new_v, grow=True)
    size = _grown_size(ws)
    grown_fused = palib.decode(*args, partition_tokens=256, phase="fused", new_key=new_k, new_value=new_v, grow=True)
    fixed = palib.decode(*args, partition_tokens=size, new_key=new_k, new_value=new_v)
    torch.cuda.synchronize()
    assert size == expected_size(case["context_lengths"].tolist(), 4096, 8, 256, 16, _capacity(gpu)) > 256
    assert torch.equal(grown_fused.view(torch.int16), grown.view(torch.int16))
    assert torch.equal(fixed.view(torch.int16), grown.view(torch.int16))


def test_public_broad_region_grows_and_captures(gpu, palib, ragged96):
    import torch

    import radeon_kernels as rk

    _, d, expected = ragged96
    ws = _workspace(palib, d, 256)
    palib.decode(*_args(d), partition_tokens=256, workspace=ws, grow=True)
    size = _grown_size(ws)
    announce("partition growth: rk.paged_attention_decode broad region")
    eager = rk.paged_attention_decode(*_args(d))
    record = rk.get_last_dispatch()
    assert record["entry_id"] == "paged_attention_decode-gfx950-region"
    assert record["launch"]["grow_partitions"] is True
    from radeon_kernels.cabi import LIBRARY_PATH
    import importlib.util

    spec = importlib.util.spec_from_file_location("rk_pa_gfx950", LIBRARY_PATH.parent / "rk_pa_gfx950.so")
    binding = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(binding)
    scale = 128 ** -0.5
    fixed = binding.decode_mfma(*_args(d), scale, partition_tokens=size, merge="fused")
    torch.cuda.synchronize()
    assert torch.equal(eager.view(torch.int16), fixed.view(torch.int16))
    assert_within(eager, expected, "bf16", "broad region grown")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            rk.paged_attention_decode(*_args(d))
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = rk.paged_attention_decode(*_args(d))
    for _ in range(3):
        scratch = torch.randn(1 << 20, device=gpu)  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16))
        del scratch
