"""Work-queue schedule of the partition kernel (RK_PA_SCHEDULE_QUEUE) against the one-workgroup-per-item
grid (RK_PA_SCHEDULE_GRID).

Both schedules run the same per-item code, so outputs must be bit-identical (compared as raw bits,
NaN rows of empty contexts included); the queue form is also checked against the float64 oracle.
The cases cover what the queue's item map is built from: ragged contexts whose partition counts
differ per sequence, empty and negative contexts (one NaN item), contexts past the table, int32 and
int64 indices, head chunks of 1, 2 and 4 query heads (and two chunks per KV head), block sizes below
a tile, every head_dim, the fused, two-launch, phase-split, append and allocation-free entries, a
garbage-filled workspace header, repeated calls and a smaller call after a larger one, and the calls
on which the queue runs two KV heads per workgroup: the 128-sequence ragged workload (also under graph
capture) and six other layouts (head chunks of 4, 2 and 1, blocks of 16 to 128 tokens, both dtypes and
index types, one to eight KV-head pairs per sequence).
"""

from __future__ import annotations

import pytest

from _helpers import announce, assert_within, make_case, oracle64, to_device

pytestmark = pytest.mark.gpu


def same_bits(a, b) -> bool:
    import torch

    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def ragged_contexts(batch, limit, seed):
    """Context lengths in [1, limit] with an empty, a negative and a past-the-table length mixed in."""

    import random

    rng = random.Random(seed)
    contexts = [rng.randint(1, limit) for _ in range(batch)]
    contexts[1] = 0
    contexts[batch // 2] = -3
    contexts[-2] = limit + 77  # clamped to the table
    contexts[-1] = limit
    return contexts


# (query_heads, kv_heads, head_dim, block_size, dtype, index_dtype, partition): head chunks of 4, 1,
# 2 and 8 (group 8 at head_dim 256: one chunk of 8 with PV on MFMA, two chunks of 4 otherwise); blocks of
# 16, 32, 8 and 1 tokens; every head_dim; and multi-query (one KV head, four 8-head chunks).
SHAPES = [
    (32, 8, 128, 16, "bf16", "int32", 128),
    (16, 16, 64, 32, "bf16", "int64", 64),
    (16, 8, 128, 8, "fp16", "int64", 128),
    (64, 8, 128, 1, "bf16", "int32", 64),
    (32, 8, 256, 16, "fp16", "int32", 128),
    (64, 8, 256, 16, "bf16", "int32", 256),
    (32, 1, 128, 16, "fp16", "int32", 128),
]


def shape_id(shape):
    hq, hkv, d, bs, dtype, index, partition = shape
    return f"h{hq}x{hkv}-d{d}-bs{bs}-{dtype}-{index}-p{partition}"


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
@pytest.mark.parametrize("shape", SHAPES, ids=shape_id)
def test_queue_matches_grid_and_oracle(gpu, palib, shape, variant):
    import torch

    hq, hkv, d, bs, dtype, index, partition = shape
    batch, limit = 40, 1000
    contexts = ragged_contexts(batch, limit, seed=d + bs)
    max_blocks = -(-limit // bs)
    case = make_case(torch, batch=batch, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=bs,
                     contexts=contexts, max_blocks=max_blocks, dtype=dtype, index_dtype=index, seed=11)
    dev = to_device(case, gpu)
    args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    announce(f"queue vs grid {shape_id(shape)} batch {batch} variant={variant}")
    grid = palib.decode(*args, partition_tokens=partition, schedule="grid", variant=variant)
    queue = palib.decode(*args, partition_tokens=partition, schedule="queue", variant=variant)
    auto = palib.decode(*args, partition_tokens=partition, variant=variant)
    torch.cuda.synchronize()
    assert same_bits(queue, grid)
    assert same_bits(auto, grid)
    assert_within(queue, oracle64(case), dtype, f"queue {shape_id(shape)}")


@pytest.mark.parametrize("phase", ["fused", "split"])
def test_queue_in_every_launch_form(gpu, palib, phase):
    import torch

    batch, limit, bs, partition = 48, 2048, 16, 128
    case = make_case(torch, batch=batch, query_heads=32, kv_heads=8, head_dim=128, block_size=bs,
                     contexts=ragged_contexts(batch, limit, seed=3), max_blocks=limit // bs, seed=5)
    dev = to_device(case, gpu)
    args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    announce(f"queue launch form {phase}")
    expected = palib.decode(*args, partition_tokens=partition, schedule="grid")
    if phase == "fused":
        counters = torch.zeros(palib.counter_words(batch, 32, 8), dtype=torch.int32, device=gpu)
        got = palib.decode(*args, partition_tokens=partition, phase="fused", counters=counters, schedule="queue")
        again = palib.decode(*args, partition_tokens=partition, phase="fused", counters=counters, schedule="queue")
        torch.cuda.synchronize()
        assert same_bits(again, got)
        assert int(counters.abs().sum()) == 0  # every arrival counter left zero
        reference = palib.decode(*args, partition_tokens=partition, phase="fused", counters=counters,
                                 schedule="grid")
        torch.cuda.synchronize()
        assert same_bits(got, reference)
    else:
        need = palib.workspace_bytes(batch, 32, 128, bs, limit // bs, partition)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        out = torch.empty_like(dev["query"])
        palib.decode(*args, partition_tokens=partition, out=out, workspace=ws, phase="partitions", schedule="queue")
        palib.decode(*args, partition_tokens=partition, out=out, workspace=ws, phase="reduce")
        torch.cuda.synchronize()
        assert same_bits(out, expected)


def test_garbage_header_repeated_and_shrinking_calls(gpu, palib):
    """The ticket counter is zeroed in front of every queue launch: a workspace full of 0xFF, repeated
    calls on it, and a smaller call after a larger one all give the grid schedule's outputs."""

    import torch

    bs, partition, limit = 16, 128, 1536
    big = make_case(torch, batch=64, query_heads=32, kv_heads=8, head_dim=128, block_size=bs,
                    contexts=ragged_contexts(64, limit, seed=8), max_blocks=limit // bs, seed=2)
    small = make_case(torch, batch=6, query_heads=32, kv_heads=8, head_dim=128, block_size=bs,
                      contexts=ragged_contexts(6, limit, seed=9), max_blocks=limit // bs, seed=4)
    need = palib.workspace_bytes(64, 32, 128, bs, limit // bs, partition)
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=gpu)
    for name, case in (("big", big), ("small", small), ("big", big)):
        dev = to_device(case, gpu)
        args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
        announce(f"queue reuse {name}")
        expected = palib.decode(*args, partition_tokens=partition, schedule="grid")
        for _ in range(3):
            got = palib.decode(*args, partition_tokens=partition, workspace=ws, schedule="queue")
            torch.cuda.synchronize()
            assert same_bits(got, expected)


def test_append_and_noalloc_on_the_queue(gpu, palib, kvlib):
    import torch

    from test_gpu_append_decode import new_rows, new_token_slots

    batch, limit, bs, partition = 40, 1024, 16, 64
    case = make_case(torch, batch=batch, query_heads=32, kv_heads=8, head_dim=128, block_size=bs,
                     contexts=ragged_contexts(batch, limit, seed=21), max_blocks=limit // bs, seed=6)
    dev = to_device(case, gpu)
    q, kc, vc, bt, cl = (dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths"))
    announce("queue append-and-decode")
    nk, nv = new_rows(torch, q, 8, seed=13)
    ref_k, ref_v = kc.clone(), vc.clone()
    kvlib.append(nk, nv, ref_k, ref_v, new_token_slots(torch, bt, cl, bs))
    expected = palib.decode(q, ref_k, ref_v, bt, cl, partition_tokens=partition, schedule="grid")
    got_k, got_v = kc.clone(), vc.clone()
    got = palib.decode(q, got_k, got_v, bt, cl, partition_tokens=partition, new_key=nk, new_value=nv,
                       schedule="queue")
    torch.cuda.synchronize()
    assert same_bits(got, expected)
    assert torch.equal(got_k, ref_k) and torch.equal(got_v, ref_v)

    announce("queue allocation-free decode")
    plain = palib.decode(q, kc, vc, bt, cl, partition_tokens=partition, schedule="grid")
    out = torch.empty_like(q)
    palib.decode_noalloc(q, kc, vc, bt, cl, out=out, partition_tokens=partition, schedule="queue")
    torch.cuda.synchronize()
    assert same_bits(out, plain)


def test_queue_with_fewer_items_than_workgroups(gpu, palib):
    """Forced onto a grid that fits the device at once: the workgroups past the item count exit."""

    import torch

    case = make_case(torch, batch=3, query_heads=8, kv_heads=2, head_dim=128, block_size=16,
                     contexts=[300, 0, 129], max_blocks=20, seed=1)
    dev = to_device(case, gpu)
    args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    announce("queue small grid")
    grid = palib.decode(*args, partition_tokens=64, schedule="grid")
    queue = palib.decode(*args, partition_tokens=64, schedule="queue")
    torch.cuda.synchronize()
    assert same_bits(queue, grid)
    assert_within(queue, oracle64(case), "bf16", "queue small grid")


def test_ragged_b128_workload_schedules_agree(gpu, palib, c5_case):
    """The 128-sequence ragged workload (8192 work items) takes the queue by default."""

    import torch

    dev = c5_case["gpu"]
    args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    for variant in ("mfma", "mfma_qk"):
        announce(f"queue b128 ragged P=2048 variant={variant}")
        grid = palib.decode(*args, partition_tokens=2048, schedule="grid", variant=variant)
        auto = palib.decode(*args, partition_tokens=2048, variant=variant)
        torch.cuda.synchronize()
        assert same_bits(auto, grid)


def test_schedule_query_names_what_runs(gpu, palib):
    """rk_pa_decode_schedule: the ragged 128-sequence workload (8192 items) takes the queue, a grid
    the device holds at once keeps one workgroup per item, and the forcing bits are reported back."""

    from benchmarks.workloads import WORKLOADS

    announce("schedule query")
    for key, partition, expected in (("c5", 4096, "queue"), ("c5", 2048, "queue"), ("c2", 256, "grid"),
                                     ("c3", 512, "grid"), ("c1", 128, "grid")):
        w = WORKLOADS[key]
        args = (w.batch, w.query_heads, w.kv_heads, w.head_dim, w.block_size, w.max_blocks, w.dtype, partition)
        assert palib.schedule(*args) == expected, key
        assert palib.schedule(*args, schedule="grid") == "grid"
        if partition < w.max_blocks * w.block_size:  # split-K: the queue can be forced
            assert palib.schedule(*args, schedule="queue") == "queue"
    assert palib.schedule(128, 32, 8, 128, 16, 1024, "bf16", 2048, variant="valu") == "grid"
    # Partitions under 256 tokens keep the grid by default (the queue can still be forced).
    assert palib.schedule(128, 32, 8, 128, 16, 1024, "bf16", 128) == "grid"
    assert palib.schedule(128, 32, 8, 128, 16, 1024, "bf16", 128, schedule="queue") == "queue"
    assert palib.schedule(128, 32, 8, 128, 16, 1024, "bf16", 256) == "queue"


def test_queue_under_graph_capture_replays_match_eager(gpu, palib):
    """The public call on a queue-scheduled shape, captured into a HIP graph: the capture takes the
    two-launch form, whose ticket counter a one-thread kernel zeroes in front of every replay."""

    import torch

    import radeon_kernels as rk

    batch, limit, bs = 48, 2048, 16
    case = make_case(torch, batch=batch, query_heads=32, kv_heads=8, head_dim=128, block_size=bs,
                     contexts=ragged_contexts(batch, limit, seed=31), max_blocks=limit // bs, seed=9)
    dev = to_device(case, gpu)
    args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    announce("queue graph capture")
    eager = rk.paged_attention_decode(*args)
    record = rk.get_last_dispatch()
    partition = int(record["launch"]["partition_tokens"])
    assert palib.schedule(batch, 32, 8, 128, bs, limit // bs, "bf16", partition) == "queue", record["launch"]
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
        assert same_bits(captured, eager)
        del scratch


@pytest.mark.parametrize("partition", [8192, 4096])
def test_kv_head_pairs_match_the_grid(gpu, palib, c5_case, partition):
    """The 128-sequence ragged workload at partitions of at least 4096 tokens: 1024 (sequence, KV head)
    rows and head chunks of 4, so the work queue runs two KV heads per 8-wave workgroup.  Each KV head
    runs as in a one-head workgroup, so every form must match the one-head grid bit for bit: fused,
    two-launch and allocation-free; and the float64 oracle within the bf16 bar."""

    import torch

    data = c5_case["gpu"]
    args = [data[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    batch, query_heads, head_dim = (int(s) for s in data["query"].shape)
    _, block_size, kv_heads, _ = (int(s) for s in data["key_cache"].shape)
    max_blocks = int(data["block_tables"].shape[1])
    assert batch * kv_heads >= 1024
    assert palib.schedule(batch, query_heads, kv_heads, head_dim, block_size, max_blocks, "bf16", partition) == "queue"
    announce(f"c5 KV-head pairs, partition {partition}")
    grid = palib.decode(*args, partition_tokens=partition, phase="fused", schedule="grid")
    fused = palib.decode(*args, partition_tokens=partition, phase="fused")
    two_launch = palib.decode(*args, partition_tokens=partition)
    out = torch.empty_like(data["query"])
    noalloc = palib.decode_noalloc(*args, out=out, partition_tokens=partition)
    torch.cuda.synchronize()
    for name, got in (("fused", fused), ("two-launch", two_launch), ("allocation-free", noalloc)):
        assert same_bits(got, grid), f"{name} work queue differs from the grid at partition {partition}"
    assert_within(fused.cpu(), c5_case["expected"], "bf16", f"c5 pairs P{partition}")


# (query_heads, kv_heads, block_size, dtype, index_dtype, batch, limit): layouts the work queue pairs KV
# heads on besides the 128-sequence workload: head chunks of 4, 2 and 1, blocks of 16 to 128 tokens, both
# dtypes and index types, and 16, 6 (three pairs per sequence) and 2 (one pair) KV heads.
PAIR_LAYOUTS = [
    (32, 8, 64, "fp16", "int64", 128, 8192),
    (16, 8, 128, "bf16", "int32", 128, 8192),
    (8, 8, 32, "bf16", "int64", 128, 8192),
    (16, 16, 16, "fp16", "int32", 64, 8192),
    (24, 6, 32, "bf16", "int32", 176, 8192),
    (8, 2, 16, "fp16", "int64", 512, 4608),
]


@pytest.mark.parametrize("layout", PAIR_LAYOUTS, ids=lambda s: f"h{s[0]}x{s[1]}-bs{s[2]}-{s[3]}-{s[4]}-b{s[5]}-c{s[6]}")
def test_kv_head_pairs_on_other_layouts(gpu, palib, layout):
    """At least 1024 (sequence, KV head) rows at partitions of 4096 tokens: the work queue runs two KV
    heads per 8-wave workgroup.  Ragged contexts (one and two partitions, empty, negative and past the
    table) must match the one-head grid bit for bit, fused and two-launch, and the float64 oracle on
    sampled sequences (the edge ones included)."""

    import torch

    hq, hkv, bs, dtype, index, batch, limit = layout
    partition = 4096
    assert batch * hkv >= 1024 and hkv % 2 == 0 and hq // hkv <= 4
    contexts = ragged_contexts(batch, limit, seed=bs + hq)
    case = make_case(torch, batch=batch, query_heads=hq, kv_heads=hkv, head_dim=128, block_size=bs,
                     contexts=contexts, max_blocks=limit // bs, dtype=dtype, index_dtype=index, seed=hkv + bs)
    dev = to_device(case, gpu)
    args = [dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    assert palib.schedule(batch, hq, hkv, 128, bs, limit // bs, dtype, partition) == "queue"
    announce(f"KV-head pairs h{hq}x{hkv} bs{bs} {dtype} {index} batch {batch}")
    grid = palib.decode(*args, partition_tokens=partition, phase="fused", schedule="grid")
    fused = palib.decode(*args, partition_tokens=partition, phase="fused")
    two_launch = palib.decode(*args, partition_tokens=partition)
    torch.cuda.synchronize()
    assert same_bits(fused, grid)
    assert same_bits(two_launch, grid)
    sampled = sorted({0, 1, 2, 3, batch // 2, batch // 2 + 1, batch - 3, batch - 2, batch - 1})
    assert_within(fused[sampled].cpu(), oracle64(case, sequences=sampled), dtype, f"pairs h{hq}x{hkv} bs{bs}")


def test_kv_head_pairs_under_graph_capture(gpu, c5_case):
    """The public call on the 128-sequence workload (its exact dispatch entry: partitions of 8192, two KV
    heads per work-queue workgroup) captured into a HIP graph: the capture takes the two-launch form (ticket
    reset kernel, paired queue kernel, reduce kernel); every replay must equal the eager fused call bit for
    bit, with unrelated eager work between replays."""

    import torch

    import radeon_kernels as rk

    data = c5_case["gpu"]
    args = [data[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths")]
    announce("c5 KV-head pairs under graph capture")
    eager = rk.paged_attention_decode(*args)
    record = rk.get_last_dispatch()
    assert int(record["launch"]["partition_tokens"]) == 8192, record["launch"]
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
        assert same_bits(captured, eager)
        del scratch
    del graph
