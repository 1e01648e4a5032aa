"""Batches of more than 1024 sequences: the library runs them as launches of 1024 sequences (the last
shorter) on offset views of the same buffers, each launch choosing its own schedule and, with
RK_PA_PARTITION_GROW, its own partition size (workspace header word 1 + launch).

Parity: the launches agree bit for bit with the single grid launch of the whole batch, in both merge
forms and through the phase entries and append-and-decode; each launch's rows of a growing call equal
a call without growth at the size that launch ran; sampled rows on both sides of the launch boundary
match the float64 oracle (src/radeon_kernels/ops/paged_attention/reference.py:7-47 restated in
oracle/).
"""

from __future__ import annotations

import random

import pytest

from _helpers import announce, assert_within, make_case, oracle64, to_device

pytestmark = pytest.mark.gpu

BATCH = 1030  # a launch of 1024 sequences, then one of 6


@pytest.fixture(scope="module")
def big(gpu):
    """1030 sequences of 1-2048 tokens (a 2048-token table), GQA 8x2, head_dim 128, fp16."""

    import torch

    rng = random.Random(1030)
    contexts = [rng.randint(1, 2048) for _ in range(BATCH)]
    contexts[1023:1026] = [2048, 1, 1500]
    case = make_case(torch, batch=BATCH, query_heads=8, kv_heads=2, head_dim=128, block_size=16,
                     contexts=contexts, max_blocks=128, dtype="fp16", seed=1030)
    return case, to_device(case, gpu)


def _args(d):
    return d["query"], d["key_cache"], d["value_cache"], d["block_tables"], d["context_lengths"]


def _same(a, b):
    import torch

    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_launches_of_1024_match_one_grid_launch_and_the_oracle(gpu, palib, big):
    import torch

    case, d = big
    announce("1030 sequences: launches of 1024 and 6 against one grid launch")
    assert palib.schedule(BATCH, 8, 2, 128, 16, 128, "fp16", 256) == "queue"
    grid = palib.decode(*_args(d), partition_tokens=256, schedule="grid")
    outs = {
        "auto": palib.decode(*_args(d), partition_tokens=256),
        "queue": palib.decode(*_args(d), partition_tokens=256, schedule="queue"),
        "fused": palib.decode(*_args(d), partition_tokens=256, phase="fused"),
        "fused queue": palib.decode(*_args(d), partition_tokens=256, phase="fused", schedule="queue"),
    }
    torch.cuda.synchronize()
    for name, out in outs.items():
        assert _same(out, grid), name
    rows = sorted({0, 1, 511, 1022, 1023, 1024, 1025, 1026, 1029} | set(random.Random(5).sample(range(BATCH), 23)))
    expected = oracle64(case, sequences=rows)
    assert_within(grid[rows], expected, "fp16", "sampled rows")


def test_each_launch_grows_on_its_own(gpu, palib, big):
    """The first launch (1024 sequences, 16384 items) runs the queue and grows to 1024 tokens; the
    second (6 sequences, 96 items) runs the grid at 256 and leaves its header word unwritten."""

    import torch

    _, d = big
    announce("1030 sequences: partition growth per launch")
    need = palib.workspace_bytes(BATCH, 8, 128, 16, 128, 256)
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    grown = palib.decode(*_args(d), partition_tokens=256, workspace=ws, grow=True)
    fused = palib.decode(*_args(d), partition_tokens=256, phase="fused", grow=True)
    split = torch.empty_like(d["query"])
    ws2 = torch.zeros(need, dtype=torch.uint8, device=gpu)
    palib.decode(*_args(d), partition_tokens=256, out=split, workspace=ws2, phase="partitions", grow=True)
    palib.decode(*_args(d), partition_tokens=256, out=split, workspace=ws2, phase="reduce", grow=True)
    torch.cuda.synchronize()
    words = ws[:16].view(torch.int32).tolist()
    assert words[1:4] == [1024, 0, 0], words
    sizes = [1024, 256]
    assert _same(fused, grown) and _same(split, grown)
    for launch, (lo, hi) in enumerate(((0, 1024), (1024, BATCH))):
        fixed = palib.decode(*_args(d), partition_tokens=sizes[launch])
        torch.cuda.synchronize()
        assert _same(fixed[lo:hi], grown[lo:hi]), f"launch {launch} at {sizes[launch]} tokens"


def test_append_and_decode_over_1024_sequences(gpu, palib, kvlib, big):
    """Grid and fused work-queue append-and-decode, each on its own fresh copy of the caches: equal
    outputs, and caches equal to what kv_cache_append of the same rows writes into a third copy."""

    import torch

    _, d = big
    gen = torch.Generator(device=gpu).manual_seed(3)
    new_k = torch.randn(BATCH, 2, 128, generator=gen, device=gpu).to(torch.float16)
    new_v = torch.randn(BATCH, 2, 128, generator=gen, device=gpu).to(torch.float16)
    bt, cl = d["block_tables"], d["context_lengths"]
    announce("1030 sequences: append-and-decode")
    caches = {}
    outs = {}
    for form, extra in (("grid", dict(schedule="grid")), ("queue", dict(phase="fused"))):
        k, v = d["key_cache"].clone(), d["value_cache"].clone()
        outs[form] = palib.decode(d["query"], k, v, bt, cl, partition_tokens=256, new_key=new_k, new_value=new_v,
                                  **extra)
        caches[form] = (k, v)
    # The same rows through kv_cache_append: slot of position context_length - 1 (every context here
    # lies inside the table).
    bs = d["key_cache"].shape[1]
    pos = cl.long() - 1
    slots = bt.long().gather(1, (pos // bs).unsqueeze(1)).squeeze(1) * bs + pos % bs
    k_ref, v_ref = d["key_cache"].clone(), d["value_cache"].clone()
    kvlib.append(new_k, new_v, k_ref, v_ref, slots)
    torch.cuda.synchronize()
    assert _same(outs["queue"], outs["grid"])
    assert not torch.equal(k_ref, d["key_cache"])  # the appends wrote something
    for form, (k, v) in caches.items():
        assert torch.equal(k, k_ref) and torch.equal(v, v_ref), f"{form} form's caches differ from kv_cache_append"
