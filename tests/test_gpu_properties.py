"""Size-independent properties of the decode on the full 128-sequence ragged workload, bit for bit.

Each property fixes the exact output of a transformed call from the output of the original one, so it
holds at any size without an oracle:
  * relabelling the physical cache blocks (moving every block and rewriting the block tables to match)
    changes nothing: the kernel reaches K/V only through the tables;
  * permuting the sequences (queries, tables and context lengths together) permutes the output rows:
    which workgroup runs an item, and in what order the work queue hands items out, do not change
    the item's arithmetic or the fixed merge order;
  * doubling V doubles the output exactly: scaling by two is exact in bf16 and fp32, the probabilities
    do not depend on V, and every step from the PV products to the final rounding commutes with it.
The partitions cover the work queue with two KV heads per workgroup (8192 tokens) and with one (2048).
"""

from __future__ import annotations

import pytest

from _helpers import announce

pytestmark = pytest.mark.gpu

PARTITIONS = (8192, 2048)
PHASES = ("fused", "all")


def _bits(torch, x):
    return x.contiguous().view(torch.int16)


def _decode(palib, data, *, query=None, key_cache=None, value_cache=None, block_tables=None,
            context_lengths=None, partition, phase):
    return palib.decode(data["query"] if query is None else query,
                        data["key_cache"] if key_cache is None else key_cache,
                        data["value_cache"] if value_cache is None else value_cache,
                        data["block_tables"] if block_tables is None else block_tables,
                        data["context_lengths"] if context_lengths is None else context_lengths,
                        partition_tokens=partition, phase=phase)


@pytest.mark.parametrize("phase", PHASES)
@pytest.mark.parametrize("partition", PARTITIONS)
def test_block_relabelling_is_invisible(gpu, palib, c5_case, partition, phase):
    import torch

    data = c5_case["gpu"]
    k, v, bt = data["key_cache"], data["value_cache"], data["block_tables"]
    n = k.shape[0]
    announce(f"c5 block relabelling, {n} blocks, P {partition}, {phase}")
    base = _decode(palib, data, partition=partition, phase=phase)
    gen = torch.Generator().manual_seed(20261207 + partition)
    new_slot = torch.randperm(n, generator=gen).to(gpu)  # block i moves to slot new_slot[i]
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[new_slot] = k
    v2[new_slot] = v
    valid = (bt >= 0) & (bt < n)
    bt2 = torch.where(valid, new_slot[bt.long().clamp(0, n - 1)].to(bt.dtype), bt)
    assert not torch.equal(bt2, bt)
    moved = _decode(palib, data, key_cache=k2, value_cache=v2, block_tables=bt2, partition=partition, phase=phase)
    torch.cuda.synchronize()
    assert torch.equal(_bits(torch, moved), _bits(torch, base))
    del k2, v2, bt2, moved
    torch.cuda.empty_cache()


@pytest.mark.parametrize("phase", PHASES)
@pytest.mark.parametrize("partition", PARTITIONS)
def test_sequence_permutation_permutes_rows(gpu, palib, c5_case, partition, phase):
    import torch

    data = c5_case["gpu"]
    batch = data["query"].shape[0]
    announce(f"c5 sequence permutation, {batch} sequences, P {partition}, {phase}")
    base = _decode(palib, data, partition=partition, phase=phase)
    gen = torch.Generator().manual_seed(20261208 + partition)
    order = torch.randperm(batch, generator=gen).to(gpu)
    permuted = _decode(palib, data, query=data["query"][order].contiguous(),
                       block_tables=data["block_tables"][order].contiguous(),
                       context_lengths=data["context_lengths"][order].contiguous(), partition=partition, phase=phase)
    torch.cuda.synchronize()
    assert not torch.equal(order.cpu(), torch.arange(batch))
    assert torch.equal(_bits(torch, permuted), _bits(torch, base[order]))


@pytest.mark.parametrize("phase", PHASES)
@pytest.mark.parametrize("partition", PARTITIONS)
def test_doubling_v_doubles_the_output(gpu, palib, c5_case, partition, phase):
    import torch

    data = c5_case["gpu"]
    v = data["value_cache"]
    announce(f"c5 V doubled, P {partition}, {phase}")
    assert float(v.abs().max()) < 1e30  # far from bf16 overflow after doubling
    base = _decode(palib, data, partition=partition, phase=phase)
    doubled = _decode(palib, data, value_cache=v * 2, partition=partition, phase=phase)
    torch.cuda.synchronize()
    assert torch.isfinite(base.float()).all()
    assert torch.equal(_bits(torch, doubled), _bits(torch, (base.float() * 2).to(base.dtype)))
    del doubled
    torch.cuda.empty_cache()
