"""Guard bands: the decode kernels write nothing outside the output, the split-K workspace and the
arrival counters.

Each of the three buffers is carved out of a larger buffer whose margins hold a sentinel byte
pattern; after the partition launch, the reduce launch and the fused launch the margins must be
intact (the pattern of reference benchmarks/gemm/asmevo_worker.py:363-372, applied to every buffer a
decode launch writes).  The output itself starts filled with the sentinel too, and must be fully
overwritten: a row the kernels forgot would keep it.
"""

from __future__ import annotations

import pytest

from _helpers import announce, assert_within, oracle64, to_device

pytestmark = pytest.mark.gpu

GUARD = 1 << 16      # bytes of sentinel on each side of every buffer (a multiple of 256)
SENTINEL = 0xA5


class Guarded:
    """A ``nbytes`` region (256-byte aligned) inside a sentinel-filled buffer with GUARD bytes per side."""

    def __init__(self, torch, nbytes, device):
        self.nbytes = nbytes
        self.buffer = torch.full((nbytes + 2 * GUARD,), SENTINEL, dtype=torch.uint8, device=device)
        self.region = self.buffer[GUARD: GUARD + nbytes]

    def intact(self) -> bool:
        head, tail = self.buffer[:GUARD], self.buffer[GUARD + self.nbytes:]
        return bool((head == SENTINEL).all().item()) and bool((tail == SENTINEL).all().item())


def _run_guarded(palib, dev, partition, what):
    import torch

    q = dev["query"]
    batch, query_heads, head_dim = (int(s) for s in q.shape)
    _, block_size, kv_heads, _ = (int(s) for s in dev["key_cache"].shape)
    max_blocks = int(dev["block_tables"].shape[1])
    need = palib.workspace_bytes(batch, query_heads, head_dim, block_size, max_blocks, partition)
    assert need > 0, "the case must split its sequences into several partitions"
    words = palib.counter_words(batch, query_heads, kv_heads)
    args = (dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"], dev["context_lengths"])

    out = Guarded(torch, q.numel() * q.element_size(), q.device)
    ws = Guarded(torch, need, q.device)
    counters = Guarded(torch, 4 * words, q.device)
    counters.region.zero_()
    out_view = out.region.view(q.dtype).view(q.shape)
    counter_view = counters.region.view(torch.int32)

    announce(f"guard bands {what}: partition launch")
    palib.decode(*args, partition_tokens=partition, out=out_view, workspace=ws.region, phase="partitions")
    torch.cuda.synchronize()
    assert out.intact() and ws.intact() and counters.intact(), f"{what}: partition launch wrote outside its buffers"

    announce(f"guard bands {what}: reduce launch")
    palib.decode(*args, partition_tokens=partition, out=out_view, workspace=ws.region, phase="reduce")
    torch.cuda.synchronize()
    assert out.intact() and ws.intact() and counters.intact(), f"{what}: reduce launch wrote outside its buffers"
    two_launch = out_view.clone()

    # Fused form into a fresh sentinel-filled output (every element must be written again).
    out.region.fill_(SENTINEL)
    announce(f"guard bands {what}: fused launch")
    palib.decode(*args, partition_tokens=partition, out=out_view, workspace=ws.region, phase="fused",
                 counters=counter_view)
    torch.cuda.synchronize()
    assert out.intact() and ws.intact() and counters.intact(), f"{what}: fused launch wrote outside its buffers"
    assert int(counter_view.abs().sum().item()) == 0, f"{what}: arrival counters not left zero"
    assert torch.equal(out_view.view(torch.int16), two_launch.view(torch.int16)), f"{what}: fused != two-launch"
    return two_launch


@pytest.mark.parametrize("key, partition", [("c2", 64), ("c3", 128), ("c4", 64)])
def test_guard_bands_small_workloads(gpu, palib, key, partition):
    from benchmarks.workloads import make_inputs

    data = make_inputs(key)
    out = _run_guarded(palib, to_device(data, gpu), partition, key)
    assert_within(out, oracle64(data), data["workload"].dtype, f"guarded {key}")


def test_guard_bands_ragged_b128(gpu, palib, c5_case):
    out = _run_guarded(palib, c5_case["gpu"], 2048, "c5")
    assert_within(out, c5_case["expected"], "bf16", "guarded c5, all 128 rows")
