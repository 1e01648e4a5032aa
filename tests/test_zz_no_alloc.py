"""Allocation-free decode (rk_pa_decode_noalloc) against rk_pa_decode, through the C ABI.

rk_pa_decode_noalloc runs the same two launches as rk_pa_decode with the split-K records in the
library's per-GPU scratch array, so its output must equal rk_pa_decode's bit for bit.  Two calls in
a row, the second with a smaller input, check that the array's leftover contents from the first
call do not leak into the second.  Outputs are carved out of sentinel-filled buffers so a write
outside them would show.
"""

from __future__ import annotations

import pytest

from _helpers import announce, assert_within, make_case, oracle64, to_device
from radeon_kernels import cabi

pytestmark = pytest.mark.gpu

SENTINEL = 0x7E5A  # an fp16/bf16 bit pattern no decode of these inputs produces


def _guarded_output(torch, like, guard=4096):
    """``(buffer, out)``: ``out`` has ``like``'s shape and dtype, inside ``guard`` sentinels per side."""

    n = like.numel()
    buffer = torch.full((n + 2 * guard,), SENTINEL, dtype=torch.int16, device=like.device)
    out = buffer[guard: guard + n].view(like.dtype).view(like.shape)
    return buffer, out


def _guards_intact(torch, buffer, n, guard=4096):
    return bool((buffer[:guard] == SENTINEL).all().item()) and bool((buffer[guard + n:] == SENTINEL).all().item())


def _compare(palib, dev, partition, variant="mfma"):
    import torch

    args = (dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"], dev["context_lengths"])
    expected = palib.decode(*args, partition_tokens=partition, variant=variant)
    buffer, out = _guarded_output(torch, dev["query"])
    palib.decode_noalloc(*args, out=out, partition_tokens=partition, variant=variant)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), "noalloc output differs from rk_pa_decode"
    assert _guards_intact(torch, buffer, out.numel()), "noalloc wrote outside its output"
    return out


def test_noalloc_matches_decode_on_two_calls_large_then_small(gpu, palib, c5_case):
    import torch

    announce("noalloc c5 ragged b128 (P 2048, 17 MB of records), then a 3-sequence case (P 64)")
    need = palib.workspace_bytes(128, 32, 128, 16, 1024, 2048)
    assert 0 < need <= cabi.RK_PA_NOALLOC_SCRATCH_BYTES
    out = _compare(palib, c5_case["gpu"], 2048)
    assert_within(out, c5_case["expected"], "bf16", "noalloc c5 vs float64 oracle")

    small = make_case(torch, batch=3, query_heads=8, kv_heads=2, head_dim=64, block_size=16,
                      contexts=[5, 700, 1500], dtype="fp16", seed=31)
    dev = to_device(small, gpu)
    out = _compare(palib, dev, 64)
    assert_within(out, oracle64(small), "fp16", "noalloc small case vs float64 oracle")


@pytest.mark.parametrize("variant", ["mfma", "valu"])
def test_noalloc_matches_decode_on_measured_workloads(gpu, palib, variant):
    from benchmarks.workloads import make_inputs

    for key, partition in (("c2", 64), ("c3", 128), ("c4", 64), ("c1", 128)):
        data = make_inputs(key)
        announce(f"noalloc {key} partition={partition} variant={variant}")
        out = _compare(palib, to_device(data, gpu), partition, variant)
        assert_within(out, oracle64(data), data["workload"].dtype, f"noalloc {key}")


def test_noalloc_allocates_nothing_after_setup(gpu, palib):
    """After the first call on the device (which looks up the scratch address), further calls change
    neither torch's allocator statistics nor the device's free memory."""

    import torch

    case = make_case(torch, batch=8, query_heads=32, kv_heads=8, head_dim=128, block_size=16,
                     contexts=[1024 + 97 * i for i in range(8)], dtype="bf16", seed=32)
    dev = to_device(case, gpu)
    args = (dev["query"], dev["key_cache"], dev["value_cache"], dev["block_tables"], dev["context_lengths"])
    outs = [torch.empty_like(dev["query"]) for _ in range(4)]
    announce("noalloc allocation check")
    palib.decode_noalloc(*args, out=outs[0], partition_tokens=64)
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    allocated_before = torch.cuda.memory_stats()["allocation.all.allocated"]
    for out in outs[1:]:
        palib.decode_noalloc(*args, out=out, partition_tokens=64)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free_before
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == allocated_before
    for out in outs[1:]:
        assert torch.equal(out.view(torch.int16), outs[0].view(torch.int16))
