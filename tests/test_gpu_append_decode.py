"""Append-and-decode (rk_pa_decode_append): one launch that stores each sequence's new token into the
paged caches and decodes the updated context.

The bar is bit-identity with the two operators it replaces: kv_cache_append of the same rows at each
sequence's position context_length - 1, then the decode, on the same inputs.  Outputs are compared
as raw bits (NaN rows of empty contexts included) and the caches with torch.equal; the decode
itself is pinned against the oracle by the other parity tests.
"""

from __future__ import annotations

import importlib.util

import pytest

from _helpers import announce, make_case, to_device

pytestmark = pytest.mark.gpu

# The dispatch entries' partition sizes (b128: 8192 tokens, slices of 512 table entries).
WORKLOAD_PARTITIONS = {"c1": 128, "c2": 256, "c3": 512, "c4": 128, "c5": 8192}


def new_token_slots(torch, block_tables, context_lengths, block_size):
    """Slot of position context_length - 1, or -1 (nothing appended) for an empty context and for a
    context past the table's max_blocks * block_size tokens."""

    limit = block_tables.shape[1] * block_size
    pos = context_lengths.long() - 1
    inside = (pos >= 0) & (pos < limit)
    safe = pos.clamp(min=0, max=limit - 1)
    block = block_tables.long().gather(1, (safe // block_size).unsqueeze(1)).squeeze(1)
    return torch.where(inside, block * block_size + safe % block_size, torch.full_like(pos, -1))


def new_rows(torch, query, kv_heads, seed):
    gen = torch.Generator(device=query.device).manual_seed(seed)
    shape = (query.shape[0], kv_heads, query.shape[2])
    return (torch.randn(shape, generator=gen, device=query.device).to(query.dtype),
            torch.randn(shape, generator=gen, device=query.device).to(query.dtype))


def same_bits(a, b) -> bool:
    import torch

    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def check_against_two_operators(palib, kvlib, dev, partition, phase, seed=5, variant="mfma"):
    import torch

    q, kc, vc, bt, cl = (dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths"))
    nk, nv = new_rows(torch, q, kc.shape[2], seed)
    slots = new_token_slots(torch, bt, cl, kc.shape[1])
    ref_k, ref_v = kc.clone(), vc.clone()
    kvlib.append(nk, nv, ref_k, ref_v, slots)
    expected = palib.decode(q, ref_k, ref_v, bt, cl, partition_tokens=partition, phase=phase, variant=variant)
    got_k, got_v = kc.clone(), vc.clone()
    got = palib.decode(q, got_k, got_v, bt, cl, partition_tokens=partition, phase=phase, variant=variant,
                       new_key=nk, new_value=nv)
    torch.cuda.synchronize()
    assert same_bits(got, expected)
    assert torch.equal(got_k, ref_k) and torch.equal(got_v, ref_v)
    return got


@pytest.mark.parametrize("phase", ["all", "fused"])
@pytest.mark.parametrize("key", ["c1", "c2", "c3", "c4"])
def test_measured_workloads(gpu, palib, kvlib, key, phase):
    from benchmarks.workloads import make_inputs

    dev = make_inputs(key, device=gpu)
    announce(f"append-decode {key} P={WORKLOAD_PARTITIONS[key]} {phase}")
    check_against_two_operators(palib, kvlib, dev, WORKLOAD_PARTITIONS[key], phase)


@pytest.mark.parametrize("phase", ["all", "fused"])
def test_ragged_b128_workload(gpu, palib, kvlib, phase):
    import torch

    from benchmarks.workloads import make_inputs

    announce(f"append-decode c5 ragged b128 {phase}")
    dev = make_inputs("c5", device=gpu)
    check_against_two_operators(palib, kvlib, dev, WORKLOAD_PARTITIONS["c5"], phase)
    del dev
    torch.cuda.empty_cache()


SHAPES = [
    # (Hq, Hkv, D, BS, dtype)
    (8, 8, 64, 16, "fp16"),
    (16, 8, 64, 32, "bf16"),
    (12, 4, 128, 16, "bf16"),   # group 3: one padded head slot
    (64, 8, 128, 16, "fp16"),   # group 8: one 8-head chunk, which stores
    (128, 8, 64, 16, "bf16"),   # group 16: two 8-head chunks, the first one stores
    (32, 8, 256, 16, "bf16"),
    (64, 8, 256, 16, "fp16"),   # group 8 at head_dim 256: one 8-head chunk (PV on MFMA)
    (4, 4, 256, 8, "fp16"),     # blocks smaller than a tile
    (8, 2, 128, 1, "fp16"),     # one token per block
    (32, 1, 128, 16, "bf16"),   # multi-query: four 8-head chunks, the first one stores
    (8, 2, 128, 256, "fp16"),   # the largest block the C ABI takes
]


@pytest.mark.parametrize("phase", ["all", "fused"])
@pytest.mark.parametrize("partition", [16, 64, 1024])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_shape_sweep(gpu, palib, kvlib, shape, partition, phase):
    import torch

    hq, hkv, d, bs, dtype = shape
    if partition // bs > 512:
        pytest.skip("partition_tokens / block_size must be <= 512")
    # Empty context (nothing appended, NaN row), one token, block and partition boundaries, ragged.
    contexts = [0, 1, bs, bs + 1, 16, 65, 300, 1024 + 7]
    case = make_case(torch, batch=len(contexts), query_heads=hq, kv_heads=hkv, head_dim=d, block_size=bs,
                     contexts=contexts, dtype=dtype, seed=hq * 31 + d + bs)
    announce(f"append-decode shape {shape} P={partition} {phase}")
    got = check_against_two_operators(palib, kvlib, to_device(case, gpu), partition, phase, seed=hq + d)
    assert torch.isnan(got[0].float()).all() and torch.isfinite(got[1:].float()).all()


@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_invalid_new_token_block_is_skipped_and_masked(gpu, palib, kvlib, index_dtype):
    """A new token whose block id is out of range is neither stored nor attended, as the append and
    the decode each treat it."""

    import torch

    contexts = [40, 90, 33]
    case = make_case(torch, batch=3, query_heads=8, kv_heads=2, head_dim=128, block_size=16, contexts=contexts,
                     dtype="bf16", index_dtype=index_dtype, seed=3)
    num_blocks = case["key_cache"].shape[0]
    case["block_tables"][1, (90 - 1) // 16] = num_blocks + 5
    announce(f"append-decode invalid new-token block {index_dtype}")
    check_against_two_operators(palib, kvlib, to_device(case, gpu), 64, "all")


@pytest.mark.parametrize("phase", ["all", "fused"])
def test_context_past_the_table_appends_nothing(gpu, palib, kvlib, phase):
    """A context length above max_blocks * block_size puts the new token outside the table: the call
    stores nothing for that sequence (its table's tokens, the last one included, stay as they were)
    and attends over the table's tokens, as the decode alone does."""

    import torch

    case = make_case(torch, batch=3, query_heads=16, kv_heads=4, head_dim=64, block_size=16, contexts=[40, 200, 64],
                     max_blocks=4, dtype="fp16", seed=21)
    announce(f"append-decode context past the table {phase}")
    check_against_two_operators(palib, kvlib, to_device(case, gpu), 32, phase)


def test_valu_variant_is_refused(gpu, palib):
    import torch

    from radeon_kernels.cabi import RK_ERR_UNSUPPORTED, CabiError

    case = to_device(make_case(torch, batch=2, query_heads=8, kv_heads=2, head_dim=64, block_size=16,
                               contexts=[20, 50], dtype="fp16", seed=9), gpu)
    nk, nv = new_rows(torch, case["query"], 2, 1)
    announce("append-decode refuses the valu variant")
    with pytest.raises(CabiError) as info:
        palib.decode(case["query"], case["key_cache"], case["value_cache"], case["block_tables"],
                     case["context_lengths"], partition_tokens=64, variant="valu", new_key=nk, new_value=nv)
    assert info.value.status == RK_ERR_UNSUPPORTED


@pytest.mark.parametrize("merge", ["reduce", "fused"])
def test_torch_binding_matches_append_then_decode(gpu, merge):
    """decode_append_mfma of the pack binding against kv_cache_append then decode_mfma."""

    import torch

    import radeon_kernels as rk
    from radeon_kernels.cabi import LIBRARY_PATH
    from benchmarks.workloads import make_inputs

    path = LIBRARY_PATH.parent / "rk_pa_gfx950.so"
    spec = importlib.util.spec_from_file_location("rk_pa_gfx950", path)
    binding = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(binding)
    dev = make_inputs("c2", device=gpu)
    q, kc, vc, bt, cl = (dev[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths"))
    nk, nv = new_rows(torch, q, kc.shape[2], 11)
    slots = new_token_slots(torch, bt, cl, kc.shape[1])
    scale = 128 ** -0.5
    announce(f"append-decode torch binding merge={merge}")
    ref_k, ref_v = kc.clone(), vc.clone()
    rk.kv_cache_append(nk, nv, ref_k, ref_v, slots)
    expected = binding.decode_mfma(q, ref_k, ref_v, bt, cl, scale, partition_tokens=256, merge=merge)
    got_k, got_v = kc.clone(), vc.clone()
    got = binding.decode_append_mfma(q, nk, nv, got_k, got_v, bt, cl, scale, partition_tokens=256, merge=merge)
    torch.cuda.synchronize()
    assert same_bits(got, expected)
    assert torch.equal(got_k, ref_k) and torch.equal(got_v, ref_v)
