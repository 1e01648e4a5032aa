"""Pinning the KV-cache oracles (oracle/kv_oracle.py) before trusting them as the checkers.

What pins the reference algorithm (src/radeon_kernels/ops/kv_cache/reference.py:6-20):

* torch's ``index_copy_`` (a library routine, not a restatement) on the flattened slot view gives
  bit-identical caches for every case of the reference's workload file, both dtypes, both index
  types;
* the element-by-element brute force with explicit ``block = slot // BS, offset = slot % BS``
  addressing agrees on small shapes;
* invariants: slots not named by ``slot_mapping`` keep their bytes; gathering the named slots
  returns the input rows; the token order of (key, value, slot) triples does not matter.

The block copy (reference.py:23-38) is pinned the same way: torch's ``index_select`` +
``index_copy_`` snapshot on every case of kv_cache_copy-1.0.yaml, untouched blocks, skipped
out-of-range pairs and a chained mapping that only a snapshot gets right.

The product's own torch fallbacks (``radeon_kernels.ops.kv_cache.reference``) are checked against
the oracle too, and planted mistakes in copies of the oracle each fail one of the checks above.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle
from radeon_kernels.ops.kv_cache.reference import kv_cache_append_reference
from benchmarks.workloads import APPEND_CASES, make_append_inputs


def bits(t):
    return kv_oracle.as_bits(t)


def np_args(data):
    return (bits(data["key"]), bits(data["value"]), bits(data["key_cache"]), bits(data["value_cache"]),
            data["slot_mapping"].numpy())


def torch_index_copy(data):
    """The library routine: index_copy_ on the [slots, Hkv, D] view of cloned caches."""

    kc, vc = data["key_cache"].clone(), data["value_cache"].clone()
    rows = (-1, kc.shape[2], kc.shape[3])
    slots = data["slot_mapping"].to(torch.int64)
    kc.view(rows).index_copy_(0, slots, data["key"])
    vc.view(rows).index_copy_(0, slots, data["value"])
    return bits(kc), bits(vc)


@pytest.mark.parametrize("case", sorted(APPEND_CASES))
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_oracle_matches_torch_index_copy(case, dtype, index_dtype):
    data = make_append_inputs(case, dtype=dtype, index_dtype=index_dtype)
    k, v = kv_oracle.append_numpy(*np_args(data))
    k_ref, v_ref = torch_index_copy(data)
    assert np.array_equal(k, k_ref) and np.array_equal(v, v_ref)


def small(seed=3, tokens=5, num_blocks=6, block_size=4, kv_heads=2, head_dim=8, index_dtype="int64"):
    from benchmarks.workloads import AppendCase

    return make_append_inputs(AppendCase("small", tokens, num_blocks, block_size, kv_heads, head_dim),
                              dtype="fp16", index_dtype=index_dtype, seed=seed)


def test_oracle_matches_bruteforce():
    for seed in range(4):
        data = small(seed=seed)
        a = kv_oracle.append_numpy(*np_args(data))
        b = kv_oracle.append_bruteforce(*np_args(data))
        assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_untouched_slots_keep_their_bytes_and_written_slots_read_back():
    data = make_append_inputs("prefill-t128-mha32-d128-p32", dtype="bf16")
    k, v = kv_oracle.append_numpy(*np_args(data))
    case = data["case"]
    cap = case.num_blocks * case.block_size
    flat_k, flat_v = k.reshape(cap, case.kv_heads, case.head_dim), v.reshape(cap, case.kv_heads, case.head_dim)
    slots = data["slot_mapping"].numpy()
    assert np.array_equal(flat_k[slots], bits(data["key"])) and np.array_equal(flat_v[slots], bits(data["value"]))
    untouched = np.setdiff1d(np.arange(cap), slots)
    before_k = bits(data["key_cache"]).reshape(cap, case.kv_heads, case.head_dim)
    assert np.array_equal(flat_k[untouched], before_k[untouched])


def test_token_order_does_not_matter():
    data = small(seed=7, tokens=9)
    perm = torch.randperm(9, generator=torch.Generator().manual_seed(1))
    shuffled = dict(data, key=data["key"][perm], value=data["value"][perm], slot_mapping=data["slot_mapping"][perm])
    a = kv_oracle.append_numpy(*np_args(data))
    b = kv_oracle.append_numpy(*np_args(shuffled))
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_out_of_range_slots_are_skipped():
    data = small(seed=5, tokens=4)
    cap = 6 * 4
    data["slot_mapping"] = torch.tensor([3, -1, cap, 7], dtype=torch.int64)
    k, v = kv_oracle.append_numpy(*np_args(data))
    flat = k.reshape(cap, 2, 8)
    before = bits(data["key_cache"]).reshape(cap, 2, 8)
    assert np.array_equal(flat[3], bits(data["key"])[0]) and np.array_equal(flat[7], bits(data["key"])[3])
    others = [s for s in range(cap) if s not in (3, 7)]
    assert np.array_equal(flat[others], before[others])


@pytest.mark.parametrize("case", ["decode-t8-gqa8-d128-p16", "prefill-t128-mha32-d128-p32"])
def test_product_fallback_matches_oracle(case):
    data = make_append_inputs(case, dtype="fp16", index_dtype="int32")
    expected = kv_oracle.append_numpy(*np_args(data))
    kc, vc = data["key_cache"].clone(), data["value_cache"].clone()
    out = kv_cache_append_reference(torch, data["key"], data["value"], kc, vc, data["slot_mapping"])
    assert out[0] is kc and out[1] is vc
    assert np.array_equal(bits(kc), expected[0]) and np.array_equal(bits(vc), expected[1])


# --------------------------------------------------------------------------------------------
def _mutant(kind):
    def append(key, value, key_cache, value_cache, slot_mapping):
        num_blocks, block_size, kv_heads, head_dim = key_cache.shape
        k_out, v_out = key_cache.copy(), value_cache.copy()
        for token, slot in enumerate(np.asarray(slot_mapping).tolist()):
            block, offset = divmod(int(slot), block_size)
            if kind == "block_offset_swapped":
                block, offset = offset % num_blocks, block % block_size
            if kind == "off_by_one":
                offset = (offset + 1) % block_size
            src_k = key[token].T.reshape(kv_heads, head_dim) if kind == "head_dim_transposed" else key[token]
            k_out[block, offset] = src_k
            v_out[block, offset] = key[token] if kind == "value_from_key" else value[token]
        return k_out, v_out

    return append


def _pinning_checks(append) -> list[str]:
    failures = []
    for case in ("decode-t8-gqa8-d128-p16", "prefill-t128-mha32-d128-p32"):
        data = make_append_inputs(case, dtype="bf16")
        got = append(*np_args(data))
        if not all(np.array_equal(x, y) for x, y in zip(got, torch_index_copy(data))):
            failures.append(f"index_copy {case}")
    return failures


@pytest.mark.parametrize("kind", ["block_offset_swapped", "off_by_one", "head_dim_transposed", "value_from_key"])
def test_planted_mistakes_are_caught(kind):
    assert _pinning_checks(_mutant(kind)), f"mutant {kind} passed every pinning check"


def test_unmutated_restatement_passes_the_same_checks():
    assert _pinning_checks(_mutant("none")) == []


# ---------------------------------------------------------------------------------------------
# Block copy (reference.py:23-38)
from radeon_kernels.ops.kv_cache.reference import kv_cache_copy_reference  # noqa: E402
from benchmarks.workloads import COPY_CASES, CopyCase, make_copy_inputs  # noqa: E402


def copy_args(data):
    return bits(data["key_cache"]), bits(data["value_cache"]), data["block_mapping"].numpy()


def torch_snapshot_copy(data):
    """Library routines: index_select the sources, then index_copy_ into the destinations."""

    kc, vc = data["key_cache"].clone(), data["value_cache"].clone()
    mapping = data["block_mapping"].to(torch.int64)
    k_src, v_src = kc.index_select(0, mapping[:, 0]), vc.index_select(0, mapping[:, 0])
    kc.index_copy_(0, mapping[:, 1], k_src)
    vc.index_copy_(0, mapping[:, 1], v_src)
    return bits(kc), bits(vc)


@pytest.mark.parametrize("case", sorted(COPY_CASES))
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_copy_oracle_matches_torch_snapshot_copy(case, dtype, index_dtype):
    data = make_copy_inputs(case, dtype=dtype, index_dtype=index_dtype)
    got = kv_oracle.copy_numpy(*copy_args(data))
    ref = torch_snapshot_copy(data)
    assert all(np.array_equal(x, y) for x, y in zip(got, ref))


def test_copy_invariants_and_out_of_range_pairs():
    data = make_copy_inputs(CopyCase("small", 3, 10, 4, 2, 8), dtype="fp16", seed=4)
    data["block_mapping"] = torch.tensor([[1, 7], [2, 10], [-1, 3], [4, 0]], dtype=torch.int64)
    k, v = kv_oracle.copy_numpy(*copy_args(data))
    before_k = bits(data["key_cache"])
    assert np.array_equal(k[7], before_k[1]) and np.array_equal(k[0], before_k[4])
    untouched = [b for b in range(10) if b not in (7, 0)]
    assert np.array_equal(k[untouched], before_k[untouched])
    # Chained mapping (outside the contract): snapshot semantics read pre-call sources.
    chain = dict(data, block_mapping=torch.tensor([[1, 2], [2, 3]], dtype=torch.int64))
    k2, _ = kv_oracle.copy_numpy(*copy_args(chain))
    assert np.array_equal(k2[3], before_k[2]) and np.array_equal(k2[2], before_k[1])
    assert all(np.array_equal(x, y) for x, y in zip(kv_oracle.copy_numpy(*copy_args(chain)), torch_snapshot_copy(chain)))


def test_product_copy_fallback_matches_oracle():
    data = make_copy_inputs("beam-pairs32-mha32-d128-p32", dtype="bf16", index_dtype="int32")
    expected = kv_oracle.copy_numpy(*copy_args(data))
    kc, vc = data["key_cache"].clone(), data["value_cache"].clone()
    out = kv_cache_copy_reference(torch, kc, vc, data["block_mapping"])
    assert out[0] is kc and out[1] is vc
    assert np.array_equal(bits(kc), expected[0]) and np.array_equal(bits(vc), expected[1])


def _copy_mutant(kind):
    def copy(key_cache, value_cache, block_mapping):
        k_out, v_out = key_cache.copy(), value_cache.copy()
        for s, d in np.asarray(block_mapping).tolist():
            if kind == "direction_swapped":
                s, d = d, s
            k_out[d] = key_cache[s]
            v_out[d] = key_cache[s] if kind == "value_from_key" else value_cache[s]
            if kind == "first_slot_only":
                k_out[d, 1:] = key_cache[d, 1:]
        return k_out, v_out

    return copy


@pytest.mark.parametrize("kind", ["direction_swapped", "value_from_key", "first_slot_only"])
def test_copy_planted_mistakes_are_caught(kind):
    data = make_copy_inputs("beam-pairs8-gqa8-d128-p16", dtype="bf16")
    got = _copy_mutant(kind)(*copy_args(data))
    assert not all(np.array_equal(x, y) for x, y in zip(got, torch_snapshot_copy(data)))
    clean = _copy_mutant("none")(*copy_args(data))
    assert all(np.array_equal(x, y) for x, y in zip(clean, torch_snapshot_copy(data)))
