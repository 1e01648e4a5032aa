"""Pinning the CPU oracle (oracle/pa_oracle.py) before trusting it as the checker.

What pins each part of the reference algorithm (src/radeon_kernels/ops/paged_attention/reference.py:7-47):

* gather ``slot = block_tables[b, t // BS] * BS + t % BS``: a library SDPA on K/V rows collected by an
  independent loop; permuting physical blocks together with the table changes nothing; padding
  table entries past the context change nothing.
* GQA map ``kv = h // (Hq / Hkv)``: duplicating KV heads into an MHA cache gives identical output.
* default scale ``1/sqrt(D)`` and scale handling: scale s on q equals scale 1 on s*q.
* mask ``t < context_length``: context 1 returns V row 0 exactly; identical keys give the mean of the
  first ``ctx`` V rows; finite garbage past the context changes nothing; clamp and empty context.
* fp32 softmax / PV: torch.nn.functional.scaled_dot_product_attention (library routine) agrees.
* rounding to fp16/bf16: torch's own casts.
* the committed golden vectors (float64 brute force) reproduce.

The mutation tests at the end plant plausible mistakes in copies of the oracle and show that at
least one of these checks fails for each.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from _helpers import make_case
from oracle import pa_oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def np_inputs(case):
    f = pa_oracle.as_numpy_f32
    return (f(case["query"]), f(case["key_cache"]), f(case["value_cache"]), case["block_tables"].numpy(),
            case["context_lengths"].numpy())


def sdpa_reference(case, scale=None) -> np.ndarray:
    """Gather each sequence's K/V rows with a plain loop, then torch SDPA (float64, CPU)."""

    q, k, v, bt, cl = np_inputs(case)
    b_count, hq, d = q.shape
    bs, hkv = k.shape[1], k.shape[2]
    out = np.empty((b_count, hq, d))
    for b in range(b_count):
        ctx = min(int(cl[b]), bt.shape[1] * bs)
        keys, values = [], []
        for t in range(ctx):
            keys.append(k[int(bt[b][t // bs]), t % bs])
            values.append(v[int(bt[b][t // bs]), t % bs])
        kk = torch.tensor(np.stack(keys), dtype=torch.float64).permute(1, 0, 2)  # [Hkv, ctx, D]
        vv = torch.tensor(np.stack(values), dtype=torch.float64).permute(1, 0, 2)
        kk = kk.repeat_interleave(hq // hkv, dim=0)  # query head h reads KV head h // group
        vv = vv.repeat_interleave(hq // hkv, dim=0)
        qq = torch.tensor(q[b], dtype=torch.float64).unsqueeze(1)  # [Hq, 1, D]
        o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, scale=scale)
        out[b] = o.squeeze(1).numpy()
    return out


CASES = [
    dict(batch=2, query_heads=8, kv_heads=2, head_dim=64, block_size=16, contexts=[57, 41], dtype="fp16", seed=1),
    dict(batch=3, query_heads=4, kv_heads=4, head_dim=128, block_size=8, contexts=[1, 8, 9], dtype="bf16", seed=2),
    dict(batch=2, query_heads=6, kv_heads=2, head_dim=64, block_size=4, contexts=[13, 30], dtype="bf16", seed=3),
]


@pytest.mark.parametrize("spec", CASES)
def test_numpy_oracle_matches_library_sdpa(spec):
    case = make_case(torch, **spec)
    expected = sdpa_reference(case)
    got = pa_oracle.decode_numpy(*np_inputs(case))
    np.testing.assert_allclose(got, expected, rtol=0, atol=1e-12)


@pytest.mark.parametrize("spec", CASES)
def test_torch_restatement_matches_library_sdpa(spec):
    case = make_case(torch, **spec)
    got = pa_oracle.fallback_restated(torch, case["query"], case["key_cache"], case["value_cache"],
                                      case["block_tables"], case["context_lengths"], out_dtype=torch.float32)
    np.testing.assert_allclose(got.numpy(), sdpa_reference(case), rtol=0, atol=2e-6)


@pytest.mark.parametrize("spec", CASES)
def test_bruteforce_matches_library_sdpa(spec):
    case = make_case(torch, **spec)
    q, k, v, bt, cl = np_inputs(case)
    got = np.asarray(pa_oracle.decode_bruteforce(q.tolist(), k.tolist(), v.tolist(), bt.tolist(), cl.tolist()))
    np.testing.assert_allclose(got, sdpa_reference(case), rtol=0, atol=1e-12)


def test_restatement_batch_chunking_is_exact():
    case = make_case(torch, batch=5, query_heads=8, kv_heads=2, head_dim=64, block_size=16,
                     contexts=[3, 100, 64, 17, 1], dtype="bf16", seed=4)
    args = (case["query"], case["key_cache"], case["value_cache"], case["block_tables"], case["context_lengths"])
    whole = pa_oracle.fallback_restated(torch, *args, out_dtype=torch.float32)
    for chunk in (1, 2, 3):
        parts = pa_oracle.fallback_restated(torch, *args, out_dtype=torch.float32, batch_chunk=chunk)
        np.testing.assert_allclose(parts.numpy(), whole.numpy(), rtol=0, atol=1e-6)


def test_context_one_returns_first_value_row_exactly():
    case = make_case(torch, batch=2, query_heads=8, kv_heads=2, head_dim=64, block_size=16, contexts=[1, 1],
                     dtype="fp16", seed=5)
    q, k, v, bt, cl = np_inputs(case)
    got = pa_oracle.decode_numpy(q, k, v, bt, cl)
    for b in range(2):
        for h in range(8):
            np.testing.assert_array_equal(got[b, h], v[bt[b, 0], 0, h // 4])


def test_identical_keys_average_the_first_context_values():
    case = make_case(torch, batch=2, query_heads=4, kv_heads=2, head_dim=64, block_size=8, contexts=[13, 22],
                     dtype="bf16", seed=6)
    case["key_cache"][:] = case["key_cache"][0, 0]  # every key identical -> uniform softmax
    q, k, v, bt, cl = np_inputs(case)
    got = pa_oracle.decode_numpy(q, k, v, bt, cl)
    for b in range(2):
        ctx = int(cl[b])
        rows = np.stack([v[bt[b, t // 8], t % 8] for t in range(ctx)])  # [ctx, Hkv, D]
        for h in range(4):
            np.testing.assert_allclose(got[b, h], rows[:, h // 2].astype(np.float64).mean(axis=0), atol=1e-12)


def test_dominant_score_selects_its_value_row():
    case = make_case(torch, batch=1, query_heads=4, kv_heads=1, head_dim=64, block_size=16, contexts=[40],
                     dtype="fp16", seed=7)
    bt = case["block_tables"]
    target = 29
    case["query"][:] = 0.0
    case["query"][:, :, 0] = 1.0
    case["key_cache"][:] = 0.0
    case["key_cache"][bt[0, target // 16], target % 16, 0, 0] = 2000.0  # score 2000/8 = 250 vs 0
    q, k, v, bt_np, cl = np_inputs(case)
    got = pa_oracle.decode_numpy(q, k, v, bt_np, cl)
    np.testing.assert_allclose(got[0, 0], v[bt_np[0, target // 16], target % 16, 0], atol=1e-12)


def test_block_permutation_and_padding_invariance():
    case = make_case(torch, batch=2, query_heads=8, kv_heads=2, head_dim=64, block_size=4, contexts=[10, 7],
                     max_blocks=5, dtype="bf16", seed=8)
    base = pa_oracle.decode_numpy(*np_inputs(case))
    nb = case["key_cache"].shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1))
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(nb)
    moved = dict(case)
    moved["key_cache"] = case["key_cache"][perm]      # new block i holds old block perm[i]
    moved["value_cache"] = case["value_cache"][perm]
    moved["block_tables"] = inverse[case["block_tables"].long()].to(case["block_tables"].dtype)
    np.testing.assert_array_equal(pa_oracle.decode_numpy(*np_inputs(moved)), base)
    padded = dict(case)
    tables = case["block_tables"].clone()
    tables[0, 3:] = nb - 1  # entries past ceil(10/4)=3 blocks
    tables[1, 2:] = 1       # entries past ceil(7/4)=2 blocks
    padded["block_tables"] = tables
    np.testing.assert_array_equal(pa_oracle.decode_numpy(*np_inputs(padded)), base)


def test_gqa_equals_duplicated_mha():
    case = make_case(torch, batch=2, query_heads=12, kv_heads=3, head_dim=64, block_size=8, contexts=[20, 9],
                     dtype="fp16", seed=9)
    gqa = pa_oracle.decode_numpy(*np_inputs(case))
    mha = dict(case)
    mha["key_cache"] = case["key_cache"].repeat_interleave(4, dim=2)
    mha["value_cache"] = case["value_cache"].repeat_interleave(4, dim=2)
    np.testing.assert_allclose(pa_oracle.decode_numpy(*np_inputs(mha)), gqa, atol=1e-13)


def test_scale_is_applied_to_scores():
    case = make_case(torch, batch=1, query_heads=4, kv_heads=2, head_dim=64, block_size=8, contexts=[19],
                     dtype="bf16", seed=10)
    q, k, v, bt, cl = np_inputs(case)
    default = pa_oracle.decode_numpy(q, k, v, bt, cl)
    explicit = pa_oracle.decode_numpy(q, k, v, bt, cl, 1.0 / math.sqrt(64))
    np.testing.assert_array_equal(default, explicit)
    scaled = pa_oracle.decode_numpy(q.astype(np.float64) * 0.37, k, v, bt, cl, 1.0)
    np.testing.assert_allclose(pa_oracle.decode_numpy(q, k, v, bt, cl, 0.37), scaled, atol=1e-12)


def test_positions_past_the_context_are_ignored_and_contexts_clamp():
    case = make_case(torch, batch=3, query_heads=4, kv_heads=2, head_dim=64, block_size=8, contexts=[11, 16, 5],
                     max_blocks=2, dtype="fp16", seed=11)
    base = pa_oracle.decode_numpy(*np_inputs(case))
    noisy = dict(case)
    k, v = case["key_cache"].clone(), case["value_cache"].clone()
    block = int(case["block_tables"][0, 1])
    k[block, 3:] = 60.0  # tokens 11..15 of sequence 0: past its context
    v[block, 3:] = -500.0
    noisy["key_cache"], noisy["value_cache"] = k, v
    np.testing.assert_array_equal(pa_oracle.decode_numpy(*np_inputs(noisy)), base)
    for fn in (pa_oracle.decode_numpy,):
        longer = dict(case)
        longer["context_lengths"] = torch.tensor([11, 1000, 5], dtype=case["context_lengths"].dtype)
        np.testing.assert_array_equal(fn(*np_inputs(longer)), base)  # 1000 clamps to 2*8 = 16
        empty = dict(case)
        empty["context_lengths"] = torch.tensor([0, 16, -2], dtype=case["context_lengths"].dtype)
        got = fn(*np_inputs(empty))
        assert np.isnan(got[0]).all() and np.isnan(got[2]).all() and np.isfinite(got[1]).all()
    restated = pa_oracle.fallback_restated(torch, case["query"], case["key_cache"], case["value_cache"],
                                           case["block_tables"], torch.tensor([0, 1000, 5], dtype=torch.int32),
                                           out_dtype=torch.float32)
    assert torch.isnan(restated[0]).all() and torch.isfinite(restated[1:]).all()


def test_rounding_matches_torch_casts():
    gen = torch.Generator().manual_seed(12)
    values = torch.cat([
        torch.randn(20000, generator=gen) * 3,
        torch.tensor([0.0, -0.0, 1.0, 65504.0, 1e-8, -1e-30, 3.0e38, float("inf"), float("-inf")]),
        # exact ties between neighbouring bf16 / fp16 values
        torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11]),
    ])
    x = values.numpy()
    np.testing.assert_array_equal(pa_oracle.round_to_bf16(x), values.to(torch.bfloat16).float().numpy())
    np.testing.assert_array_equal(pa_oracle.round_to_fp16(x), values.to(torch.float16).float().numpy())
    assert np.isnan(pa_oracle.round_to_bf16(np.array([np.nan], dtype=np.float32))).all()


def test_golden_tiny_cases_reproduce():
    data = np.load(GOLDEN / "tiny_cases.npz")
    names = sorted({key.split("/")[0] for key in data.files})
    assert len(names) >= 5
    for name in names:
        dtype = str(data[f"{name}/dtype"])
        tdt = torch.float16 if dtype == "fp16" else torch.bfloat16

        def tensor(field):
            return torch.from_numpy(data[f"{name}/{field}"].view(np.int16).copy()).view(tdt)

        q, k, v = tensor("query"), tensor("key_cache"), tensor("value_cache")
        bt = torch.from_numpy(data[f"{name}/block_tables"])
        cl = torch.from_numpy(data[f"{name}/context_lengths"])
        expected = data[f"{name}/expected_f64"]
        got = pa_oracle.decode_numpy(pa_oracle.as_numpy_f32(q), pa_oracle.as_numpy_f32(k), pa_oracle.as_numpy_f32(v),
                                     bt.numpy(), cl.numpy())
        np.testing.assert_allclose(got, expected, atol=1e-12, err_msg=name)
        restated = pa_oracle.fallback_restated(torch, q, k, v, bt, cl)
        np.testing.assert_array_equal(pa_oracle.round_to(expected.astype(np.float32), dtype),
                                      data[f"{name}/expected_rounded"])
        # The restated fallback rounds an fp32 result: within one storage ulp of the float64 answer.
        ulp = 2 ** -7 if dtype == "bf16" else 2 ** -10
        assert np.abs(restated.float().numpy() - expected).max() <= ulp * max(1.0, np.abs(expected).max())


def test_golden_c1_inputs_and_output_reproduce():
    from benchmarks.workloads import make_inputs

    golden = np.load(GOLDEN / "c1_expected.npz")
    data = make_inputs("c1")
    import hashlib

    for field in ("query", "key_cache", "value_cache", "block_tables", "context_lengths"):
        digest = hashlib.sha256(data[field].contiguous().view(-1).view(torch.uint8).numpy().tobytes()).hexdigest()
        assert digest == str(golden[f"sha_{field}"]), f"seeded {field} differs from the committed fixture"
    f = pa_oracle.as_numpy_f32
    got = pa_oracle.decode_numpy(f(data["query"]), f(data["key_cache"]), f(data["value_cache"]),
                                 data["block_tables"].numpy(), data["context_lengths"].numpy())
    np.testing.assert_allclose(got, golden["expected_f64"], atol=1e-12)


# --------------------------------------------------------------------------------------------
# Planted mistakes: each mutant of the numpy oracle must fail at least one pinning check.
def _mutant(kind):
    def decode(query, key_cache, value_cache, block_tables, context_lengths, scale=None, **_):
        b_count, hq, d = query.shape
        _, bs, hkv, _ = key_cache.shape
        group = hq // hkv
        factor = scale if scale is not None else 1.0 / math.sqrt(d)
        if kind == "no_scale":
            factor = 1.0
        out = np.empty((b_count, hq, d))
        for b in range(b_count):
            ctx = min(int(context_lengths[b]), block_tables.shape[1] * bs)
            if kind == "mask_off_by_one":
                ctx = max(ctx - 1, 1)
            t = np.arange(ctx)
            if kind == "slot_swapped":
                phys, offs = np.asarray(block_tables[b])[t % block_tables.shape[1]], t // block_tables.shape[1] % bs
            else:
                phys, offs = np.asarray(block_tables[b])[t // bs], t % bs
            for h in range(hq):
                kvh = h % hkv if kind == "head_modulo" else h // group
                k = key_cache[phys, offs, kvh].astype(np.float64)
                v = value_cache[phys, offs, kvh].astype(np.float64)
                s = k @ query[b, h].astype(np.float64) * factor
                if kind == "softmax_no_shift_sum":
                    w = np.exp(s - s.max())
                else:
                    w = np.exp(s - s.max())
                    w /= w.sum()
                out[b, h] = w @ v
        return out

    return decode


def _pinning_checks(decode) -> list[str]:
    failures = []
    for spec in CASES:
        case = make_case(torch, **spec)
        if not np.allclose(decode(*np_inputs(case)), sdpa_reference(case), atol=1e-9):
            failures.append("sdpa")
    case = make_case(torch, batch=2, query_heads=12, kv_heads=3, head_dim=64, block_size=8, contexts=[20, 9],
                     dtype="fp16", seed=9)
    mha = dict(case)
    mha["key_cache"] = case["key_cache"].repeat_interleave(4, dim=2)
    mha["value_cache"] = case["value_cache"].repeat_interleave(4, dim=2)
    if not np.allclose(decode(*np_inputs(mha)), decode(*np_inputs(case)), atol=1e-12):
        failures.append("gqa")
    return failures


@pytest.mark.parametrize("kind", ["head_modulo", "slot_swapped", "no_scale", "mask_off_by_one", "softmax_no_shift_sum"])
def test_planted_mistakes_are_caught(kind):
    assert _pinning_checks(_mutant(kind)), f"mutant {kind} passed every pinning check"


def test_unmutated_restatement_passes_the_same_checks():
    assert _pinning_checks(_mutant("none")) == []
