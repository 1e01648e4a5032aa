"""GPU parity against the committed fixtures in tests/golden/tiny_cases.npz.

The inputs are the fixtures' own 16-bit patterns, so the kernels see exactly the tensors the float64
expected outputs were computed from (oracle/pa_oracle.py's token-by-token brute force, pinned by
tests/test_oracle.py).  The cases include the reference's fallback-acceptance shape
(developer/promotion/verify_paged_attention_fallback.py:42-47: B=2, 8/2 heads, D=64, block 16,
tables [[3,1,6,0],[7,2,5,4]], contexts [57,41]) in both dtypes, the context boundaries 1, block_size
and block_size + 1, a block size below the 16-token tile and head_dim 256.

Each case runs through the torch binding in both merge forms (fused: one launch whose last
workgroup per row merges; reduce: partition kernel plus merge kernel) and through the C ABI, for
every kernel variant, at partition sizes that split every sequence and at one that does not.
Bars: max abs error against the float64 outputs <= 2e-3 (fp16), <= 1.6e-2 (bf16).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from _helpers import TOLERANCE, announce, assert_within

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "tiny_cases.npz"


def _cases() -> list[str]:
    with np.load(GOLDEN) as z:
        return sorted({name.split("/", 1)[0] for name in z.files})


def _load(name: str) -> dict:
    with np.load(GOLDEN) as z:
        return {key.split("/", 1)[1]: z[key] for key in z.files if key.startswith(name + "/")}


def _device_inputs(torch, fixture: dict, device) -> tuple:
    dt = torch.float16 if str(fixture["dtype"]) == "fp16" else torch.bfloat16

    def bits(name):
        return torch.from_numpy(fixture[name].astype(np.int16)).view(dt).to(device)

    return (bits("query"), bits("key_cache"), bits("value_cache"),
            torch.from_numpy(fixture["block_tables"]).to(device),
            torch.from_numpy(fixture["context_lengths"]).to(device))


def _binding():
    import importlib.util

    from radeon_kernels.cabi import LIBRARY_PATH

    spec = importlib.util.spec_from_file_location("rk_pa_gfx950", LIBRARY_PATH.parent / "rk_pa_gfx950.so")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_fixture_set_is_the_committed_one():
    """The reference's acceptance tables are among the fixtures this module runs."""

    fixture = _load("acceptance_fp16")
    assert fixture["block_tables"].tolist() == [[3, 1, 6, 0], [7, 2, 5, 4]]
    assert fixture["context_lengths"].tolist() == [57, 41]
    assert set(_cases()) >= {"acceptance_fp16", "acceptance_bf16", "boundaries_bf16"}


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk", "valu"])
@pytest.mark.parametrize("name", _cases())
def test_binding_both_merge_forms_match_golden(gpu, name, variant):
    import torch

    fixture = _load(name)
    dtype = str(fixture["dtype"])
    q, k, v, bt, cl = _device_inputs(torch, fixture, gpu)
    expected = fixture["expected_f64"]
    block_size = k.shape[1]
    table_tokens = bt.shape[1] * block_size
    decode = getattr(_binding(), f"decode_{variant}")
    scale = 1.0 / float(np.sqrt(q.shape[-1]))
    outs = {}
    # 16-token partitions split every sequence (records and a merge); one partition covering the
    # whole table needs no merge at all.
    for partition in sorted({16, max(16, -(-table_tokens // 16) * 16)}):
        if partition // block_size > 512:
            continue
        for merge in ("fused", "reduce"):
            announce(f"golden {name} variant={variant} partition={partition} merge={merge}")
            out = decode(q, k, v, bt, cl, scale, partition_tokens=partition, merge=merge)
            torch.cuda.synchronize()
            assert_within(out.cpu(), expected, dtype, f"{name}/{variant}/P{partition}/{merge}")
            outs[partition, merge] = out
    for partition in {p for p, _ in outs}:
        assert torch.equal(outs[partition, "fused"].view(torch.int16), outs[partition, "reduce"].view(torch.int16))


@pytest.mark.parametrize("variant", ["mfma", "mfma_qk"])
@pytest.mark.parametrize("name", _cases())
def test_cabi_matches_golden(gpu, palib, name, variant):
    import torch

    fixture = _load(name)
    dtype = str(fixture["dtype"])
    q, k, v, bt, cl = _device_inputs(torch, fixture, gpu)
    announce(f"golden {name} through the C ABI variant={variant}")
    out = palib.decode(q, k, v, bt, cl, partition_tokens=32, variant=variant)
    torch.cuda.synchronize()
    err = assert_within(out.cpu(), fixture["expected_f64"], dtype, f"{name}/{variant} C ABI")
    assert err <= TOLERANCE[dtype]
