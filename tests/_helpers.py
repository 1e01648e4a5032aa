"""Shared test helpers: case construction, oracle evaluation and tolerance checks."""

from __future__ import annotations

import math
import sys
from typing import Any

import numpy as np

from oracle import pa_oracle

# Max-abs-error bars against the fp32 (here: float64) result of the reference algorithm on the
# same quantised inputs.
TOLERANCE = {"fp16": 2e-3, "bf16": 1.6e-2}


def announce(message: str) -> None:
    """Name the case on stderr before a GPU step so a crash log says what was running."""

    sys.stderr.write(f"[case] {message}\n")
    sys.stderr.flush()


def torch_dtype(torch: Any, name: str) -> Any:
    return {"fp16": torch.float16, "bf16": torch.bfloat16}[name]


def make_case(
    torch: Any,
    *,
    batch: int,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    block_size: int,
    contexts: list[int],
    max_blocks: int | None = None,
    num_blocks: int | None = None,
    dtype: str = "bf16",
    index_dtype: str = "int32",
    seed: int = 0,
    kv_std: float = 1.0,
) -> dict[str, Any]:
    """CPU tensors for an arbitrary shape: disjoint random block tables, padding entries = 0."""

    gen = torch.Generator().manual_seed(seed)
    needed = [max(1, math.ceil(max(c, 1) / block_size)) for c in contexts]
    if max_blocks is None:
        max_blocks = max(needed)
    if num_blocks is None:
        num_blocks = sum(min(n, max_blocks) for n in needed) + 3
    perm = torch.randperm(num_blocks, generator=gen)
    tables = torch.zeros((batch, max_blocks), dtype=torch.int64)
    cursor = 0
    for b in range(batch):
        count = min(needed[b], max_blocks)
        ids = perm[cursor: cursor + count]
        if len(ids) < count:  # not enough distinct blocks: reuse (still valid ids)
            ids = torch.randint(0, num_blocks, (count,), generator=gen)
        tables[b, :count] = ids
        cursor += count
    dt = torch_dtype(torch, dtype)
    shape = (num_blocks, block_size, kv_heads, head_dim)
    query = torch.randn((batch, query_heads, head_dim), generator=gen).to(dt)
    key_cache = (torch.randn(shape, generator=gen) * kv_std).to(dt)
    value_cache = (torch.randn(shape, generator=gen) * kv_std).to(dt)
    index = {"int32": torch.int32, "int64": torch.int64}[index_dtype]
    return {
        "query": query,
        "key_cache": key_cache,
        "value_cache": value_cache,
        "block_tables": tables.to(index),
        "context_lengths": torch.tensor(contexts, dtype=index),
        "dtype": dtype,
    }


def to_device(case: dict[str, Any], device: Any) -> dict[str, Any]:
    return {k: (v.to(device) if hasattr(v, "to") and not isinstance(v, str) else v) for k, v in case.items()}


def oracle64(case: dict[str, Any], scale: float | None = None, sequences=None) -> np.ndarray:
    """float64 numpy oracle on the quantised inputs of ``case`` (CPU or GPU tensors)."""

    f = pa_oracle.as_numpy_f32
    return pa_oracle.decode_numpy(
        f(case["query"]), f(case["key_cache"]), f(case["value_cache"]),
        case["block_tables"].cpu().numpy(), case["context_lengths"].cpu().numpy(),
        scale, accum=np.float64, sequences=sequences,
    )


def oracle64_rows(case: dict[str, Any], scale: float | None = None, workers: int = 8) -> np.ndarray:
    """float64 oracle of every sequence of a large CPU-resident case, one sequence at a time.

    Each sequence's blocks are gathered first (``index_select`` of its table entries up to its
    context), so only the rows it attends to are converted to float; the sequences run on a thread
    pool (numpy's matrix products release the GIL).
    """

    import math as _math
    from concurrent.futures import ThreadPoolExecutor

    import torch

    query, key_cache, value_cache = case["query"], case["key_cache"], case["value_cache"]
    tables, contexts = case["block_tables"].cpu(), case["context_lengths"].cpu()
    block_size = int(key_cache.shape[1])
    cap = int(tables.shape[1]) * block_size
    f = pa_oracle.as_numpy_f32

    def one(b: int) -> np.ndarray:
        ctx = min(int(contexts[b]), cap)
        blocks = max(1, _math.ceil(max(ctx, 0) / block_size))
        ids = tables[b, :blocks].to(torch.int64)
        compact = np.arange(blocks, dtype=np.int64)[None]
        return pa_oracle.decode_numpy(f(query[b:b + 1]), f(key_cache.index_select(0, ids)),
                                      f(value_cache.index_select(0, ids)), compact, [ctx], scale,
                                      accum=np.float64)[0]

    with ThreadPoolExecutor(max_workers=workers) as pool:
        rows = list(pool.map(one, range(int(query.shape[0]))))
    return np.stack(rows)


def max_abs_error(actual: Any, expected: np.ndarray) -> float:
    got = pa_oracle.as_numpy_f32(actual).astype(np.float64)
    if got.shape != expected.shape:
        raise AssertionError(f"shape {got.shape} != {expected.shape}")
    both_nan = np.isnan(got) & np.isnan(expected)
    if np.any(np.isnan(got) != np.isnan(expected)):
        raise AssertionError("NaN pattern differs from the oracle")
    diff = np.abs(got - expected)
    diff[both_nan] = 0.0
    return float(diff.max()) if diff.size else 0.0


def assert_within(actual: Any, expected: np.ndarray, dtype: str, what: str = "") -> float:
    err = max_abs_error(actual, expected)
    bar = TOLERANCE[dtype]
    assert err <= bar, f"{what}: max abs error {err:.3e} > {bar:.1e} ({dtype})"
    return err
