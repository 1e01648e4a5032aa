"""CPU oracle for paged-attention decode -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
this module, and only as the checker (or the timed CPU baseline).  The product path
(``radeon_kernels``) never imports it.

Three independent restatements of the reference algorithm
(src/radeon_kernels/ops/paged_attention/reference.py:7-47; semantics in
contracts/paged_attention_decode-1.0.json:15-25):

``fallback_restated``  torch on the CPU, the reference's own sequence of torch operations
                       (reference.py:17-47), plus two options the reference lacks: ``batch_chunk``
                       (evaluate a few sequences at a time so the 128-sequence x 16384-position
                       workload fits in host memory -- unchunked it expands ~112 GB of fp32) and
                       ``out_dtype=torch.float32`` (the fp32 result before the final cast, which is
                       what the tolerances are measured against).
``decode_numpy``       numpy, gathering only the valid tokens of each sequence, any float dtype.
``decode_bruteforce``  pure-Python float64 loops, token by token (tiny shapes only).

Edge semantics (all three): context lengths are clamped to ``max_blocks * block_size`` (the
reference builds exactly that many positions, reference.py:19); a context length <= 0 gives NaN
(softmax over an all ``-inf`` row, reference.py:43-45).  ``fallback_restated`` additionally shares
the reference's treatment of padding slots: their V rows are multiplied by probability 0, so
non-finite values stored there leak into the result (``0 * inf = nan``); the other two never read
slots past the context.

Pinning of each function (what the tests check it against) is listed in the test module
``tests/test_oracle.py``.
"""

from __future__ import annotations

import math
from typing import Any, Sequence

import numpy as np


# --------------------------------------------------------------------------------------------
# torch-CPU restatement of the reference fallback.
def fallback_restated(
    torch: Any,
    query: Any,
    key_cache: Any,
    value_cache: Any,
    block_tables: Any,
    context_lengths: Any,
    scale: float | None = None,
    *,
    out_dtype: Any | None = None,
    batch_chunk: int | None = None,
) -> Any:
    """reference.py:7-47 on whatever device the tensors are on, optionally batch-chunked."""

    batch = int(query.shape[0])
    step = batch if not batch_chunk else max(1, int(batch_chunk))
    if step >= batch:
        return _fallback_block(torch, query, key_cache, value_cache, block_tables, context_lengths, scale, out_dtype)
    parts = [
        _fallback_block(
            torch,
            query[start : start + step],
            key_cache,
            value_cache,
            block_tables[start : start + step],
            context_lengths[start : start + step],
            scale,
            out_dtype,
        )
        for start in range(0, batch, step)
    ]
    return torch.cat(parts, dim=0)


def _fallback_block(torch, query, key_cache, value_cache, block_tables, context_lengths, scale, out_dtype):
    batch, query_heads, head_dim = (int(s) for s in query.shape)
    block_size = int(key_cache.shape[1])
    kv_heads = int(key_cache.shape[2])
    max_context = int(block_tables.shape[1]) * block_size  # reference.py:19
    positions = torch.arange(max_context, device=query.device)  # :20
    blocks = block_tables.to(dtype=torch.int64).index_select(1, positions // block_size)  # :21-25
    slots = blocks * block_size + (positions % block_size).unsqueeze(0)  # :26-28
    flat = slots.reshape(-1)
    keys = key_cache.view(-1, kv_heads, head_dim).index_select(0, flat)  # :30-32
    values = value_cache.view(-1, kv_heads, head_dim).index_select(0, flat)  # :33
    keys = keys.view(batch, max_context, kv_heads, head_dim)  # :34
    values = values.view(batch, max_context, kv_heads, head_dim)
    heads = torch.arange(query_heads, device=query.device) // (query_heads // kv_heads)  # :36-37
    keys = keys.index_select(2, heads).float()  # :38
    values = values.index_select(2, heads).float()  # :39
    factor = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)  # :41
    scores = torch.einsum("bhd,bthd->bht", query.float(), keys) * factor  # :40-42
    valid = positions.unsqueeze(0) < context_lengths.to(dtype=torch.int64).unsqueeze(1)  # :43
    scores = scores.masked_fill(~valid.unsqueeze(1), float("-inf"))  # :44
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32)  # :45
    output = torch.einsum("bht,bthd->bhd", weights, values)  # :46
    return output.to(dtype=query.dtype if out_dtype is None else out_dtype)  # :47


# --------------------------------------------------------------------------------------------
# numpy restatement (valid tokens only).
def decode_numpy(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_tables: np.ndarray,
    context_lengths: Sequence[int] | np.ndarray,
    scale: float | None = None,
    *,
    accum: Any = np.float64,
    sequences: Sequence[int] | None = None,
) -> np.ndarray:
    """Inputs are float arrays holding the (already fp16/bf16-quantised) values.

    Returns ``[len(sequences) or B, Hq, D]`` in ``accum`` precision.  ``sequences`` restricts the
    evaluation to a subset of batch rows (used to spot-check the 128-sequence workload).
    """

    batch, query_heads, head_dim = query.shape
    _, block_size, kv_heads, _ = key_cache.shape
    group = query_heads // kv_heads
    factor = accum(scale if scale is not None else 1.0 / math.sqrt(head_dim))
    cap = block_tables.shape[1] * block_size
    rows = list(range(batch)) if sequences is None else list(sequences)
    out = np.empty((len(rows), query_heads, head_dim), dtype=accum)
    for position, b in enumerate(rows):
        ctx = min(int(context_lengths[b]), cap)
        if ctx <= 0:
            out[position] = np.nan
            continue
        tokens = np.arange(ctx)
        phys = np.asarray(block_tables[b], dtype=np.int64)[tokens // block_size]
        offs = tokens % block_size
        k = key_cache[phys, offs].astype(accum)  # [ctx, Hkv, D]
        v = value_cache[phys, offs].astype(accum)
        q = query[b].astype(accum).reshape(kv_heads, group, head_dim)  # head h -> kv h // group
        # scores[k, g, t] = sum_d q[k, g, d] * k[t, k, d], as one matmul per KV head (BLAS-backed).
        scores = np.matmul(q, k.transpose(1, 2, 0)) * factor
        peak = scores.max(axis=-1, keepdims=True)
        weights = np.exp(scores - peak)
        weights /= weights.sum(axis=-1, keepdims=True)
        # out[k, g, d] = sum_t weights[k, g, t] * v[t, k, d]
        out[position] = np.matmul(weights, v.transpose(1, 0, 2)).reshape(query_heads, head_dim)
    return out


# --------------------------------------------------------------------------------------------
# float64 brute force, token by token.
def decode_bruteforce(query, key_cache, value_cache, block_tables, context_lengths, scale=None) -> list:
    """Nested Python loops in float64; returns nested lists ``[B][Hq][D]``."""

    batch, query_heads, head_dim = (len(query), len(query[0]), len(query[0][0]))
    block_size = len(key_cache[0])
    kv_heads = len(key_cache[0][0])
    cap = len(block_tables[0]) * block_size
    factor = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    result = []
    for b in range(batch):
        ctx = min(int(context_lengths[b]), cap)
        per_head = []
        for h in range(query_heads):
            kvh = h // (query_heads // kv_heads)
            scores = []
            rows = []
            for t in range(max(ctx, 0)):
                block = int(block_tables[b][t // block_size])
                slot = t % block_size
                key = key_cache[block][slot][kvh]
                dot = 0.0
                for d in range(head_dim):
                    dot += float(query[b][h][d]) * float(key[d])
                scores.append(dot * factor)
                rows.append(value_cache[block][slot][kvh])
            if not scores:
                per_head.append([math.nan] * head_dim)
                continue
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = sum(weights)
            per_head.append([sum(w * float(r[d]) for w, r in zip(weights, rows)) / total for d in range(head_dim)])
        result.append(per_head)
    return result


# --------------------------------------------------------------------------------------------
# Rounding to the 16-bit storage types (round to nearest, ties to even).
def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 value, returned as float32 (NaN stays NaN)."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16 << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32).copy()
    out[np.isnan(x)] = np.nan
    return out


def round_to_fp16(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # values past 65504 round to inf, as the cast defines
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    return round_to_bf16(x) if dtype == "bf16" else round_to_fp16(x)


def as_numpy_f32(tensor: Any) -> np.ndarray:
    """Exact float32 copy of a (CPU or GPU) fp16/bf16/fp32 torch tensor."""

    return tensor.detach().float().cpu().numpy()
