"""Seeded paged-decode workloads: the five measured shapes, the reference's workload cases and a
generic builder.

Each workload fixes batch, heads, head_dim, block size, dtype, cache size and how block tables and
context lengths are drawn.  Inputs are drawn on the CPU, so a seed names one input set on every
machine, in a fixed order: context lengths, block permutation, query, keys, values.

* ``draw="serial"``: every tensor from one ``torch.Generator`` seeded with the workload seed.
* ``draw="chunked"`` (the 4.24 GB ragged workload): context lengths, permutation and query as above;
  each cache is drawn in fixed chunks of ``CHUNK_ELEMENTS`` values, chunk ``i`` of cache ``c``
  (0 = keys, 1 = values) from its own generator seeded ``chunk_seed(seed, c, i)``.  The chunks are
  independent, so they are drawn on a thread pool; the result does not depend on the number of
  threads.

``input_digests`` gives the SHA-256 of every input tensor's bytes, which ties a test's inputs to a
benchmark run's.

KV accounting (``kv_bytes``) counts the K and V rows a decode must read: for every sequence,
``min(context, max_blocks * block_size)`` tokens x kv_heads x head_dim x 2 tensors x element size.
Padding table entries and tokens past the context are not counted.
"""

from __future__ import annotations

import hashlib
import math
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field
from typing import Any

DEFAULT_SEED_BASE = 20261201
CHUNK_ELEMENTS = 1 << 24


@dataclass(frozen=True)
class Workload:
    key: str
    name: str
    batch: int
    query_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    dtype: str  # "fp16" | "bf16"
    max_blocks: int
    num_blocks: int | None  # None: sum of blocks the drawn contexts need (ragged workload)
    context: int | tuple[int, int]  # fixed length, or inclusive uniform range
    kv_std: float = 1.0
    seed: int = DEFAULT_SEED_BASE
    notes: str = ""
    # "normal": q ~ N(0, 1), K/V ~ N(0, kv_std^2).  "uniform": q, K, V ~ U(-0.125, 0.125), the
    # reference benchmark's draw (benchmarks/paged_attention/benchmark.py:74-77).
    distribution: str = "normal"
    draw: str = "serial"  # "serial" | "chunked" (see the module docstring)
    extra: dict[str, Any] = field(default_factory=dict)

    @property
    def ragged(self) -> bool:
        return isinstance(self.context, tuple)

    @property
    def elem_size(self) -> int:
        return 2


WORKLOADS: dict[str, Workload] = {
    "c1": Workload(
        key="c1", name="b1-gqa32x8-c128-d128-p16-fp16", batch=1, query_heads=32, kv_heads=8, head_dim=128,
        block_size=16, dtype="fp16", max_blocks=8, num_blocks=64, context=128, seed=DEFAULT_SEED_BASE + 0,
        notes="block table = first 8 entries of a seeded permutation of 0..63",
    ),
    "c2": Workload(
        key="c2", name="b8-gqa32x8-c1024-d128-p16-bf16", batch=8, query_heads=32, kv_heads=8, head_dim=128,
        block_size=16, dtype="bf16", max_blocks=64, num_blocks=1024, context=1024, seed=DEFAULT_SEED_BASE + 1,
        notes="64 block ids per sequence drawn without replacement from a seeded permutation of 0..1023",
    ),
    "c3": Workload(
        key="c3", name="b4-mha16-c2048-d64-p32-bf16", batch=4, query_heads=16, kv_heads=16, head_dim=64,
        block_size=32, dtype="bf16", max_blocks=64, num_blocks=512, context=2048, seed=DEFAULT_SEED_BASE + 2,
        notes="disjoint seeded block tables of 64 blocks each",
    ),
    "c4": Workload(
        key="c4", name="b4-gqa32x8-c1024-d256-p16-fp16", batch=4, query_heads=32, kv_heads=8, head_dim=256,
        block_size=16, dtype="fp16", max_blocks=64, num_blocks=512, context=1024, kv_std=0.5,
        seed=DEFAULT_SEED_BASE + 3, notes="K/V ~ N(0, 0.5^2) (0.5 read as the standard deviation)",
    ),
    "c5": Workload(
        key="c5", name="b128-gqa32x8-ragged1024to16384-d128-p16-bf16", batch=128, query_heads=32, kv_heads=8,
        head_dim=128, block_size=16, dtype="bf16", max_blocks=1024, num_blocks=None, context=(1024, 16384),
        seed=DEFAULT_SEED_BASE + 4, draw="chunked",
        notes="context ~ U[1024, 16384]; tables padded to 1024 with block 0; blocks assigned by seeded shuffle",
    ),
}

# The reference's paged-decode workload cases (benchmarks/workloads/paged_attention_decode-1.0.yaml:13-22),
# each in fp16 and bf16, drawn as the reference's benchmark draws them (benchmark.py:79-117): every
# sequence has the case's context length, num_blocks = batch * ceil(context / block_size), the tables
# are one permutation of all blocks, and q, K, V ~ U(-0.125, 0.125).  Seeds are the benchmark's three
# (benchmark.py:200), used with a CPU generator.
REFERENCE_CASES: tuple[tuple[str, int, int, int, int, int, int], ...] = (
    # id, batch, query_heads, kv_heads, context, head_dim, block_size
    ("b1-gqa32x8-c128-d128-p16", 1, 32, 8, 128, 128, 16),
    ("b1-gqa32x8-c1024-d128-p16", 1, 32, 8, 1024, 128, 16),
    ("b1-gqa32x8-c4096-d128-p16", 1, 32, 8, 4096, 128, 16),
    ("b8-gqa32x8-c128-d128-p16", 8, 32, 8, 128, 128, 16),
    ("b8-gqa32x8-c1024-d128-p16", 8, 32, 8, 1024, 128, 16),
    ("b16-gqa32x8-c2048-d128-p16", 16, 32, 8, 2048, 128, 16),
    ("b4-mha16-c2048-d64-p32", 4, 16, 16, 2048, 64, 32),
    ("b4-gqa32x8-c1024-d256-p16", 4, 32, 8, 1024, 256, 16),
)
REFERENCE_SEEDS = (20260918, 20260919, 20260920)


def _reference_workload(case: tuple[str, int, int, int, int, int, int], dtype: str) -> Workload:
    case_id, batch, hq, hkv, context, head_dim, block_size = case
    max_blocks = math.ceil(context / block_size)
    return Workload(
        key=f"{case_id}-{dtype}", name=f"{case_id}-{dtype}", batch=batch, query_heads=hq, kv_heads=hkv,
        head_dim=head_dim, block_size=block_size, dtype=dtype, max_blocks=max_blocks,
        num_blocks=batch * max_blocks, context=context, seed=REFERENCE_SEEDS[0], distribution="uniform",
        notes="reference workload case: one permutation of batch * max_blocks blocks, q/K/V ~ U(-0.125, 0.125)",
    )


for _case in REFERENCE_CASES:
    for _dtype in ("fp16", "bf16"):
        _w = _reference_workload(_case, _dtype)
        WORKLOADS[_w.key] = _w
REFERENCE_KEYS = tuple(f"{case[0]}-{dtype}" for case in REFERENCE_CASES for dtype in ("fp16", "bf16"))


# Shapes sampled from the broad gfx950 dispatch region (paged_attention_decode-gfx950-region), which takes
# every shape no exact entry names: head layouts from MHA to groups of 16 (8-head chunks), head_dim 64 / 128 /
# 256, blocks of 8 to 128 tokens (below the 16-token tile too), both dtypes, int32 and int64 indices, fixed
# and ragged contexts.  The last is the reference's fallback-acceptance shape
# (developer/promotion/verify_paged_attention_fallback.py:42-47: B=2, 8/2 heads, D=64, block 16), which
# selects this region on gfx950.  extra["index_dtype"] names the index type the sample is drawn with.
def _region_sample(name: str, batch: int, hq: int, hkv: int, head_dim: int, block_size: int, dtype: str,
                   context: int | tuple[int, int], index_dtype: str, seed: int) -> Workload:
    top = context if isinstance(context, int) else context[1]
    max_blocks = math.ceil(top / block_size)
    return Workload(
        key=f"region-{name}", name=f"region-{name}", batch=batch, query_heads=hq, kv_heads=hkv, head_dim=head_dim,
        block_size=block_size, dtype=dtype, max_blocks=max_blocks,
        num_blocks=None if isinstance(context, tuple) else batch * max_blocks, context=context, seed=seed,
        notes="broad-region sample", extra={"index_dtype": index_dtype})


REGION_SAMPLES: tuple[Workload, ...] = (
    _region_sample("b16-gqa64x8-ragged512to4096-d128-p16-bf16", 16, 64, 8, 128, 16, "bf16", (512, 4096), "int32", 20261301),
    _region_sample("b8-mha32-c2048-d128-p32-fp16", 8, 32, 32, 128, 32, "fp16", 2048, "int32", 20261302),
    _region_sample("b32-gqa16x8-ragged100to3000-d64-p8-bf16", 32, 16, 8, 64, 8, "bf16", (100, 3000), "int64", 20261303),
    _region_sample("b8-gqa16x4-ragged256to2048-d256-p16-fp16", 8, 16, 4, 256, 16, "fp16", (256, 2048), "int32", 20261304),
    _region_sample("b4-gqa128x8-c8192-d64-p64-bf16", 4, 128, 8, 64, 64, "bf16", 8192, "int32", 20261305),
    _region_sample("b4-gqa32x8-c4096-d128-p128-bf16", 4, 32, 8, 128, 128, "bf16", 4096, "int64", 20261306),
    _region_sample("b64-gqa32x8-ragged1to2048-d128-p16-fp16", 64, 32, 8, 128, 16, "fp16", (1, 2048), "int64", 20261307),
    _region_sample("b2-gqa8x2-ragged41to57-d64-p16-fp16", 2, 8, 2, 64, 16, "fp16", (41, 57), "int32", 20261308),
)
for _w in REGION_SAMPLES:
    WORKLOADS[_w.key] = _w


def torch_dtype(torch: Any, name: str) -> Any:
    return {"fp16": torch.float16, "bf16": torch.bfloat16}[name]


def chunk_seed(seed: int, cache: int, chunk: int) -> int:
    """Seed of chunk ``chunk`` of cache ``cache`` (0 keys, 1 values) in the chunked draw."""

    return (seed << 24) + (cache << 20) + chunk


def _chunked_normal(torch: Any, shape: tuple[int, ...], std: float, dtype: Any, seed: int, cache: int,
                    workers: int | None) -> Any:
    out = torch.empty(shape, dtype=dtype)
    flat = out.view(-1)
    total = flat.numel()

    def fill(chunk: int) -> None:
        start = chunk * CHUNK_ELEMENTS
        count = min(CHUNK_ELEMENTS, total - start)
        gen = torch.Generator().manual_seed(chunk_seed(seed, cache, chunk))
        values = torch.randn(count, generator=gen, dtype=torch.float32)
        if std != 1.0:
            values.mul_(std)
        flat[start:start + count].copy_(values)

    chunks = (total + CHUNK_ELEMENTS - 1) // CHUNK_ELEMENTS
    workers = workers or min(16, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(fill, range(chunks)))
    return out


def make_inputs(
    workload: Workload | str,
    *,
    seed: int | None = None,
    device: Any = "cpu",
    index_dtype: str = "int32",
    torch_module: Any | None = None,
    workers: int | None = None,
) -> dict[str, Any]:
    """Draw the workload's tensors on the CPU; returns query, key_cache, value_cache, block_tables,
    context_lengths (all on ``device``) plus ``num_blocks``, ``kv_bytes`` and ``contexts``."""

    if torch_module is None:
        import torch as torch_module
    torch = torch_module
    w = WORKLOADS[workload] if isinstance(workload, str) else workload
    seed = w.seed if seed is None else seed
    generator = torch.Generator().manual_seed(seed)
    index = {"int32": torch.int32, "int64": torch.int64}[index_dtype]
    dtype = torch_dtype(torch, w.dtype)

    if w.ragged:
        low, high = w.context
        contexts = torch.randint(low, high + 1, (w.batch,), generator=generator)
    else:
        contexts = torch.full((w.batch,), int(w.context), dtype=torch.int64)
    needed = [math.ceil(int(c) / w.block_size) for c in contexts]
    if w.num_blocks is None:
        num_blocks = int(sum(needed))
        permutation = torch.randperm(num_blocks, generator=generator)
        tables = torch.zeros((w.batch, w.max_blocks), dtype=torch.int64)
        cursor = 0
        for b, count in enumerate(needed):
            tables[b, :count] = permutation[cursor : cursor + count]
            cursor += count
    else:
        num_blocks = w.num_blocks
        permutation = torch.randperm(num_blocks, generator=generator)
        tables = permutation[: w.batch * w.max_blocks].view(w.batch, w.max_blocks).clone()

    def draw(shape: tuple[int, ...], std: float) -> Any:
        if w.distribution == "uniform":
            values = torch.rand(shape, generator=generator, dtype=torch.float32).mul_(0.25).sub_(0.125)
        else:
            values = torch.randn(shape, generator=generator, dtype=torch.float32)
            if std != 1.0:
                values.mul_(std)
        return values.to(dtype=dtype)

    cache_shape = (num_blocks, w.block_size, w.kv_heads, w.head_dim)
    query = draw((w.batch, w.query_heads, w.head_dim), 1.0)
    if w.draw == "chunked":
        if w.distribution != "normal":
            raise ValueError("the chunked draw is defined for normal values only")
        key_cache = _chunked_normal(torch, cache_shape, w.kv_std, dtype, seed, 0, workers)
        value_cache = _chunked_normal(torch, cache_shape, w.kv_std, dtype, seed, 1, workers)
    else:
        key_cache = draw(cache_shape, w.kv_std)
        value_cache = draw(cache_shape, w.kv_std)
    context_list = [int(c) for c in contexts]
    return {
        "query": query.to(device),
        "key_cache": key_cache.to(device),
        "value_cache": value_cache.to(device),
        "block_tables": tables.to(dtype=index).to(device),
        "context_lengths": contexts.to(dtype=index).to(device),
        "num_blocks": num_blocks,
        "kv_bytes": kv_bytes(w, context_list),
        "contexts": context_list,
        "workload": w,
        "seed": seed,
    }


INPUT_NAMES = ("query", "key_cache", "value_cache", "block_tables", "context_lengths")


def input_digests(data: dict[str, Any], workers: int = 5) -> dict[str, str]:
    """SHA-256 of the bytes of every input tensor (copied to the host), keyed by input name."""

    def digest(name: str) -> tuple[str, str]:
        tensor = data[name].detach().contiguous().cpu()
        raw = tensor.view(-1).view(__import__("torch").uint8).numpy()
        return name, hashlib.sha256(memoryview(raw)).hexdigest()

    with ThreadPoolExecutor(max_workers=workers) as pool:
        return dict(pool.map(digest, INPUT_NAMES))


def kv_bytes(workload: Workload, contexts: list[int]) -> int:
    cap = workload.max_blocks * workload.block_size
    tokens = sum(min(max(int(c), 0), cap) for c in contexts)
    return tokens * workload.kv_heads * workload.head_dim * 2 * workload.elem_size


def aux_bytes(workload: Workload, contexts: list[int], index_size: int = 4) -> int:
    """Query + output + block-table entries + context lengths a decode touches."""

    qo = 2 * workload.batch * workload.query_heads * workload.head_dim * workload.elem_size
    cap = workload.max_blocks * workload.block_size
    table = sum(math.ceil(min(max(int(c), 0), cap) / workload.block_size) for c in contexts) * index_size
    return qo + table + workload.batch * index_size


# ---------------------------------------------------------------------------------------------
# Paged KV-cache append: the cases of the reference's workload file
# (benchmarks/workloads/kv_cache_append-1.0.yaml:12-18), each in fp16 and bf16.
@dataclass(frozen=True)
class AppendCase:
    key: str
    tokens: int
    num_blocks: int
    block_size: int
    kv_heads: int
    head_dim: int

    def row_elements(self) -> int:
        return self.kv_heads * self.head_dim

    def bytes_moved(self, elem_size: int = 2) -> int:
        """Algorithmic bytes of one append: read K and V rows, write K and V rows."""

        return 4 * self.tokens * self.row_elements() * elem_size


APPEND_CASES: dict[str, AppendCase] = {
    case.key: case
    for case in (
        AppendCase("decode-t1-gqa8-d128-p16", 1, 256, 16, 8, 128),
        AppendCase("decode-t8-gqa8-d128-p16", 8, 256, 16, 8, 128),
        AppendCase("decode-t32-gqa8-d128-p16", 32, 256, 16, 8, 128),
        AppendCase("prefill-t128-gqa8-d128-p16", 128, 256, 16, 8, 128),
        AppendCase("decode-t32-gqa8-d256-p16", 32, 256, 16, 8, 256),
        AppendCase("prefill-t128-mha32-d128-p32", 128, 128, 32, 32, 128),
    )
}
APPEND_SEED = 20261301


def make_append_inputs(case: AppendCase | str, *, dtype: str = "bf16", index_dtype: str = "int64",
                       seed: int = APPEND_SEED, device: Any = "cpu") -> dict[str, Any]:
    """Seeded inputs of one append case, generated on the CPU and moved to ``device``.

    Draw order: key cache, value cache, key, value (uniform in [-0.5, 0.5), as the reference's
    benchmark draws them, benchmarks/kv_cache/benchmark.py:77-80), then the slots: the first
    ``tokens`` entries of a permutation of all ``num_blocks * block_size`` slots (unique, in range;
    benchmark.py:100-106).
    """

    import torch

    if isinstance(case, str):
        case = APPEND_CASES[case]
    gen = torch.Generator().manual_seed(seed)
    t_dtype = torch_dtype(torch, dtype)
    cache_shape = (case.num_blocks, case.block_size, case.kv_heads, case.head_dim)
    token_shape = (case.tokens, case.kv_heads, case.head_dim)

    def uniform(shape):
        return (torch.rand(shape, generator=gen, dtype=torch.float32) - 0.5).to(t_dtype)

    key_cache, value_cache = uniform(cache_shape), uniform(cache_shape)
    key, value = uniform(token_shape), uniform(token_shape)
    slots = torch.randperm(case.num_blocks * case.block_size, generator=gen)[: case.tokens]
    slots = slots.to(torch.int64 if index_dtype == "int64" else torch.int32).contiguous()
    out = {"key": key, "value": value, "key_cache": key_cache, "value_cache": value_cache, "slot_mapping": slots}
    return {name: tensor.to(device) for name, tensor in out.items()} | {"case": case, "seed": seed}


# ---------------------------------------------------------------------------------------------
# Paged KV-cache block copy: the cases of the reference's workload file
# (benchmarks/workloads/kv_cache_copy-1.0.yaml:12-17), each in fp16 and bf16.
@dataclass(frozen=True)
class CopyCase:
    key: str
    pairs: int
    num_blocks: int
    block_size: int
    kv_heads: int
    head_dim: int

    def block_elements(self) -> int:
        return self.block_size * self.kv_heads * self.head_dim

    def bytes_moved(self, elem_size: int = 2) -> int:
        """Algorithmic bytes of one copy: read source K and V blocks, write destination K and V blocks."""

        return 4 * self.pairs * self.block_elements() * elem_size


COPY_CASES: dict[str, CopyCase] = {
    case.key: case
    for case in (
        CopyCase("beam-pairs1-gqa8-d128-p16", 1, 256, 16, 8, 128),
        CopyCase("beam-pairs8-gqa8-d128-p16", 8, 256, 16, 8, 128),
        CopyCase("beam-pairs32-gqa8-d128-p16", 32, 256, 16, 8, 128),
        CopyCase("beam-pairs64-gqa8-d256-p16", 64, 256, 16, 8, 256),
        CopyCase("beam-pairs32-mha32-d128-p32", 32, 128, 32, 32, 128),
    )
}
COPY_SEED = 20261401


def make_copy_inputs(case: CopyCase | str, *, dtype: str = "bf16", index_dtype: str = "int64",
                     seed: int = COPY_SEED, device: Any = "cpu") -> dict[str, Any]:
    """Seeded inputs of one copy case, generated on the CPU and moved to ``device``.

    Draw order: key cache, value cache (uniform in [-0.5, 0.5)), then one permutation of the block
    ids whose first ``pairs`` entries are the sources and next ``pairs`` the destinations: unique,
    in range and disjoint from the sources, as the contract requires
    (contracts/kv_cache_copy-1.0.json:17; the reference's benchmark uses sources 0..pairs-1 and
    destinations pairs..2*pairs-1, benchmarks/kv_cache/benchmark.py:115-122).
    """

    import torch

    if isinstance(case, str):
        case = COPY_CASES[case]
    gen = torch.Generator().manual_seed(seed)
    t_dtype = torch_dtype(torch, dtype)
    shape = (case.num_blocks, case.block_size, case.kv_heads, case.head_dim)
    key_cache = (torch.rand(shape, generator=gen, dtype=torch.float32) - 0.5).to(t_dtype)
    value_cache = (torch.rand(shape, generator=gen, dtype=torch.float32) - 0.5).to(t_dtype)
    ids = torch.randperm(case.num_blocks, generator=gen)[: 2 * case.pairs]
    mapping = torch.stack((ids[: case.pairs], ids[case.pairs:]), dim=1)
    mapping = mapping.to(torch.int64 if index_dtype == "int64" else torch.int32).contiguous()
    out = {"key_cache": key_cache, "value_cache": value_cache, "block_mapping": mapping}
    return {name: tensor.to(device) for name, tensor in out.items()} | {"case": case, "seed": seed}


# ---------------------------------------------------------------------------------------------
# sdpa (prefill self-attention): the reference's cases (benchmarks/workloads/sdpa-1.0.yaml:13-21) and
# two long-prefill shapes of this build that fill the chip (not reference workloads).
@dataclass(frozen=True)
class SdpaCase:
    key: str
    batch: int
    query_heads: int
    kv_heads: int
    sequence: int
    head_dim: int
    causal: bool

    def flops(self) -> int:
        """Algorithmic FLOPs: 2 (QK^T) + 2 (PV) per head dim per attended (query, key) pair."""

        pairs = self.sequence * (self.sequence + 1) // 2 if self.causal else self.sequence * self.sequence
        return 4 * self.batch * self.query_heads * self.head_dim * pairs


SDPA_CASES = {case.key: case for case in (
    SdpaCase("b1-mha16-s128-d64-causal", 1, 16, 16, 128, 64, True),
    SdpaCase("b1-gqa32x8-s128-d128-causal", 1, 32, 8, 128, 128, True),
    SdpaCase("b1-gqa32x8-s256-d128-causal", 1, 32, 8, 256, 128, True),
    SdpaCase("b1-gqa32x8-s512-d128-causal", 1, 32, 8, 512, 128, True),
    SdpaCase("b4-gqa32x8-s128-d128-causal", 4, 32, 8, 128, 128, True),
    SdpaCase("b8-gqa32x8-s64-d128-causal", 8, 32, 8, 64, 128, True),
    SdpaCase("b1-mha16-s256-d64-noncausal", 1, 16, 16, 256, 64, False),
    SdpaCase("b2-gqa16x4-s256-d256-causal", 2, 16, 4, 256, 256, True),
)}
SDPA_LONG_CASES = {case.key: case for case in (
    SdpaCase("b4-gqa32x8-s4096-d128-causal", 4, 32, 8, 4096, 128, True),
    SdpaCase("b4-gqa32x8-s4096-d128-noncausal", 4, 32, 8, 4096, 128, False),
)}
SDPA_SEED = 20261501


def make_sdpa_inputs(case: SdpaCase | str, *, dtype: str = "bf16", seed: int = SDPA_SEED, device: Any = "cpu",
                     generator_device: Any = "cpu") -> dict[str, Any]:
    """Seeded N(0, 1) query/key/value of one case (generated on ``generator_device``)."""

    import torch

    c = case if isinstance(case, SdpaCase) else {**SDPA_CASES, **SDPA_LONG_CASES}[case]
    gen = torch.Generator(device=generator_device).manual_seed(seed)
    dt = torch_dtype(torch, dtype)
    shape_q = (c.batch, c.query_heads, c.sequence, c.head_dim)
    shape_kv = (c.batch, c.kv_heads, c.sequence, c.head_dim)
    tensors = {name: torch.randn(shape, generator=gen, device=generator_device).to(dt).to(device)
               for name, shape in (("query", shape_q), ("key", shape_kv), ("value", shape_kv))}
    return {**tensors, "case": c}
