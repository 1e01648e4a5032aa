"""gfx950 dispatch entries and kernel-pack manifest, rendered after each build.

The reference binds each dispatch entry to the exact artifact digest and environment
(src/radeon_kernels/runtime/registry.py:179-220, schemas/dispatch.schema.json:71-102), so the
build stamps those two fields into the documents produced here.  Everything else -- which workload
regions get which entrypoint and launch parameters -- is this table.

Operators and regions:

* ``paged_attention_decode``: one exact entry (priority 100) per case of the reference's workload file
  in each dtype, plus the 128-sequence ragged shape, with the partition size chosen for that shape
  (``launch.partition_tokens``) and how its partition records
  are merged (``launch.merge``: ``fused`` -- the partition kernel's last workgroup per sequence and
  head slot merges, one launch -- measured 7-12% faster on the 256-workgroup shapes and 1-2% faster
  on the ragged batch's work queue; ``reduce`` -- a separate reduce launch), and one broad gfx950
  region (priority 10) covering every shape the library accepts with ``merge: auto`` (fused) and
  ``grow_partitions`` (the work-queue kernel picks a larger partition size from the live contexts);
* ``kv_cache_append`` and ``kv_cache_copy``: one exact entry per case of the reference's workload files
  (benchmarks/workloads/kv_cache_append-1.0.yaml:12-18, kv_cache_copy-1.0.yaml:12-17) and one broad
  gfx950 region each; their bindings (entrypoints ``append`` and ``copy``) share one kernel source;
* ``sdpa``: one exact entry per case of benchmarks/workloads/sdpa-1.0.yaml:13-21 (both dtypes) and
  one broad gfx950 region (the reference publishes no sdpa winner at all: dispatch/sdpa-1.0.json).

Shapes a kernel rejects at launch time (a ValueError) are demoted to the torch fallback by the
runtime with the reason recorded.  Each operator has its own binding artifact and evidence id; both
live in one pack (``packs/gfx950``).
"""

from __future__ import annotations

from typing import Any

OPERATOR = "paged_attention_decode"
SEMANTIC_VERSION = "1.0"
PACK_ID = "rk-paged-attention-gfx950"
PACK_VERSION = "1.0.0"
EVIDENCE_ID = "mi355x-gfx950-paged_attention_decode-splitk-1"
ENTRYPOINT = "decode_mfma"
ARTIFACT = "lib/rk_pa_gfx950.so"

KV_APPEND = "kv_cache_append"
KV_EVIDENCE_ID = "mi355x-gfx950-kv_cache_append-rowcopy-1"
KV_ENTRYPOINT = "append"
KV_ARTIFACT = "lib/rk_kv_append_gfx950.so"
KV_COPY = "kv_cache_copy"
KV_COPY_EVIDENCE_ID = "mi355x-gfx950-kv_cache_copy-blockcopy-1"
KV_COPY_ENTRYPOINT = "copy"
KV_COPY_ARTIFACT = "lib/rk_kv_copy_gfx950.so"
SDPA = "sdpa"
SDPA_EVIDENCE_ID = "mi355x-gfx950-sdpa-flash-1"
SDPA_ENTRYPOINT = "forward"
SDPA_ARTIFACT = "lib/rk_sdpa_gfx950.so"

_INT_MAX = 2**31 - 1
_POW2_BLOCKS = [1, 2, 4, 8, 16, 32, 64, 128, 256]

# The reference's paged-decode workload cases (benchmarks/workloads/paged_attention_decode-1.0.yaml:13-22),
# each in fp16 and bf16: id, batch, query heads, KV heads, context, head_dim, block size.  An entry
# fixes every shape field but num_blocks (the cache size does not change the launch), so it also
# covers the measured b1 / b8 / b4 shapes whose caches hold more blocks than their tables use.
REFERENCE_CASES: list[tuple[str, int, int, int, int, int, int]] = [
    ("b1-gqa32x8-c128-d128-p16", 1, 32, 8, 128, 128, 16),
    ("b1-gqa32x8-c1024-d128-p16", 1, 32, 8, 1024, 128, 16),
    ("b1-gqa32x8-c4096-d128-p16", 1, 32, 8, 4096, 128, 16),
    ("b8-gqa32x8-c128-d128-p16", 8, 32, 8, 128, 128, 16),
    ("b8-gqa32x8-c1024-d128-p16", 8, 32, 8, 1024, 128, 16),
    ("b16-gqa32x8-c2048-d128-p16", 16, 32, 8, 2048, 128, 16),
    ("b4-mha16-c2048-d64-p32", 4, 16, 16, 2048, 64, 32),
    ("b4-gqa32x8-c1024-d256-p16", 4, 32, 8, 1024, 256, 16),
]

# Launch parameters per reference case (both dtypes): partition size and merge form, the fastest whole
# call of a sweep of every case and dtype over partition sizes 16..4096 in both merge forms on MI355X,
# with K/V rotated over enough copies to read from HBM.  The fused merge won every case; both dtypes
# chose the same partition size (b1 c128 bf16 ties at 128 and 256).
_CASE_PARTITION = {
    "b1-gqa32x8-c128-d128-p16": 128,    # one partition: no merge at all
    "b1-gqa32x8-c1024-d128-p16": 128,
    "b1-gqa32x8-c4096-d128-p16": 256,
    "b8-gqa32x8-c128-d128-p16": 128,    # one partition
    "b8-gqa32x8-c1024-d128-p16": 256,
    "b16-gqa32x8-c2048-d128-p16": 1024,
    "b4-mha16-c2048-d64-p32": 512,
    "b4-gqa32x8-c1024-d256-p16": 128,
}
REFERENCE_LAUNCH: dict[tuple[str, str], dict[str, Any]] = {
    (case[0], dtype): {"partition_tokens": _CASE_PARTITION[case[0]], "merge": "fused"}
    for case in REFERENCE_CASES for dtype in ("fp16", "bf16")
}


def _reference_region(case: tuple[str, int, int, int, int, int, int], dtype: str) -> dict[str, Any]:
    _, batch, hq, hkv, context, head_dim, block_size = case
    return {"dtype": dtype, "batch": batch, "query_heads": hq, "kv_heads": hkv, "head_dim": head_dim,
            "num_blocks": [1, _INT_MAX], "block_size": block_size,
            "max_blocks_per_sequence": -(-context // block_size)}


# (id suffix, workload constraints, launch parameters)
EXACT_REGIONS: list[tuple[str, dict[str, Any], dict[str, Any]]] = [
    (f"{case[0]}-{dtype}", _reference_region(case, dtype), REFERENCE_LAUNCH[case[0], dtype])
    for case in REFERENCE_CASES for dtype in ("fp16", "bf16")
] + [
    (
        "b128-gqa32x8-ragged-d128-p16-bf16",
        {"dtype": "bf16", "batch": 128, "query_heads": 32, "kv_heads": 8, "head_dim": 128,
         "num_blocks": [1, _INT_MAX], "block_size": 16, "max_blocks_per_sequence": 1024},
        # Work-queue schedule (the library's choice for this batch): partitions of 8192 tokens, the
        # largest size the library takes, measured fastest, fused.  Five separately allocated call
        # instances each (workspace, counters, output) ran 642.8-646.2 us per call against
        # 644.3-659.2 at 4096; 6144 ran 652.1 and, earlier, 3072 651.9 and 2048 656.6.
        {"partition_tokens": 8192, "merge": "fused"},
    ),
]

BROAD_REGION: dict[str, Any] = {
    "dtype": {"one_of": ["fp16", "bf16"]},
    "batch": [1, _INT_MAX],
    "query_heads": [1, 1 << 20],
    "kv_heads": [1, 1 << 20],
    "head_dim": {"one_of": [64, 128, 256]},
    "num_blocks": [1, _INT_MAX],
    "block_size": {"one_of": _POW2_BLOCKS},
    "max_blocks_per_sequence": [1, _INT_MAX],
}
# Partitions of at least 256 tokens; on the work-queue schedule the kernel doubles them (up to 4096)
# as the context tokens per workgroup allow, judged from the live context lengths, so a table sized
# for long sequences does not coarsen the split of short ones.  On eleven batches of 16-1024
# sequences of 1 to 64k tokens it ran the fastest fixed size, 21-37% faster than 256 tokens; a
# 128k-token table (too wide for the queue at 256) starts from 512 on the queue and ran 1.5-5.9x
# faster than the grid schedule at 256.
BROAD_LAUNCH = {"partition_tokens": 256, "merge": "auto", "grow_partitions": True}

_COMMON = {
    "index_dtype": {"one_of": ["int32", "int64"]},
    "cache_layout": "block_slot_head_dim",
    "scale_mode": {"one_of": ["default", "explicit"]},
    "contiguous": True,
    "requires_grad": False,
}


# kv_cache_append: (id suffix, workload constraints).  The reference's cases, each for both dtypes.
KV_EXACT_REGIONS: list[tuple[str, dict[str, Any]]] = [
    ("decode-t1-gqa8-d128-p16", {"tokens": 1, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("decode-t8-gqa8-d128-p16", {"tokens": 8, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("decode-t32-gqa8-d128-p16", {"tokens": 32, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("prefill-t128-gqa8-d128-p16", {"tokens": 128, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("decode-t32-gqa8-d256-p16", {"tokens": 32, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 256}),
    ("prefill-t128-mha32-d128-p32", {"tokens": 128, "num_blocks": 128, "block_size": 32, "kv_heads": 32, "head_dim": 128}),
]
KV_BROAD_REGION: dict[str, Any] = {
    "tokens": [1, _INT_MAX],
    "num_blocks": [1, _INT_MAX],
    "block_size": [1, _INT_MAX],
    "kv_heads": [1, 1 << 20],
    "head_dim": {"one_of": [64, 128, 256]},
}
_KV_COMMON = {
    "dtype": {"one_of": ["fp16", "bf16"]},
    "index_dtype": {"one_of": ["int32", "int64"]},
    "layout": "block_slot_head_dim",
    "contiguous": True,
    "requires_grad": False,
}


# kv_cache_copy: (id suffix, workload constraints).  The reference's cases, each for both dtypes.
KV_COPY_EXACT_REGIONS: list[tuple[str, dict[str, Any]]] = [
    ("beam-pairs1-gqa8-d128-p16", {"pairs": 1, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("beam-pairs8-gqa8-d128-p16", {"pairs": 8, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("beam-pairs32-gqa8-d128-p16", {"pairs": 32, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 128}),
    ("beam-pairs64-gqa8-d256-p16", {"pairs": 64, "num_blocks": 256, "block_size": 16, "kv_heads": 8, "head_dim": 256}),
    ("beam-pairs32-mha32-d128-p32", {"pairs": 32, "num_blocks": 128, "block_size": 32, "kv_heads": 32, "head_dim": 128}),
]
KV_COPY_BROAD_REGION: dict[str, Any] = {
    "pairs": [1, 1 << 30],
    "num_blocks": [1, _INT_MAX],
    "block_size": [1, 1 << 20],
    "kv_heads": [1, 1 << 20],
    "head_dim": {"one_of": [64, 128, 256]},
}


# sdpa: (id suffix, workload constraints).  The reference's cases (benchmarks/workloads/sdpa-1.0.yaml:13-21),
# each for both dtypes.
SDPA_EXACT_REGIONS: list[tuple[str, dict[str, Any]]] = [
    (case, {"batch": b, "query_heads": hq, "kv_heads": hkv, "sequence": s, "head_dim": d,
            "attention_mode": "causal" if causal else "noncausal"})
    for case, b, hq, hkv, s, d, causal in (
        ("b1-mha16-s128-d64-causal", 1, 16, 16, 128, 64, True),
        ("b1-gqa32x8-s128-d128-causal", 1, 32, 8, 128, 128, True),
        ("b1-gqa32x8-s256-d128-causal", 1, 32, 8, 256, 128, True),
        ("b1-gqa32x8-s512-d128-causal", 1, 32, 8, 512, 128, True),
        ("b4-gqa32x8-s128-d128-causal", 4, 32, 8, 128, 128, True),
        ("b8-gqa32x8-s64-d128-causal", 8, 32, 8, 64, 128, True),
        ("b1-mha16-s256-d64-noncausal", 1, 16, 16, 256, 64, False),
        ("b2-gqa16x4-s256-d256-causal", 2, 16, 4, 256, 256, True),
    )
]
# Every shape of the box launches natively: grids of one round (<= 512 workgroups) take the 2-D order,
# larger ones the 1-D XCD-owned order, whose grid of at most batch * query_heads * (ceil(sequence / 128)
# + 7) workgroups stays below 2^31 here (1024 * 256 * 4103); the element count stays below 2^62.
SDPA_BROAD_REGION: dict[str, Any] = {
    "batch": [1, 1024],
    "query_heads": [1, 256],
    "kv_heads": [1, 256],
    "sequence": [1, 1 << 19],
    "head_dim": {"one_of": [64, 128, 256]},
    "attention_mode": {"one_of": ["causal", "noncausal"]},
}
_SDPA_COMMON = {
    "dtype": {"one_of": ["fp16", "bf16"]},
    "layout": "batch_head_sequence_dim",
    "scale_mode": {"one_of": ["default", "explicit"]},
    "contiguous": True,
    "requires_grad": False,
}


def _winner(artifact: str, entrypoint: str, sha256: str) -> dict[str, Any]:
    return {"provider": "native", "artifact": artifact, "entrypoint": entrypoint, "sha256": sha256,
            "format": "python_extension"}


def _entry(operator: str, suffix: str, priority: int, environment: dict[str, Any], workload: dict[str, Any],
           winner: dict[str, Any], launch: dict[str, Any], evidence_id: str) -> dict[str, Any]:
    return {
        "id": f"{operator}-gfx950-{suffix}",
        "priority": priority,
        "environment": dict(environment),
        "workload": workload,
        "winner": winner,
        "launch": dict(launch),
        "fallbacks": ["torch"],
        "evidence_id": evidence_id,
    }


def render_dispatch_manifest(operator: str, *, environment: dict[str, Any], sha256: str) -> dict[str, Any]:
    """The dispatch manifest of ``operator``; ``sha256`` is the digest of its binding artifact."""

    if operator == OPERATOR:
        winner = _winner(ARTIFACT, ENTRYPOINT, sha256)
        entries = [_entry(OPERATOR, suffix, 100, environment, {**region, **_COMMON}, winner, launch, EVIDENCE_ID)
                   for suffix, region, launch in EXACT_REGIONS]
        entries.append(_entry(OPERATOR, "region", 10, environment, {**BROAD_REGION, **_COMMON}, winner,
                              BROAD_LAUNCH, EVIDENCE_ID))
    elif operator == KV_APPEND:
        winner = _winner(KV_ARTIFACT, KV_ENTRYPOINT, sha256)
        entries = [_entry(KV_APPEND, suffix, 100, environment, {**region, **_KV_COMMON}, winner, {}, KV_EVIDENCE_ID)
                   for suffix, region in KV_EXACT_REGIONS]
        entries.append(_entry(KV_APPEND, "region", 10, environment, {**KV_BROAD_REGION, **_KV_COMMON}, winner, {},
                              KV_EVIDENCE_ID))
    elif operator == KV_COPY:
        winner = _winner(KV_COPY_ARTIFACT, KV_COPY_ENTRYPOINT, sha256)
        entries = [_entry(KV_COPY, suffix, 100, environment, {**region, **_KV_COMMON}, winner, {},
                          KV_COPY_EVIDENCE_ID) for suffix, region in KV_COPY_EXACT_REGIONS]
        entries.append(_entry(KV_COPY, "region", 10, environment, {**KV_COPY_BROAD_REGION, **_KV_COMMON}, winner,
                              {}, KV_COPY_EVIDENCE_ID))
    elif operator == SDPA:
        winner = _winner(SDPA_ARTIFACT, SDPA_ENTRYPOINT, sha256)
        entries = [_entry(SDPA, suffix, 100, environment, {**region, **_SDPA_COMMON}, winner, {}, SDPA_EVIDENCE_ID)
                   for suffix, region in SDPA_EXACT_REGIONS]
        entries.append(_entry(SDPA, "region", 10, environment, {**SDPA_BROAD_REGION, **_SDPA_COMMON}, winner, {},
                              SDPA_EVIDENCE_ID))
    else:
        raise KeyError(operator)
    return {
        "schema_version": "1.0",
        "operator": operator,
        "semantic_version": SEMANTIC_VERSION,
        "default_fallbacks": ["torch"],
        "entries": entries,
    }


def render_pack_manifest(*, environment: dict[str, Any], digests: dict[str, str]) -> dict[str, Any]:
    """The pack manifest; ``digests`` maps each operator to its binding artifact's SHA-256."""

    artifacts = [
        {"operator": OPERATOR, "semantic_version": SEMANTIC_VERSION,
         **_winner(ARTIFACT, ENTRYPOINT, digests[OPERATOR]), "evidence_id": EVIDENCE_ID},
        {"operator": KV_APPEND, "semantic_version": SEMANTIC_VERSION,
         **_winner(KV_ARTIFACT, KV_ENTRYPOINT, digests[KV_APPEND]), "evidence_id": KV_EVIDENCE_ID},
        {"operator": KV_COPY, "semantic_version": SEMANTIC_VERSION,
         **_winner(KV_COPY_ARTIFACT, KV_COPY_ENTRYPOINT, digests[KV_COPY]), "evidence_id": KV_COPY_EVIDENCE_ID},
        {"operator": SDPA, "semantic_version": SEMANTIC_VERSION,
         **_winner(SDPA_ARTIFACT, SDPA_ENTRYPOINT, digests[SDPA]), "evidence_id": SDPA_EVIDENCE_ID},
    ]
    return {
        "schema_version": "1.0",
        "pack_id": PACK_ID,
        "pack_version": PACK_VERSION,
        "environment": dict(environment),
        "artifacts": artifacts,
    }
