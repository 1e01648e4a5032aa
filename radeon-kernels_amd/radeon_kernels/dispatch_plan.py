"""gfx950 dispatch entries and kernel-pack manifest, rendered after each build.

The reference binds each dispatch entry to the exact artifact digest and environment
(src/radeon_kernels/runtime/registry.py:179-220, schemas/dispatch.schema.json:71-102), so the
build stamps those two fields into the documents produced here.  Everything else -- which workload
regions get which entrypoint and launch parameters -- is this table.

Regions:

* one exact entry (priority 100) per measured workload shape, with the partition size chosen for
  that shape (``launch.partition_tokens``);
* one broad gfx950 region (priority 10) covering every shape the library accepts, so any other
  gfx950 request also runs natively; shapes the kernel rejects at launch time (a ValueError) are
  demoted to the torch fallback by the runtime with the reason recorded.

All gfx950 entries share one evidence id and one pack (``packs/gfx950``).
"""

from __future__ import annotations

from typing import Any

OPERATOR = "paged_attention_decode"
SEMANTIC_VERSION = "1.0"
PACK_ID = "rk-paged-attention-decode-gfx950"
PACK_VERSION = "1.0.0"
EVIDENCE_ID = "mi355x-gfx950-paged_attention_decode-splitk-1"
ENTRYPOINT = "decode_mfma"

_INT_MAX = 2**31 - 1
_POW2_BLOCKS = [1, 2, 4, 8, 16, 32, 64, 128, 256]

# (id suffix, workload constraints, launch parameters)
EXACT_REGIONS: list[tuple[str, dict[str, Any], dict[str, Any]]] = [
    (
        "b1-gqa32x8-c128-d128-p16-fp16",
        {"dtype": "fp16", "batch": 1, "query_heads": 32, "kv_heads": 8, "head_dim": 128, "num_blocks": 64,
         "block_size": 16, "max_blocks_per_sequence": 8},
        {"partition_tokens": 128},
    ),
    (
        "b8-gqa32x8-c1024-d128-p16-bf16",
        {"dtype": "bf16", "batch": 8, "query_heads": 32, "kv_heads": 8, "head_dim": 128, "num_blocks": 1024,
         "block_size": 16, "max_blocks_per_sequence": 64},
        {"partition_tokens": 256},
    ),
    (
        "b4-mha16-c2048-d64-p32-bf16",
        {"dtype": "bf16", "batch": 4, "query_heads": 16, "kv_heads": 16, "head_dim": 64, "num_blocks": 512,
         "block_size": 32, "max_blocks_per_sequence": 64},
        {"partition_tokens": 512},
    ),
    (
        "b4-gqa32x8-c1024-d256-p16-fp16",
        {"dtype": "fp16", "batch": 4, "query_heads": 32, "kv_heads": 8, "head_dim": 256, "num_blocks": 512,
         "block_size": 16, "max_blocks_per_sequence": 64},
        {"partition_tokens": 128},
    ),
    (
        "b128-gqa32x8-ragged-d128-p16-bf16",
        {"dtype": "bf16", "batch": 128, "query_heads": 32, "kv_heads": 8, "head_dim": 128,
         "num_blocks": [1, _INT_MAX], "block_size": 16, "max_blocks_per_sequence": 1024},
        {"partition_tokens": 2048},
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
BROAD_LAUNCH = {"partition_tokens": 256}

_COMMON = {
    "index_dtype": {"one_of": ["int32", "int64"]},
    "cache_layout": "block_slot_head_dim",
    "scale_mode": {"one_of": ["default", "explicit"]},
    "contiguous": True,
    "requires_grad": False,
}


def _winner(artifact: str, sha256: str) -> dict[str, Any]:
    return {"provider": "native", "artifact": artifact, "entrypoint": ENTRYPOINT, "sha256": sha256,
            "format": "python_extension"}


def render_dispatch_manifest(*, environment: dict[str, Any], artifact: str, sha256: str) -> dict[str, Any]:
    entries = []
    for suffix, region, launch in EXACT_REGIONS:
        entries.append({
            "id": f"{OPERATOR}-gfx950-{suffix}",
            "priority": 100,
            "environment": dict(environment),
            "workload": {**region, **_COMMON},
            "winner": _winner(artifact, sha256),
            "launch": dict(launch),
            "fallbacks": ["torch"],
            "evidence_id": EVIDENCE_ID,
        })
    entries.append({
        "id": f"{OPERATOR}-gfx950-region",
        "priority": 10,
        "environment": dict(environment),
        "workload": {**BROAD_REGION, **_COMMON},
        "winner": _winner(artifact, sha256),
        "launch": dict(BROAD_LAUNCH),
        "fallbacks": ["torch"],
        "evidence_id": EVIDENCE_ID,
    })
    return {
        "schema_version": "1.0",
        "operator": OPERATOR,
        "semantic_version": SEMANTIC_VERSION,
        "default_fallbacks": ["torch"],
        "entries": entries,
    }


def render_pack_manifest(*, environment: dict[str, Any], artifact: str, sha256: str) -> dict[str, Any]:
    return {
        "schema_version": "1.0",
        "pack_id": PACK_ID,
        "pack_version": PACK_VERSION,
        "environment": dict(environment),
        "artifacts": [{
            "operator": OPERATOR,
            "semantic_version": SEMANTIC_VERSION,
            **_winner(artifact, sha256),
            "evidence_id": EVIDENCE_ID,
        }],
    }
