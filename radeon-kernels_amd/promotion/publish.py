"""Turn GPU evaluations of the gfx950 pack into the reference's signed promotion records.

    python radeon-kernels_amd/promotion/publish.py        (also run by the build after every compile)

Inputs: ``evaluations/<operator>-gfx950.json`` (written on the GPU by evaluate.py), the built pack
(``packs/gfx950``) and the rendered dispatch manifests.  Outputs, all under ``radeon-kernels_amd``
and all in the reference's formats:

* ``packs/gfx950/manifest.sig.json`` -- detached signature of the pack manifest, which the runtime
  requires before it loads anything from the pack (runtime/packs.py);
* ``proposals/<proposal_id>.json`` -- the deterministic gates of
  developer/promotion/create_operator_proposal.py:87-237 (artifact and environment consistency,
  correctness, CV <= 3%, latency reduction and the lower end of its 95% paired-bootstrap interval
  >= 3% against the torch fallback) on the headline entry, and the same timing gates on every exact
  gfx950 dispatch entry of the operator, each of which must also have correctness cases;
* for a proposal whose gates all pass: ``approvals/<approval_id>.json`` (schemas/approval.schema.json),
  ``evidence/<evidence_id>.json`` (schemas/evidence.schema.json; the pack-level record, timed on the
  headline entry), one ``evidence/<evidence_id>.<entry>.json`` per exact entry (that entry's
  workload, correctness cases and timing, as the reference publishes one record per winner) and
  ``pack-index/<operator>-1.0.json`` (schemas/pack-index.schema.json), each with its ``.sig.json``;
* ``releases/<pack_id>-<pack_version>.tar.gz`` -- the release archive the pack-index record names:
  exactly the manifest, its signature and the artifacts the manifest lists (the payload the
  reference's installer accepts, installer.py:187-220), written byte-reproducibly.

What differs from the reference's flow, deliberately:

* the approval is automated and says so: reviewer ``rk-gfx950-build-gates``, a reason stating that
  every deterministic gate passed and that it is not a human release decision.  The pack and the
  records are signed with the gfx950 release key ``rk-gfx950-release-2026-12``, whose public half
  the built-in keyring ships and whose private half stays in ``.signing/`` (never committed;
  created once by ``publish.py --create-release-key``).  A machine without it signs with its own
  development key, trusted only by a process that names ``.signing/dev-trusted-keys.json`` in
  RADEON_KERNELS_DEV_TRUSTED_KEYS; this tool never writes the built-in keyring after set-up;
* one pack holds all four operators, so the pack names one evidence id per operator (the record
  timed on the headline entry) and the per-entry records sit beside it under the same approval,
  where the reference builds one pack and one evidence record per workload.

Records of a proposal that no longer passes (for example after a kernel change, until the GPU
evaluation is rerun) are removed, so the tree never shows evidence for artifacts it does not hold.
"""

from __future__ import annotations

import base64
import gzip
import hashlib
import io
import json
import os
import random
import statistics
import sys
import tarfile
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
if str(PACKAGE_ROOT) not in sys.path:
    sys.path.insert(0, str(PACKAGE_ROOT))

from radeon_kernels.errors import ConfigError  # noqa: E402
from radeon_kernels.runtime.ed25519 import Ed25519PrivateKey  # noqa: E402
from radeon_kernels.runtime.signing import (  # noqa: E402
    BUILTIN_KEYRING,
    DEV_KEYRING_ENV,
    TrustedKey,
    TrustedKeyring,
    signature_document,
)

RELEASE_KEY_ID = "rk-gfx950-release-2026-12"
DEV_KEY_ID = "rk-gfx950-dev"
KEY_DIR = PACKAGE_ROOT / ".signing"
DEV_KEYRING = KEY_DIR / "dev-trusted-keys.json"
PACK_DIR = PACKAGE_ROOT / "packs" / "gfx950"
EVALUATIONS = PACKAGE_ROOT / "evaluations"
RECORD_DIRS = {name: PACKAGE_ROOT / name for name in ("proposals", "approvals", "evidence", "pack-index")}
RELEASES = PACKAGE_ROOT / "releases"
OPERATORS = ("paged_attention_decode", "kv_cache_append", "kv_cache_copy", "sdpa")
MINIMUM_IMPROVEMENT_PCT = 3.0
MAXIMUM_CV = 0.03
REVIEWER = "rk-gfx950-build-gates"
DEV_KEY_REASON = ("development key of one gfx950 build machine: trusted only through "
                  "RADEON_KERNELS_DEV_TRUSTED_KEYS; not a release key")
RELEASE_KEY_REASON = "release key of the gfx950 pack: signs its manifest and its promotion records"


def _sha256(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def _json_bytes(value: Any) -> bytes:
    return (json.dumps(value, indent=2, sort_keys=True) + "\n").encode("utf-8")


def _write(path: Path, data: bytes) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    if path.is_file() and path.read_bytes() == data:
        return
    temporary = path.with_name(f".{path.name}.tmp")
    temporary.write_bytes(data)
    os.replace(temporary, path)


# ---------------------------------------------------------------------------------------------
# Keys
def load_private_key(path: Path) -> tuple[str, Ed25519PrivateKey, str]:
    """(key_id, key, created_at) from a private key document (developer/promotion/signing.py:66-96)."""

    if path.stat().st_mode & 0o077:
        raise ConfigError(str(path), "private key permissions must be 0600 or stricter")
    value = json.loads(path.read_text(encoding="utf-8"))
    fields = {"schema_version", "algorithm", "key_id", "private_key", "public_key", "created_at"}
    if not isinstance(value, dict) or set(value) != fields or value["algorithm"] != "ed25519":
        raise ConfigError(str(path), "invalid private key document")
    key = Ed25519PrivateKey.from_private_bytes(base64.b64decode(value["private_key"], validate=True))
    if key.public_key().public_bytes() != base64.b64decode(value["public_key"], validate=True):
        raise ConfigError(str(path), "private and public key material do not match")
    return value["key_id"], key, value["created_at"]


def generate_private_key(path: Path, key_id: str) -> None:
    key = Ed25519PrivateKey.generate()
    document = {"schema_version": "1.0", "algorithm": "ed25519", "key_id": key_id,
                "private_key": base64.b64encode(key.private_bytes()).decode("ascii"),
                "public_key": base64.b64encode(key.public_key().public_bytes()).decode("ascii"),
                "created_at": datetime.now(timezone.utc).isoformat()}
    path.parent.mkdir(parents=True, exist_ok=True)
    descriptor = os.open(path, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o600)
    with os.fdopen(descriptor, "w", encoding="utf-8") as stream:
        json.dump(document, stream, indent=2, sort_keys=True)


def _public_b64(key: Ed25519PrivateKey) -> str:
    return base64.b64encode(key.public_key().public_bytes()).decode("ascii")


def signing_key() -> tuple[str, Ed25519PrivateKey]:
    """(key_id, key) that signs the pack and the promotion records.

    The release key ``rk-gfx950-release-2026-12`` when its private half is present in ``.signing/``
    and matches the public key the built-in keyring ships; otherwise this machine's development key
    (created on first use), whose public half goes to ``.signing/dev-trusted-keys.json`` only.  The
    built-in keyring (radeon_kernels/keys/trusted-keys.json) is never written here: a pack signed with
    a development key loads only in a process that sets RADEON_KERNELS_DEV_TRUSTED_KEYS to that file.
    """

    release = KEY_DIR / f"{RELEASE_KEY_ID}.private.json"
    if release.is_file():
        key_id, key, _ = load_private_key(release)
        shipped = {entry.key_id: entry for entry in TrustedKeyring.from_file(BUILTIN_KEYRING).keys}
        entry = shipped.get(key_id)
        if entry is None or entry.status != "active" or entry.public_key != key.public_key().public_bytes():
            raise ConfigError(str(release), "release key does not match the active key the built-in keyring ships")
        return key_id, key
    path = KEY_DIR / f"{DEV_KEY_ID}.private.json"
    if not path.is_file():
        generate_private_key(path, DEV_KEY_ID)
    key_id, key, created_at = load_private_key(path)
    dev_ring = TrustedKeyring([TrustedKey(key_id, key.public_key().public_bytes(), "active", created_at,
                                          DEV_KEY_REASON)])
    _write(DEV_KEYRING, _json_bytes(dev_ring.to_dict()))
    sys.stderr.write(f"warning: no release key in {KEY_DIR}; the pack is signed with the development key {key_id} "
                     f"and loads only with {DEV_KEYRING_ENV}={DEV_KEYRING}\n")
    return key_id, key


def create_release_key() -> str:
    """One-time set-up of the gfx950 release key: its private half goes to ``.signing/`` (never
    committed) and its public half is added to the built-in keyring.  Refuses to replace a key."""

    path = KEY_DIR / f"{RELEASE_KEY_ID}.private.json"
    keyring = TrustedKeyring.from_file(BUILTIN_KEYRING)
    if any(entry.key_id == RELEASE_KEY_ID for entry in keyring.keys) or path.exists():
        raise ConfigError(RELEASE_KEY_ID, "the release key already exists; rotate it by hand, not by this tool")
    generate_private_key(path, RELEASE_KEY_ID)
    key_id, key, created_at = load_private_key(path)
    keys = [entry for entry in keyring.keys]
    keys.append(TrustedKey(key_id, key.public_key().public_bytes(), "active", created_at, RELEASE_KEY_REASON))
    _write(BUILTIN_KEYRING, _json_bytes(TrustedKeyring(keys).to_dict()))
    return _public_b64(key)


def sign(path: Path, key_id: str, key: Ed25519PrivateKey, signed_file: str | None = None) -> Path:
    """Write ``<stem>.sig.json`` beside ``path`` (``manifest.sig.json`` for ``manifest.json``)."""

    name = signed_file or path.name
    document = signature_document(private_key=key, key_id=key_id, signed_file=name,
                                  signed_sha256=_sha256(path.read_bytes()))
    target = path.with_name(path.name[: -len(".json")] + ".sig.json")
    _write(target, _json_bytes(document))
    return target


# ---------------------------------------------------------------------------------------------
# Gates (developer/promotion/create_operator_proposal.py:37-58,87-237)
def latency_reduction(candidate: list[float], baseline: list[float]) -> float:
    return (1.0 - statistics.median(candidate) / statistics.median(baseline)) * 100.0


def bootstrap_interval(candidate: list[float], baseline: list[float], resamples: int = 10_000) -> tuple[float, float]:
    """95% paired-bootstrap interval of the latency reduction (fixed seed: reproducible)."""

    if len(candidate) != len(baseline) or len(candidate) < 2:
        raise ConfigError("evaluation.timing", "candidate and baseline samples must be paired")
    generator = random.Random(20260917)
    estimates = []
    n = len(candidate)
    for _ in range(resamples):
        picks = [generator.randrange(n) for _ in range(n)]
        estimates.append(latency_reduction([candidate[i] for i in picks], [baseline[i] for i in picks]))
    estimates.sort()
    return estimates[int(0.025 * (resamples - 1))], estimates[int(0.975 * (resamples - 1))]


def _scalar_workload(constraints: dict[str, Any]) -> dict[str, Any]:
    """A dispatch workload constraint as the scalar mapping the evidence schema allows."""

    out = {}
    for key, value in constraints.items():
        if isinstance(value, list):
            out[key] = f"{value[0]}..{value[1]}"
        elif isinstance(value, dict):
            out[key] = "|".join(str(item) for item in value["one_of"])
        else:
            out[key] = value
    return out


def timing_summary(timing: dict[str, Any], baseline_name: str) -> dict[str, Any]:
    """The evidence schema's timing object from one paired timing record of an evaluation."""

    candidate = [float(v) for v in timing["candidate"]["samples_ms"]]
    baseline = [float(v) for v in timing["baseline"]["samples_ms"]]
    interval = bootstrap_interval(candidate, baseline)
    candidate_cv = float(timing["candidate"]["coefficient_of_variation"])
    baseline_cv = float(timing["baseline"]["coefficient_of_variation"])
    return {
        "baseline": baseline_name,
        "candidate_samples_ms": candidate,
        "baseline_samples_ms": baseline,
        "candidate_median_ms": float(timing["candidate"]["median_ms"]),
        "baseline_median_ms": float(timing["baseline"]["median_ms"]),
        "candidate_cv": candidate_cv,
        "baseline_cv": baseline_cv,
        "latency_reduction_pct": latency_reduction(candidate, baseline),
        "confidence_interval_pct": list(interval),
        "stable": candidate_cv <= MAXIMUM_CV and baseline_cv <= MAXIMUM_CV,
    }


def public_case(case: dict[str, Any]) -> dict[str, Any]:
    """A correctness case in the evidence schema's fields (guards_intact where it was checked)."""

    out = {"case_id": case["case_id"], "seed": int(case["seed"]), "runtime_ok": bool(case["runtime_ok"]),
           "finite": bool(case["finite"]), "max_absolute_error": float(case["max_absolute_error"])}
    if "guards_intact" in case:
        out["guards_intact"] = bool(case["guards_intact"])
    return out


def proposal_for(operator: str, evaluation_path: Path) -> dict[str, Any]:
    from radeon_kernels.runtime.pack import KernelPack
    from radeon_kernels.runtime.registry import DispatchManifest

    evaluation = json.loads(evaluation_path.read_text(encoding="utf-8"))
    pack = KernelPack.from_directory(PACK_DIR, verify_artifacts=True)
    dispatch_path = PACKAGE_ROOT / "radeon_kernels" / "dispatch" / f"{operator}-1.0.json"
    dispatch_raw = json.loads(dispatch_path.read_text(encoding="utf-8"))
    manifest = DispatchManifest.from_mapping(dispatch_raw, str(dispatch_path))
    item = pack.get(operator, "1.0")
    gfx950 = [entry for entry in manifest.entries if entry.environment.architecture == "gfx950"]
    exact_ids = {entry.id for entry in gfx950 if not entry.id.endswith("-region")}
    headline_entry = next((raw for raw in dispatch_raw["entries"] if raw["id"] == evaluation["headline_entry_id"]),
                          None)
    if headline_entry is None:
        raise ConfigError(str(evaluation_path), f"no dispatch entry {evaluation['headline_entry_id']!r}")
    timing = evaluation["timing"]
    candidate = [float(v) for v in timing["candidate"]["samples_ms"]]
    baseline = [float(v) for v in timing["baseline"]["samples_ms"]]
    reduction = latency_reduction(candidate, baseline)
    interval = bootstrap_interval(candidate, baseline)
    per_entry = {entry_id: timing_summary(record["timing"], record["timing"].get("baseline_method",
                                                                                  evaluation["baseline"]))
                 for entry_id, record in evaluation.get("entries", {}).items()}
    env = evaluation["environment"]
    pack_env = pack.environment
    gates = {
        "artifact_matches_dispatch": all(entry.winner == item.artifact for entry in gfx950),
        "artifact_hash_consistent": evaluation["candidate"]["artifact_sha256"] == item.artifact.sha256,
        "environment_consistent": (env["architecture"] == pack_env.architecture
                                   and int(env["wavefront_size"]) == pack_env.wavefront_size
                                   and env["rocm_abi"] == pack_env.rocm_abi
                                   and env["pytorch_version"] == pack_env.pytorch_version),
        "exact_entries_covered": exact_ids <= {case["entry_id"] for case in evaluation["cases"]},
        "correctness_passed": all(case["passed"] for case in evaluation["cases"]),
        "candidate_stable": timing["candidate"]["coefficient_of_variation"] <= MAXIMUM_CV,
        "baseline_stable": timing["baseline"]["coefficient_of_variation"] <= MAXIMUM_CV,
        "improvement_threshold_passed": reduction >= MINIMUM_IMPROVEMENT_PCT,
        "confidence_threshold_passed": interval[0] >= MINIMUM_IMPROVEMENT_PCT,
        "every_exact_entry_timed": exact_ids <= set(per_entry),
        "graph_replays_match_eager": all(record["timing"].get("graph_replay_matches_eager", True)
                                         for record in evaluation.get("entries", {}).values()),
        "every_entry_stable": bool(per_entry) and all(t["stable"] for t in per_entry.values()),
        "every_entry_improved": bool(per_entry) and all(
            t["latency_reduction_pct"] >= MINIMUM_IMPROVEMENT_PCT
            and t["confidence_interval_pct"][0] >= MINIMUM_IMPROVEMENT_PCT for t in per_entry.values()),
    }
    failed = [name for name, passed in gates.items() if not passed]
    decision = "promote" if not failed else "needs_review"
    sources = {
        "candidate_source": evaluation["candidate"]["source_sha256"],
        "dispatch": _sha256(dispatch_path.read_bytes()),
        "evaluation": _sha256(evaluation_path.read_bytes()),
        "manifest": _sha256((PACK_DIR / "manifest.json").read_bytes()),
    }
    environment = {k: v for k, v in pack_env.to_dict().items() if k != "features"}
    case_entry = {case["case_id"]: case["entry_id"] for case in evaluation["cases"]}
    workload = _scalar_workload(headline_entry["workload"])
    workload["evidence_scope"] = (f"all {len(exact_ids)} exact gfx950 entries (correctness); "
                                  f"timing on {evaluation['headline_entry_id']}")
    public_evidence = {
        "schema_version": "1.0",
        "evidence_id": item.evidence_id,
        "operator": operator,
        "semantic_version": "1.0",
        "candidate_content_hash": item.artifact.sha256,
        "captured_at": evaluation["captured_at"],
        "environment": environment,
        "workload": workload,
        "correctness": {
            "passed": gates["correctness_passed"],
            "oracle": evaluation["oracle"],
            "cases": [public_case(case) for case in evaluation["cases"]],
        },
        "timing": timing_summary(timing, evaluation["baseline"]),
        "source_evidence_hashes": sources,
        "decision": decision,
        "guarantee_boundary": (
            f"Exact {pack_env.architecture}, ROCm {pack_env.rocm_abi}, {pack_env.python_abi}, PyTorch "
            f"{pack_env.pytorch_version}; the exact gfx950 dispatch entries "
            f"{', '.join(sorted(exact_ids))}; contiguous inference only."),
    }
    # One evidence record per exact entry, as the reference publishes one per winner: that entry's
    # workload, correctness cases and paired timing.
    raw_entries = {raw["id"]: raw for raw in dispatch_raw["entries"]}
    prefix = f"{operator}-gfx950-"
    entry_evidence = []
    for entry_id in sorted(exact_ids & set(per_entry)):
        entry_cases = [case for case in public_evidence["correctness"]["cases"]
                       if case_entry.get(case["case_id"]) == entry_id]
        entry_evidence.append({
            **public_evidence,
            "evidence_id": f"{item.evidence_id}.{entry_id[len(prefix):]}",
            "workload": _scalar_workload(raw_entries[entry_id]["workload"]),
            "correctness": {"passed": all(c["passed"] for c in evaluation["cases"] if c["entry_id"] == entry_id),
                            "oracle": evaluation["oracle"], "cases": entry_cases},
            "timing": per_entry[entry_id],
            "guarantee_boundary": (
                f"Exact {pack_env.architecture}, ROCm {pack_env.rocm_abi}, {pack_env.python_abi}, PyTorch "
                f"{pack_env.pytorch_version}; the gfx950 dispatch entry {entry_id}; contiguous inference only."),
        })
    # The broad region, when the evaluation sampled it: one record over all its sampled shapes (timing on the
    # first) and one per sampled shape with that shape's cases and paired timing.
    for region_id in sorted(entry.id for entry in gfx950 if entry.id.endswith("-region")):
        samples = [key for key in evaluation.get("entries", {}) if key.startswith(region_id + "/")]
        if not samples:
            continue
        region_cases = [case for case in public_evidence["correctness"]["cases"]
                        if case_entry.get(case["case_id"]) == region_id]
        names = [evaluation["entries"][key]["workload"] for key in samples]
        correctness = {"passed": all(c["passed"] for c in evaluation["cases"] if c["entry_id"] == region_id),
                       "oracle": evaluation["oracle"], "cases": region_cases}
        boundary = (f"Exact {pack_env.architecture}, ROCm {pack_env.rocm_abi}, {pack_env.python_abi}, PyTorch "
                    f"{pack_env.pytorch_version}; the gfx950 dispatch entry {region_id}")
        entry_evidence.append({
            **public_evidence,
            "evidence_id": f"{item.evidence_id}.{region_id[len(prefix):]}",
            "workload": {**_scalar_workload(raw_entries[region_id]["workload"]),
                         "evidence_scope": (f"{len(samples)} sampled shapes of the region ({', '.join(names)}): "
                                            f"correctness on every one, timing on {names[0]} (each shape's timing in "
                                            f"its own record)")},
            "correctness": correctness,
            "timing": per_entry[samples[0]],
            "guarantee_boundary": boundary + "; the sampled shapes named in the workload; contiguous inference only.",
        })
        for key, name in zip(samples, names):
            cases_here = [case for case in region_cases if case["case_id"].startswith(name + "-seed")]
            entry_evidence.append({
                **public_evidence,
                "evidence_id": f"{item.evidence_id}.{name}",
                "workload": {**evaluation["entries"][key]["region_sample"], "evidence_scope": f"sampled from {region_id}"},
                "correctness": {"passed": all(c["passed"] for c in evaluation["cases"]
                                              if c["entry_id"] == region_id and c["workload"] == name),
                                "oracle": evaluation["oracle"], "cases": cases_here},
                "timing": per_entry[key],
                "guarantee_boundary": boundary + f", on the sampled shape {name}; contiguous inference only.",
            })
    identity = _sha256(json.dumps({"evidence_id": item.evidence_id, "sources": sources},
                                  sort_keys=True).encode())[:16]
    return {
        "schema_version": "1.0",
        "proposal_id": f"proposal-{item.evidence_id}-{identity}",
        "created_at": evaluation["captured_at"],
        "operator": operator,
        "semantic_version": "1.0",
        "entry_ids": sorted(entry.id for entry in gfx950),
        "pack": {"pack_id": pack.pack_id, "pack_version": pack.pack_version, "manifest_sha256": sources["manifest"],
                 "environment": environment, "artifacts": [a.to_dict() for a in pack.artifacts]},
        "source_evidence_hashes": sources,
        "gates": gates,
        "minimum_improvement_pct": MINIMUM_IMPROVEMENT_PCT,
        "maximum_cv": MAXIMUM_CV,
        "recommended_decision": decision,
        "reasons": ["all deterministic promotion gates passed"] if not failed else failed,
        "public_evidence": public_evidence,
        "entry_evidence": entry_evidence,
    }


# ---------------------------------------------------------------------------------------------
# Release archive
def release_archive(pack_id: str, pack_version: str, files: list[str]) -> Path:
    """Byte-reproducible ``<pack_id>-<version>.tar.gz`` of ``files`` (paths relative to the pack)."""

    buffer = io.BytesIO()
    with tarfile.open(fileobj=buffer, mode="w", format=tarfile.PAX_FORMAT) as archive:
        for name in sorted(files):
            data = (PACK_DIR / name).read_bytes()
            info = tarfile.TarInfo(f"{pack_id}/{name}")
            info.size = len(data)
            info.mode = 0o755 if name.endswith(".so") else 0o644
            info.mtime = 0
            info.uid = info.gid = 0
            info.uname = info.gname = ""
            archive.addfile(info, io.BytesIO(data))
    compressed = io.BytesIO()
    with gzip.GzipFile(fileobj=compressed, mode="wb", mtime=0, filename="") as stream:
        stream.write(buffer.getvalue())
    target = RELEASES / f"{pack_id}-{pack_version}.tar.gz"
    _write(target, compressed.getvalue())
    return target


# ---------------------------------------------------------------------------------------------
def publish(verbose: bool = False) -> dict[str, str]:
    """Sign the pack and (re)write every promotion record; returns operator -> decision."""

    key_id, key = signing_key()
    manifest_path = PACK_DIR / "manifest.json"
    manifest_sig = sign(manifest_path, key_id, key)
    manifest = json.loads(manifest_path.read_text(encoding="utf-8"))
    archive = release_archive(manifest["pack_id"], manifest["pack_version"],
                              ["manifest.json", "manifest.sig.json", *[a["artifact"] for a in manifest["artifacts"]]])
    release_bytes = archive.read_bytes()

    keep: set[Path] = set()
    decisions = {}
    for operator in OPERATORS:
        evaluation = EVALUATIONS / f"{operator}-gfx950.json"
        if not evaluation.is_file():
            decisions[operator] = "not evaluated"
            continue
        proposal = proposal_for(operator, evaluation)
        proposal_path = RECORD_DIRS["proposals"] / f"{proposal['proposal_id']}.json"
        _write(proposal_path, _json_bytes(proposal))
        keep.add(proposal_path)
        decisions[operator] = proposal["recommended_decision"]
        if proposal["recommended_decision"] != "promote":
            continue
        approval_id = f"approval-{proposal['proposal_id']}-approved"
        approval = {
            "schema_version": "1.0",
            "approval_id": approval_id,
            "proposal_id": proposal["proposal_id"],
            "proposal_sha256": _sha256(proposal_path.read_bytes()),
            "decision": "approved",
            "reviewer": REVIEWER,
            "reviewed_at": proposal["created_at"],
            "reason": ("Automated approval by the gfx950 build: every deterministic promotion gate passed ("
                       + ", ".join(proposal["gates"]) + f"). Signed with {key_id}; "
                       "not a human release decision."),
        }
        evidence = dict(proposal["public_evidence"], approval_id=approval_id)
        index = {
            "schema_version": "1.0",
            "operator": operator,
            "semantic_version": "1.0",
            "packs": [{
                "pack_id": manifest["pack_id"],
                "pack_version": manifest["pack_version"],
                "environment": manifest["environment"],
                "manifest_sha256": _sha256(manifest_path.read_bytes()),
                "manifest_signature": json.loads(manifest_sig.read_text(encoding="utf-8")),
                "release_file": archive.name,
                "release_sha256": _sha256(release_bytes),
                "release_size": len(release_bytes),
                "artifacts": manifest["artifacts"],
                "approval_id": approval_id,
            }],
        }
        documents = [("approvals", approval_id, approval), ("evidence", evidence["evidence_id"], evidence),
                     ("pack-index", f"{operator}-1.0", index)]
        documents += [("evidence", record["evidence_id"], dict(record, approval_id=approval_id))
                      for record in proposal["entry_evidence"]]
        for directory, name, document in documents:
            path = RECORD_DIRS[directory] / f"{name}.json"
            _write(path, _json_bytes(document))
            keep.update({path, sign(path, key_id, key)})
    for directory in RECORD_DIRS.values():
        for stale in directory.glob("*.json") if directory.is_dir() else ():
            if stale not in keep:
                stale.unlink()
    if verbose:
        print(json.dumps(decisions), flush=True)
    return decisions


if __name__ == "__main__":
    if sys.argv[1:] == ["--create-release-key"]:
        print(f"created {RELEASE_KEY_ID}: public key {create_release_key()}")
    else:
        publish(verbose=True)
