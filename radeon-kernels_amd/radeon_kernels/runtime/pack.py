"""Kernel-pack manifests (``<pack>/manifest.json``).

Document format of the reference's schemas/kernel-pack.schema.json and rules of
src/radeon_kernels/runtime/pack.py:35-157: a pack binds one exact environment to a list of
artifacts, each tagged with operator, semantic version, provider, relative path, entrypoint,
SHA-256, format and evidence id; (operator, semantic_version) pairs and artifact paths are unique
within a pack.
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Mapping

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime.compatibility import EnvironmentConstraint
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.loader import PrecompiledArtifactLoader
from radeon_kernels.runtime.registry import ArtifactSpec, identifier, require_fields

_VERSION = re.compile(r"\d+\.\d+")
_PACK_VERSION = re.compile(r"\d+\.\d+\.\d+")
SUPPORTED_SCHEMA_VERSION = "1.0"
_ARTIFACT_FIELDS = ("operator", "semantic_version", "provider", "artifact", "entrypoint", "sha256", "format", "evidence_id")
_PACK_FIELDS = ("schema_version", "pack_id", "pack_version", "environment", "artifacts")


def _checked_version(value: Any, path: str, pattern: re.Pattern[str]) -> str:
    if isinstance(value, str) and pattern.fullmatch(value):
        return value
    raise ConfigError(path, "invalid version")


@dataclass(frozen=True)
class KernelPackArtifact:
    operator: str
    semantic_version: str
    artifact: ArtifactSpec
    evidence_id: str

    @classmethod
    def from_mapping(cls, value: Any, path: str) -> KernelPackArtifact:
        if not isinstance(value, Mapping):
            raise ConfigError(path, "expected a mapping")
        require_fields(value, _ARTIFACT_FIELDS, _ARTIFACT_FIELDS, path)
        spec = ArtifactSpec.from_mapping(
            {key: value[key] for key in ("provider", "artifact", "entrypoint", "sha256", "format")}, path
        )
        return cls(
            operator=identifier(value["operator"], f"{path}.operator"),
            semantic_version=_checked_version(value["semantic_version"], f"{path}.semantic_version", _VERSION),
            artifact=spec,
            evidence_id=identifier(value["evidence_id"], f"{path}.evidence_id"),
        )

    def to_dict(self) -> dict[str, Any]:
        record = {"operator": self.operator, "semantic_version": self.semantic_version}
        record.update(self.artifact.to_dict())
        record["evidence_id"] = self.evidence_id
        return record


@dataclass(frozen=True)
class KernelPack:
    root: Path
    schema_version: str
    pack_id: str
    pack_version: str
    environment: EnvironmentConstraint
    artifacts: tuple[KernelPackArtifact, ...]

    @classmethod
    def from_directory(cls, root: Path, *, verify_artifacts: bool = True) -> KernelPack:
        try:
            resolved = Path(root).resolve(strict=True)
        except OSError as error:
            raise ConfigError(str(root), "kernel pack directory does not exist") from error
        manifest_path = resolved / "manifest.json"
        try:
            document = json.loads(manifest_path.read_text(encoding="utf-8"))
        except OSError as error:
            raise ConfigError(str(manifest_path), str(error)) from error
        except json.JSONDecodeError as error:
            raise ConfigError(str(manifest_path), f"invalid JSON: {error.msg}") from error
        path = str(manifest_path)
        if not isinstance(document, Mapping):
            raise ConfigError(path, "expected a mapping")
        require_fields(document, _PACK_FIELDS, _PACK_FIELDS, path)
        schema_version = _checked_version(document["schema_version"], f"{path}.schema_version", _VERSION)
        if schema_version != SUPPORTED_SCHEMA_VERSION:
            raise ConfigError(f"{path}.schema_version", f"unsupported version {schema_version!r}")
        raw_artifacts = document["artifacts"]
        if not isinstance(raw_artifacts, list) or not raw_artifacts:
            raise ConfigError(f"{path}.artifacts", "expected a non-empty list")
        pack = cls(
            root=resolved,
            schema_version=schema_version,
            pack_id=identifier(document["pack_id"], f"{path}.pack_id"),
            pack_version=_checked_version(document["pack_version"], f"{path}.pack_version", _PACK_VERSION),
            environment=EnvironmentConstraint.from_mapping(document["environment"], f"{path}.environment"),
            artifacts=tuple(
                KernelPackArtifact.from_mapping(item, f"{path}.artifacts[{index}]")
                for index, item in enumerate(raw_artifacts)
            ),
        )
        keys = [(item.operator, item.semantic_version) for item in pack.artifacts]
        if len(set(keys)) != len(keys):
            raise ConfigError(f"{path}.artifacts", "operator semantic versions must be unique")
        paths = [item.artifact.artifact for item in pack.artifacts]
        if len(set(paths)) != len(paths):
            raise ConfigError(f"{path}.artifacts", "artifact paths must be unique")
        if verify_artifacts:
            loader = PrecompiledArtifactLoader(pack.root)
            for item in pack.artifacts:
                loader.resolve_and_verify(item.artifact)
        return pack

    def matches(self, fingerprint: EnvironmentFingerprint) -> bool:
        return self.environment.matches(fingerprint)

    def get(self, operator: str, semantic_version: str) -> KernelPackArtifact:
        for item in self.artifacts:
            if item.operator == operator and item.semantic_version == semantic_version:
                return item
        raise ConfigError(
            self.pack_id, f"pack has no artifact for {operator!r} semantic version {semantic_version!r}"
        )
