"""Kernel-pack manifests (``<pack>/manifest.json``).

Document format of the reference's schemas/kernel-pack.schema.json, rules of
src/radeon_kernels/runtime/pack.py:35-157: a pack binds one environment constraint to a non-empty
list of artifacts.  An artifact record is a dispatch winner (provider, relative path, entrypoint,
SHA-256, format -- every field required here) tagged with the operator, semantic version and
evidence id it serves.  Within a pack, (operator, semantic version) pairs and artifact paths are
unique; the pack is indexed by the former, which is how the runtime looks artifacts up.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field, replace
from pathlib import Path
from types import MappingProxyType
from typing import Any, Mapping

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime import fields
from radeon_kernels.runtime.compatibility import EnvironmentConstraint
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.loader import PrecompiledArtifactLoader
from radeon_kernels.runtime.registry import ARTIFACT_FIELDS, ArtifactSpec

SUPPORTED_SCHEMA_VERSION = "1.0"

_SPEC_NAMES = tuple(spec.name for spec in ARTIFACT_FIELDS)
_ARTIFACT_RECORD = (
    fields.Field("operator", fields.identifier),
    fields.Field("semantic_version", fields.major_minor),
    *(replace(spec, required=True) for spec in ARTIFACT_FIELDS),
    fields.Field("evidence_id", fields.identifier),
)


@dataclass(frozen=True)
class KernelPackArtifact:
    operator: str
    semantic_version: str
    artifact: ArtifactSpec
    evidence_id: str

    @classmethod
    def from_mapping(cls, value: Any, path: str) -> KernelPackArtifact:
        record = fields.read_record(value, _ARTIFACT_RECORD, path)
        spec = ArtifactSpec(**{name: record.pop(name) for name in _SPEC_NAMES})
        return cls(artifact=spec, **record)

    def to_dict(self) -> dict[str, Any]:
        return {"operator": self.operator, "semantic_version": self.semantic_version, **self.artifact.to_dict(),
                "evidence_id": self.evidence_id}


def _schema_version(value: Any, path: str) -> str:
    version = fields.major_minor(value, path)
    if version != SUPPORTED_SCHEMA_VERSION:
        raise ConfigError(path, f"unsupported version {version!r}")
    return version


def _artifact_list(value: Any, path: str) -> tuple[KernelPackArtifact, ...]:
    if not isinstance(value, list) or not value:
        raise ConfigError(path, "expected a non-empty list")
    items = tuple(KernelPackArtifact.from_mapping(item, f"{path}[{index}]") for index, item in enumerate(value))
    if len({(item.operator, item.semantic_version) for item in items}) != len(items):
        raise ConfigError(path, "operator semantic versions must be unique")
    if len({item.artifact.artifact for item in items}) != len(items):
        raise ConfigError(path, "artifact paths must be unique")
    return items


_PACK_RECORD = (
    fields.Field("schema_version", _schema_version),
    fields.Field("pack_id", fields.identifier),
    fields.Field("pack_version", fields.pack_version),
    fields.Field("environment", EnvironmentConstraint.from_mapping),
    fields.Field("artifacts", _artifact_list),
)


@dataclass(frozen=True)
class KernelPack:
    root: Path
    schema_version: str
    pack_id: str
    pack_version: str
    environment: EnvironmentConstraint
    artifacts: tuple[KernelPackArtifact, ...]
    _by_operator: Mapping[tuple[str, str], KernelPackArtifact] = field(
        init=False, compare=False, repr=False, hash=False)

    def __post_init__(self) -> None:
        index = {(item.operator, item.semantic_version): item for item in self.artifacts}
        object.__setattr__(self, "_by_operator", MappingProxyType(index))

    @classmethod
    def from_directory(cls, root: Path, *, verify_artifacts: bool = True) -> KernelPack:
        try:
            resolved = Path(root).resolve(strict=True)
        except OSError as error:
            raise ConfigError(str(root), "kernel pack directory does not exist") from error
        manifest = resolved / "manifest.json"
        try:
            document = json.loads(manifest.read_text(encoding="utf-8"))
        except OSError as error:
            raise ConfigError(str(manifest), str(error)) from error
        except json.JSONDecodeError as error:
            raise ConfigError(str(manifest), f"invalid JSON: {error.msg}") from error
        pack = cls(root=resolved, **fields.read_record(document, _PACK_RECORD, str(manifest)))
        if verify_artifacts:
            loader = PrecompiledArtifactLoader(pack.root)
            for item in pack.artifacts:
                loader.resolve_and_verify(item.artifact)
        return pack

    def matches(self, fingerprint: EnvironmentFingerprint) -> bool:
        return self.environment.matches(fingerprint)

    def find(self, operator: str, semantic_version: str) -> KernelPackArtifact | None:
        return self._by_operator.get((operator, semantic_version))

    def get(self, operator: str, semantic_version: str) -> KernelPackArtifact:
        item = self.find(operator, semantic_version)
        if item is None:
            raise ConfigError(self.pack_id,
                              f"pack has no artifact for {operator!r} semantic version {semantic_version!r}")
        return item
