"""Dispatch manifests: strict parsing, constraint algebra and overlap validation.

Keeps the document format and matching rules of the reference
(src/radeon_kernels/runtime/registry.py:60-401, schemas/dispatch.schema.json:1-112) so that gfx950
entries can be appended to the reference's published manifest:

* a workload constraint is a scalar (``eq``: equal value *and* identical Python type), an integer
  range ``[minimum, maximum]`` with ``minimum >= 1``, or ``{"one_of": [...]}``;
* an entry matches when its environment matches the fingerprint and every workload key is present
  in the request signature and satisfied;
* two entries of one manifest that can match the same request must have different priorities, and
  the higher one must be a strict subset of the lower one.
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass
from pathlib import Path, PurePosixPath
from types import MappingProxyType
from typing import Any, Iterable, Mapping

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime.compatibility import EnvironmentConstraint
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint

IDENTIFIER = re.compile(r"[a-z][a-z0-9_.-]*")
VERSION = re.compile(r"\d+\.\d+")
SHA256 = re.compile(r"[0-9a-f]{64}")
SUPPORTED_SCHEMA_VERSION = "1.0"
ARTIFACT_FORMATS = ("python_extension", "hsaco")


def as_mapping(value: Any, path: str) -> Mapping[str, Any]:
    if not isinstance(value, Mapping):
        raise ConfigError(path, "expected a mapping")
    for key in value:
        if not isinstance(key, str):
            raise ConfigError(path, "keys must be strings")
    return value


def require_fields(value: Mapping[str, Any], allowed: Iterable[str], required: Iterable[str], path: str) -> None:
    unknown = sorted(set(value) - set(allowed))
    if unknown:
        raise ConfigError(path, f"unknown fields: {unknown}")
    missing = sorted(set(required) - set(value))
    if missing:
        raise ConfigError(path, f"missing fields: {missing}")


def identifier(value: Any, path: str) -> str:
    if isinstance(value, str) and IDENTIFIER.fullmatch(value):
        return value
    raise ConfigError(path, "expected a lowercase identifier")


def version(value: Any, path: str) -> str:
    if isinstance(value, str) and VERSION.fullmatch(value):
        return value
    raise ConfigError(path, "expected MAJOR.MINOR")


def scalar(value: Any, path: str) -> str | int | float | bool:
    if isinstance(value, (str, int, float, bool)):
        return value
    raise ConfigError(path, "expected a string, number or boolean")


def _is_int(value: Any) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _same(a: Any, b: Any) -> bool:
    """Equality with type identity: ``1 != 1.0 != True`` for dispatch purposes."""

    return type(a) is type(b) and a == b


@dataclass(frozen=True)
class ValueConstraint:
    kind: str  # "eq" | "range" | "one_of"
    value: Any

    @classmethod
    def from_raw(cls, value: Any, path: str) -> ValueConstraint:
        if isinstance(value, list):
            ok = len(value) == 2 and all(_is_int(item) for item in value)
            if not ok or value[0] <= 0 or value[1] < value[0]:
                raise ConfigError(path, "integer ranges must be [minimum, maximum]")
            return cls("range", (value[0], value[1]))
        if isinstance(value, Mapping):
            raw = as_mapping(value, path)
            require_fields(raw, {"one_of"}, {"one_of"}, path)
            choices = raw["one_of"]
            if not isinstance(choices, list) or not choices:
                raise ConfigError(f"{path}.one_of", "expected a non-empty list")
            normalized = tuple(scalar(item, f"{path}.one_of") for item in choices)
            if len(set(normalized)) != len(normalized):
                raise ConfigError(f"{path}.one_of", "contains duplicate values")
            return cls("one_of", normalized)
        return cls("eq", scalar(value, path))

    def matches(self, value: Any) -> bool:
        if self.kind == "range":
            low, high = self.value
            return _is_int(value) and low <= value <= high
        if self.kind == "eq":
            return _same(value, self.value)
        return any(_same(value, choice) for choice in self.value)

    def values(self) -> tuple[Any, ...]:
        """Representative values: the choices, or a range's endpoints."""

        if self.kind == "eq":
            return (self.value,)
        if self.kind == "one_of":
            return tuple(self.value)
        low, high = self.value
        return (low,) if low == high else (low, high)

    def overlaps(self, other: ValueConstraint) -> bool:
        if self.kind == "range" and other.kind == "range":
            return max(self.value[0], other.value[0]) <= min(self.value[1], other.value[1])
        if self.kind == "range":
            return any(self.matches(item) for item in other.values())
        return any(other.matches(item) for item in self.values())

    def is_subset_of(self, other: ValueConstraint) -> bool:
        if self.kind != "range":
            return all(other.matches(item) for item in self.values())
        low, high = self.value
        if other.kind == "range":
            return other.value[0] <= low and high <= other.value[1]
        # A multi-valued range is never treated as covered by an enumeration.
        return low == high and other.matches(low)

    def to_raw(self) -> Any:
        if self.kind == "range":
            return [self.value[0], self.value[1]]
        if self.kind == "one_of":
            return {"one_of": list(self.value)}
        return self.value


@dataclass(frozen=True)
class WorkloadConstraint:
    values: Mapping[str, ValueConstraint]

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any], path: str) -> WorkloadConstraint:
        raw = as_mapping(value, path)
        if not raw:
            raise ConfigError(path, "must contain at least one constraint")
        parsed: dict[str, ValueConstraint] = {}
        for key, item in raw.items():
            if IDENTIFIER.fullmatch(key) is None:
                raise ConfigError(path, f"invalid workload field: {key!r}")
            parsed[key] = ValueConstraint.from_raw(item, f"{path}.{key}")
        return cls(parsed)

    def matches(self, signature: Mapping[str, Any]) -> bool:
        for key, constraint in self.values.items():
            if key not in signature or not constraint.matches(signature[key]):
                return False
        return True

    def overlaps(self, other: WorkloadConstraint) -> bool:
        # Keys constrained by only one side do not separate the regions.
        for key in set(self.values) & set(other.values):
            if not self.values[key].overlaps(other.values[key]):
                return False
        return True

    def is_subset_of(self, other: WorkloadConstraint) -> bool:
        for key, constraint in other.values.items():
            mine = self.values.get(key)
            if mine is None or not mine.is_subset_of(constraint):
                return False
        return True

    def is_strict_subset_of(self, other: WorkloadConstraint) -> bool:
        if not self.is_subset_of(other):
            return False
        if set(self.values) > set(other.values):
            return True
        return any(not other.values[key].is_subset_of(self.values[key]) for key in other.values)

    def to_dict(self) -> dict[str, Any]:
        return {key: constraint.to_raw() for key, constraint in self.values.items()}


@dataclass(frozen=True)
class ArtifactSpec:
    provider: str
    artifact: str
    entrypoint: str
    sha256: str
    format: str = "python_extension"

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any], path: str) -> ArtifactSpec:
        raw = as_mapping(value, path)
        require_fields(
            raw,
            {"provider", "artifact", "entrypoint", "sha256", "format"},
            {"provider", "artifact", "entrypoint", "sha256"},
            path,
        )
        provider = identifier(raw["provider"], f"{path}.provider")
        artifact = raw["artifact"]
        if not isinstance(artifact, str) or not artifact:
            raise ConfigError(f"{path}.artifact", "expected a relative path")
        pure = PurePosixPath(artifact)
        if pure.is_absolute() or ".." in pure.parts or pure.as_posix() != artifact:
            raise ConfigError(f"{path}.artifact", "must be a normalized relative path")
        entrypoint = raw["entrypoint"]
        if not isinstance(entrypoint, str) or not entrypoint.isidentifier():
            raise ConfigError(f"{path}.entrypoint", "expected a Python/C identifier")
        digest = raw["sha256"]
        if not isinstance(digest, str) or SHA256.fullmatch(digest) is None:
            raise ConfigError(f"{path}.sha256", "expected a lowercase SHA-256")
        artifact_format = raw.get("format", "python_extension")
        if artifact_format not in ARTIFACT_FORMATS:
            raise ConfigError(f"{path}.format", "expected python_extension or hsaco")
        return cls(provider, artifact, entrypoint, digest, artifact_format)

    def to_dict(self) -> dict[str, Any]:
        return {
            "provider": self.provider,
            "artifact": self.artifact,
            "entrypoint": self.entrypoint,
            "sha256": self.sha256,
            "format": self.format,
        }


_ENTRY_FIELDS = ("id", "priority", "environment", "workload", "winner", "launch", "fallbacks", "evidence_id")


@dataclass(frozen=True)
class DispatchEntry:
    id: str
    priority: int
    environment: EnvironmentConstraint
    workload: WorkloadConstraint
    winner: ArtifactSpec
    launch: Mapping[str, str | int | float | bool]
    fallbacks: tuple[str, ...]
    evidence_id: str

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any], path: str) -> DispatchEntry:
        raw = as_mapping(value, path)
        require_fields(raw, _ENTRY_FIELDS, _ENTRY_FIELDS, path)
        priority = raw["priority"]
        if not _is_int(priority) or priority < 0:
            raise ConfigError(f"{path}.priority", "expected a non-negative integer")
        fallbacks = raw["fallbacks"]
        if not isinstance(fallbacks, list):
            raise ConfigError(f"{path}.fallbacks", "expected a list")
        parsed_fallbacks = tuple(identifier(item, f"{path}.fallbacks") for item in fallbacks)
        if len(set(parsed_fallbacks)) != len(parsed_fallbacks):
            raise ConfigError(f"{path}.fallbacks", "contains duplicates")
        launch: dict[str, str | int | float | bool] = {}
        for key, item in as_mapping(raw["launch"], f"{path}.launch").items():
            if IDENTIFIER.fullmatch(key) is None:
                raise ConfigError(f"{path}.launch", f"invalid parameter: {key!r}")
            launch[key] = scalar(item, f"{path}.launch.{key}")
        return cls(
            id=identifier(raw["id"], f"{path}.id"),
            priority=priority,
            environment=EnvironmentConstraint.from_mapping(raw["environment"], f"{path}.environment"),
            workload=WorkloadConstraint.from_mapping(raw["workload"], f"{path}.workload"),
            winner=ArtifactSpec.from_mapping(raw["winner"], f"{path}.winner"),
            launch=MappingProxyType(launch),
            fallbacks=parsed_fallbacks,
            evidence_id=identifier(raw["evidence_id"], f"{path}.evidence_id"),
        )

    def matches(self, fingerprint: EnvironmentFingerprint, signature: Mapping[str, Any]) -> bool:
        return self.environment.matches(fingerprint) and self.workload.matches(signature)

    def to_dict(self) -> dict[str, Any]:
        environment = self.environment.to_dict()
        if not environment["features"]:
            del environment["features"]
        return {
            "id": self.id,
            "priority": self.priority,
            "environment": environment,
            "workload": self.workload.to_dict(),
            "winner": self.winner.to_dict(),
            "launch": dict(self.launch),
            "fallbacks": list(self.fallbacks),
            "evidence_id": self.evidence_id,
        }


_MANIFEST_FIELDS = ("schema_version", "operator", "semantic_version", "default_fallbacks", "entries")


@dataclass(frozen=True)
class DispatchManifest:
    schema_version: str
    operator: str
    semantic_version: str
    default_fallbacks: tuple[str, ...]
    entries: tuple[DispatchEntry, ...]

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any], path: str = "dispatch") -> DispatchManifest:
        raw = as_mapping(value, path)
        require_fields(raw, _MANIFEST_FIELDS, _MANIFEST_FIELDS, path)
        entries = raw["entries"]
        if not isinstance(entries, list):
            raise ConfigError(f"{path}.entries", "expected a list")
        fallbacks = raw["default_fallbacks"]
        if not isinstance(fallbacks, list) or not fallbacks:
            raise ConfigError(f"{path}.default_fallbacks", "expected a non-empty list")
        schema_version = version(raw["schema_version"], f"{path}.schema_version")
        if schema_version != SUPPORTED_SCHEMA_VERSION:
            raise ConfigError(
                f"{path}.schema_version", f"unsupported dispatch schema version {schema_version!r}"
            )
        manifest = cls(
            schema_version=schema_version,
            operator=identifier(raw["operator"], f"{path}.operator"),
            semantic_version=version(raw["semantic_version"], f"{path}.semantic_version"),
            default_fallbacks=tuple(identifier(item, f"{path}.default_fallbacks") for item in fallbacks),
            entries=tuple(
                DispatchEntry.from_mapping(item, f"{path}.entries[{position}]")
                for position, item in enumerate(entries)
            ),
        )
        manifest.validate_relations(path)
        return manifest

    def validate_relations(self, path: str) -> None:
        if len(set(self.default_fallbacks)) != len(self.default_fallbacks):
            raise ConfigError(f"{path}.default_fallbacks", "contains duplicates")
        ids = [entry.id for entry in self.entries]
        if len(set(ids)) != len(ids):
            raise ConfigError(f"{path}.entries", "entry ids must be unique")
        for index, first in enumerate(self.entries):
            for second in self.entries[index + 1 :]:
                if not (first.environment.overlaps(second.environment) and first.workload.overlaps(second.workload)):
                    continue
                if first.priority == second.priority:
                    raise ConfigError(
                        f"{path}.entries", f"ambiguous overlapping entries {first.id!r} and {second.id!r}"
                    )
                high, low = (first, second) if first.priority > second.priority else (second, first)
                nested = high.environment.is_subset_of(low.environment) and high.workload.is_subset_of(low.workload)
                narrower = high.environment.is_strict_subset_of(low.environment) or high.workload.is_strict_subset_of(
                    low.workload
                )
                if not (nested and narrower):
                    raise ConfigError(
                        f"{path}.entries", f"higher-priority entry {high.id!r} must be a strict subset of {low.id!r}"
                    )

    @classmethod
    def from_file(cls, path: Path) -> DispatchManifest:
        try:
            document = json.loads(Path(path).read_text(encoding="utf-8"))
        except OSError as error:
            raise ConfigError(str(path), str(error)) from error
        except json.JSONDecodeError as error:
            raise ConfigError(str(path), f"invalid JSON: {error.msg}") from error
        return cls.from_mapping(document, str(path))

    def to_dict(self) -> dict[str, Any]:
        return {
            "schema_version": self.schema_version,
            "operator": self.operator,
            "semantic_version": self.semantic_version,
            "default_fallbacks": list(self.default_fallbacks),
            "entries": [entry.to_dict() for entry in self.entries],
        }


class DispatchRegistry:
    """Manifests keyed by (operator, semantic_version)."""

    def __init__(self, manifests: Iterable[DispatchManifest] = ()) -> None:
        self._by_key: dict[tuple[str, str], DispatchManifest] = {}
        for manifest in manifests:
            self.add(manifest)

    def add(self, manifest: DispatchManifest) -> None:
        key = (manifest.operator, manifest.semantic_version)
        if key in self._by_key:
            raise ConfigError("dispatch", f"duplicate manifest for {key[0]} {key[1]}")
        self._by_key[key] = manifest

    def get(self, operator: str, semantic_version: str) -> DispatchManifest:
        manifest = self._by_key.get((operator, semantic_version))
        if manifest is None:
            raise ConfigError(
                "dispatch", f"no manifest for operator {operator!r} semantic version {semantic_version!r}"
            )
        return manifest

    @classmethod
    def from_directory(cls, directory: Path) -> DispatchRegistry:
        directory = Path(directory)
        if not directory.is_dir():
            raise ConfigError(str(directory), "dispatch directory does not exist")
        files = sorted(directory.rglob("*.json"))
        if not files:
            raise ConfigError(str(directory), "contains no dispatch manifests")
        return cls(DispatchManifest.from_file(item) for item in files)

    def keys(self) -> tuple[tuple[str, str], ...]:
        return tuple(sorted(self._by_key))
