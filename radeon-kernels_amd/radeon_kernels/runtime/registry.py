"""Dispatch manifests: strict parsing into regions, and a per-environment index of them.

Document format and rules of the reference (src/radeon_kernels/runtime/registry.py:60-401,
schemas/dispatch.schema.json:1-112), so gfx950 entries can be appended to the reference's
published manifest unchanged.

Each entry covers a *region*: its environment constraint times a workload box that holds one value
set per constrained signature key (a key the entry does not name ranges over everything).  A value
set is kept in a normal form -- closed integer intervals plus a set of typed non-integer tokens:

* a scalar ``16`` is the interval ``[16, 16]``; ``"bf16"``, ``1.5`` and ``true`` are tokens
  ``(type, value)``, so ``16``, ``16.0`` and ``true`` stay three different values;
* ``[minimum, maximum]`` (integers, ``minimum >= 1``) is one interval;
* ``{"one_of": [...]}`` is one point interval per integer choice plus the other choices' tokens.

Membership, intersection and inclusion are then interval and set operations.  Inclusion asks each
interval of the inner set to lie inside a single interval of the outer one, so a multi-valued range
is never covered by an enumeration of its members -- the reference's rule, kept.

With regions ordered by inclusion the manifest rules read: two entries whose regions intersect must
differ in priority, and the higher-priority region must be a proper subset of the lower one.
Regions of different environment keys never intersect, so a manifest is compiled once into groups
by key, each in descending priority; validation compares pairs within a group only, and selection
walks only the caller's group and takes the first entry that matches.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path
from types import MappingProxyType
from typing import Any, Iterable, Mapping

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime import fields
from radeon_kernels.runtime.compatibility import EnvironmentConstraint
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint, EnvironmentKey

SUPPORTED_SCHEMA_VERSION = "1.0"
ARTIFACT_FORMATS = ("python_extension", "hsaco")


def _is_int(value: Any) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


class ValueConstraint:
    """The admissible values of one workload key, in document form and in normal form."""

    __slots__ = ("kind", "value", "_intervals", "_tokens")

    def __init__(self, kind: str, value: Any) -> None:
        self.kind = kind  # document form: "eq" | "range" | "one_of"
        self.value = value  # the scalar, (minimum, maximum) or the tuple of choices
        if kind == "range":
            points: tuple[Any, ...] = ()
            self._intervals = (tuple(value),)
        else:
            points = value if kind == "one_of" else (value,)
            self._intervals = tuple((item, item) for item in points if _is_int(item))
        self._tokens = frozenset((type(item), item) for item in points if not _is_int(item))

    @classmethod
    def from_raw(cls, value: Any, path: str) -> ValueConstraint:
        if isinstance(value, list):
            if len(value) != 2 or not all(map(_is_int, value)) or not 1 <= value[0] <= value[1]:
                raise ConfigError(path, "integer ranges must be [minimum, maximum]")
            return cls("range", (value[0], value[1]))
        if isinstance(value, Mapping):
            choices = fields.read_record(value, [fields.Field("one_of", _choices)], path)["one_of"]
            return cls("one_of", choices)
        return cls("eq", fields.scalar(value, path))

    # -- set algebra ---------------------------------------------------------------------------
    def matches(self, value: Any) -> bool:
        if _is_int(value):
            return any(low <= value <= high for low, high in self._intervals)
        try:
            return (type(value), value) in self._tokens
        except TypeError:  # an unhashable request value is never admissible
            return False

    def overlaps(self, other: ValueConstraint) -> bool:
        return not self._tokens.isdisjoint(other._tokens) or any(
            max(a_low, b_low) <= min(a_high, b_high)
            for a_low, a_high in self._intervals for b_low, b_high in other._intervals)

    def is_subset_of(self, other: ValueConstraint) -> bool:
        return self._tokens <= other._tokens and all(
            any(b_low <= a_low and a_high <= b_high for b_low, b_high in other._intervals)
            for a_low, a_high in self._intervals)

    # -- document form -------------------------------------------------------------------------
    def to_raw(self) -> Any:
        if self.kind == "range":
            return list(self.value)
        if self.kind == "one_of":
            return {"one_of": list(self.value)}
        return self.value

    def _form(self) -> tuple[Any, ...]:
        values = self.value if self.kind != "eq" else (self.value,)
        return (self.kind, tuple((type(item), item) for item in values))

    def __eq__(self, other: object) -> bool:
        return isinstance(other, ValueConstraint) and self._form() == other._form()

    def __hash__(self) -> int:
        return hash(self._form())

    def __repr__(self) -> str:
        return f"ValueConstraint({self.kind!r}, {self.value!r})"


def _choices(value: Any, path: str) -> tuple[Any, ...]:
    if not isinstance(value, list) or not value:
        raise ConfigError(path, "expected a non-empty list")
    choices = tuple(fields.scalar(item, path) for item in value)
    if len({(type(item), item) for item in choices}) != len(choices):
        raise ConfigError(path, "contains duplicate values")
    return choices


@dataclass(frozen=True)
class WorkloadConstraint:
    """A box over signature keys: one value set per key the entry names."""

    values: Mapping[str, ValueConstraint]

    @classmethod
    def from_mapping(cls, value: Any, path: str) -> WorkloadConstraint:
        raw = fields.mapping(value, path)
        if not raw:
            raise ConfigError(path, "must contain at least one constraint")
        for key in raw:
            if not fields.is_identifier(key):
                raise ConfigError(path, f"invalid workload field: {key!r}")
        return cls(MappingProxyType({key: ValueConstraint.from_raw(item, f"{path}.{key}")
                                     for key, item in raw.items()}))

    def __eq__(self, other: object) -> bool:
        return isinstance(other, WorkloadConstraint) and dict(self.values) == dict(other.values)

    def __hash__(self) -> int:
        return hash(frozenset(self.values.items()))

    def matches(self, signature: Mapping[str, Any]) -> bool:
        return all(key in signature and allowed.matches(signature[key]) for key, allowed in self.values.items())

    def overlaps(self, other: WorkloadConstraint) -> bool:
        return all(allowed.overlaps(other.values[key]) for key, allowed in self.values.items()
                   if key in other.values)

    def is_subset_of(self, other: WorkloadConstraint) -> bool:
        # Every key ``other`` constrains must be constrained at least as tightly here.
        return all(key in self.values and self.values[key].is_subset_of(bound)
                   for key, bound in other.values.items())

    def is_strict_subset_of(self, other: WorkloadConstraint) -> bool:
        return self.is_subset_of(other) and not other.is_subset_of(self)

    def to_dict(self) -> dict[str, Any]:
        return {key: allowed.to_raw() for key, allowed in self.values.items()}


ARTIFACT_FIELDS = (
    fields.Field("provider", fields.identifier),
    fields.Field("artifact", fields.relative_path),
    fields.Field("entrypoint", fields.code_identifier),
    fields.Field("sha256", fields.sha256),
    fields.Field("format", fields.one_of(*ARTIFACT_FORMATS), required=False, default="python_extension"),
)


@dataclass(frozen=True)
class ArtifactSpec:
    provider: str
    artifact: str
    entrypoint: str
    sha256: str
    format: str = "python_extension"

    @classmethod
    def from_mapping(cls, value: Any, path: str) -> ArtifactSpec:
        return cls(**fields.read_record(value, ARTIFACT_FIELDS, path))

    def to_dict(self) -> dict[str, Any]:
        return {item.name: getattr(self, item.name) for item in ARTIFACT_FIELDS}


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
    def from_mapping(cls, value: Any, path: str) -> DispatchEntry:
        record = fields.read_record(value, _ENTRY_FIELDS, path)
        record["launch"] = MappingProxyType(record["launch"])
        return cls(**record)

    def __hash__(self) -> int:
        return hash((self.id, self.priority, self.environment, self.workload, self.winner))

    # -- regions -------------------------------------------------------------------------------
    def matches(self, fingerprint: EnvironmentFingerprint, signature: Mapping[str, Any]) -> bool:
        return self.environment.matches(fingerprint) and self.workload.matches(signature)

    def intersects(self, other: DispatchEntry) -> bool:
        return self.environment.overlaps(other.environment) and self.workload.overlaps(other.workload)

    def within(self, other: DispatchEntry) -> bool:
        return self.environment.is_subset_of(other.environment) and self.workload.is_subset_of(other.workload)

    def to_dict(self) -> dict[str, Any]:
        environment = self.environment.to_dict()
        if not environment["features"]:
            del environment["features"]
        return {"id": self.id, "priority": self.priority, "environment": environment,
                "workload": self.workload.to_dict(), "winner": self.winner.to_dict(), "launch": dict(self.launch),
                "fallbacks": list(self.fallbacks), "evidence_id": self.evidence_id}


_ENTRY_FIELDS = (
    fields.Field("id", fields.identifier),
    fields.Field("priority", fields.non_negative_int),
    fields.Field("environment", EnvironmentConstraint.from_mapping),
    fields.Field("workload", WorkloadConstraint.from_mapping),
    fields.Field("winner", ArtifactSpec.from_mapping),
    fields.Field("launch", fields.scalar_mapping),
    fields.Field("fallbacks", fields.identifier_list(non_empty=False)),
    fields.Field("evidence_id", fields.identifier),
)


def _schema_version(value: Any, path: str) -> str:
    version = fields.major_minor(value, path)
    if version != SUPPORTED_SCHEMA_VERSION:
        raise ConfigError(path, f"unsupported dispatch schema version {version!r}")
    return version


def _entry_list(value: Any, path: str) -> tuple[DispatchEntry, ...]:
    if not isinstance(value, list):
        raise ConfigError(path, "expected a list")
    return tuple(DispatchEntry.from_mapping(item, f"{path}[{position}]") for position, item in enumerate(value))


_MANIFEST_FIELDS = (
    fields.Field("schema_version", _schema_version),
    fields.Field("operator", fields.identifier),
    fields.Field("semantic_version", fields.major_minor),
    fields.Field("default_fallbacks", fields.identifier_list(non_empty=True)),
    fields.Field("entries", _entry_list),
)


def compile_groups(entries: Iterable[DispatchEntry], path: str) -> dict[EnvironmentKey, tuple[DispatchEntry, ...]]:
    """Entries grouped by environment key, each group in descending priority; relations checked."""

    groups: dict[EnvironmentKey, list[DispatchEntry]] = {}
    seen: set[str] = set()
    for entry in entries:
        if entry.id in seen:
            raise ConfigError(f"{path}.entries", "entry ids must be unique")
        seen.add(entry.id)
        groups.setdefault(entry.environment.key, []).append(entry)
    compiled = {}
    for key, group in groups.items():
        group.sort(key=lambda entry: -entry.priority)  # stable: equal priorities keep document order
        for position, high in enumerate(group):
            for low in group[position + 1:]:
                if not high.intersects(low):
                    continue
                if high.priority == low.priority:
                    raise ConfigError(f"{path}.entries",
                                      f"ambiguous overlapping entries {high.id!r} and {low.id!r}")
                if not high.within(low) or low.within(high):
                    raise ConfigError(f"{path}.entries",
                                      f"higher-priority entry {high.id!r} must be a strict subset of {low.id!r}")
        compiled[key] = tuple(group)
    return compiled


@dataclass(frozen=True)
class DispatchManifest:
    schema_version: str
    operator: str
    semantic_version: str
    default_fallbacks: tuple[str, ...]
    entries: tuple[DispatchEntry, ...]
    source: str = field(default="dispatch", compare=False, repr=False)
    _groups: Mapping[EnvironmentKey, tuple[DispatchEntry, ...]] = field(
        init=False, compare=False, repr=False, hash=False)

    def __post_init__(self) -> None:
        object.__setattr__(self, "_groups", MappingProxyType(compile_groups(self.entries, self.source)))

    @classmethod
    def from_mapping(cls, value: Any, path: str = "dispatch") -> DispatchManifest:
        return cls(**fields.read_record(value, _MANIFEST_FIELDS, path), source=path)

    @classmethod
    def from_file(cls, path: Path) -> DispatchManifest:
        try:
            document = json.loads(Path(path).read_text(encoding="utf-8"))
        except OSError as error:
            raise ConfigError(str(path), str(error)) from error
        except json.JSONDecodeError as error:
            raise ConfigError(str(path), f"invalid JSON: {error.msg}") from error
        return cls.from_mapping(document, str(path))

    def candidates(self, fingerprint: EnvironmentFingerprint) -> tuple[DispatchEntry, ...]:
        """The entries for the fingerprint's environment key, highest priority first."""

        return self._groups.get(fingerprint.key, ())

    def select(self, fingerprint: EnvironmentFingerprint, signature: Mapping[str, Any]) -> DispatchEntry | None:
        """The highest-priority matching entry (unique: entries that can both match differ in priority)."""

        for entry in self.candidates(fingerprint):
            if entry.matches(fingerprint, signature):
                return entry
        return None

    def to_dict(self) -> dict[str, Any]:
        return {"schema_version": self.schema_version, "operator": self.operator,
                "semantic_version": self.semantic_version, "default_fallbacks": list(self.default_fallbacks),
                "entries": [entry.to_dict() for entry in self.entries]}


class DispatchRegistry:
    """Manifests keyed by (operator, semantic_version)."""

    def __init__(self, manifests: Iterable[DispatchManifest] = ()) -> None:
        self._manifests: dict[tuple[str, str], DispatchManifest] = {}
        for manifest in manifests:
            self.add(manifest)

    @classmethod
    def from_directory(cls, directory: Path) -> DispatchRegistry:
        directory = Path(directory)
        if not directory.is_dir():
            raise ConfigError(str(directory), "dispatch directory does not exist")
        paths = sorted(directory.rglob("*.json"))
        if not paths:
            raise ConfigError(str(directory), "contains no dispatch manifests")
        return cls(map(DispatchManifest.from_file, paths))

    def add(self, manifest: DispatchManifest) -> None:
        operator, version = key = (manifest.operator, manifest.semantic_version)
        if key in self._manifests:
            raise ConfigError("dispatch", f"duplicate manifest for {operator} {version}")
        self._manifests[key] = manifest

    def get(self, operator: str, semantic_version: str) -> DispatchManifest:
        try:
            return self._manifests[operator, semantic_version]
        except KeyError:
            raise ConfigError("dispatch", f"no manifest for operator {operator!r} "
                                          f"semantic version {semantic_version!r}") from None

    def keys(self) -> tuple[tuple[str, str], ...]:
        return tuple(sorted(self._manifests))

