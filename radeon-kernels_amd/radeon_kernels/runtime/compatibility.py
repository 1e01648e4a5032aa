"""Environment constraints of dispatch entries and kernel packs.

Semantics of src/radeon_kernels/runtime/compatibility.py:27-127 in the reference: a constraint
matches a fingerprint when the five identity fields are equal and the constraint's feature set is
a subset of the fingerprint's.  Two constraints overlap when their identity fields are equal
(features only narrow); a constraint is a subset of another when it overlaps it and requires at
least the other's features.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Any, Mapping

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime.fingerprint import (
    EnvironmentFingerprint,
    FingerprintError,
    normalize_rocm_abi,
)

_REQUIRED = ("architecture", "wavefront_size", "rocm_abi", "python_abi", "pytorch_version")
_ALLOWED = frozenset(_REQUIRED + ("features",))
_ARCH = re.compile(r"gfx[0-9a-f]+")


def _identity(constraint: "EnvironmentConstraint") -> tuple[Any, ...]:
    return (
        constraint.architecture,
        constraint.wavefront_size,
        constraint.rocm_abi,
        constraint.python_abi,
        constraint.pytorch_version,
    )


@dataclass(frozen=True)
class EnvironmentConstraint:
    architecture: str
    wavefront_size: int
    rocm_abi: str
    python_abi: str
    pytorch_version: str
    features: frozenset[str] = frozenset()

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any], path: str) -> EnvironmentConstraint:
        if not isinstance(value, Mapping):
            raise ConfigError(path, "expected a mapping")
        unknown = sorted(set(value) - _ALLOWED)
        if unknown:
            raise ConfigError(path, f"unknown fields: {unknown}")
        missing = sorted(set(_REQUIRED) - set(value))
        if missing:
            raise ConfigError(path, f"missing fields: {missing}")

        architecture = value["architecture"]
        if not isinstance(architecture, str) or _ARCH.fullmatch(architecture) is None:
            raise ConfigError(f"{path}.architecture", "expected a gfx architecture")
        wavefront = value["wavefront_size"]
        if isinstance(wavefront, bool) or wavefront not in (32, 64):
            raise ConfigError(f"{path}.wavefront_size", "expected 32 or 64")
        features = value.get("features", [])
        if isinstance(features, (str, bytes)) or not isinstance(features, list):
            raise ConfigError(f"{path}.features", "expected a list")
        for item in features:
            if not isinstance(item, str) or not item or not item.replace("_", "").isalnum():
                raise ConfigError(f"{path}.features", "contains an invalid feature")
        python_abi = value["python_abi"]
        if not isinstance(python_abi, str) or not python_abi.startswith("cp") or not python_abi[2:].isdigit():
            raise ConfigError(f"{path}.python_abi", "expected a cpXY ABI tag")
        pytorch_version = value["pytorch_version"]
        if not isinstance(pytorch_version, str) or not pytorch_version:
            raise ConfigError(f"{path}.pytorch_version", "expected an exact build version")
        rocm = value["rocm_abi"]
        if not isinstance(rocm, str):
            raise ConfigError(f"{path}.rocm_abi", "expected MAJOR.MINOR")
        try:
            rocm_abi = normalize_rocm_abi(rocm)
        except FingerprintError as error:
            raise ConfigError(f"{path}.rocm_abi", "expected MAJOR.MINOR") from error
        return cls(
            architecture=architecture,
            wavefront_size=wavefront,
            rocm_abi=rocm_abi,
            python_abi=python_abi,
            pytorch_version=pytorch_version,
            features=frozenset(features),
        )

    def matches(self, fingerprint: EnvironmentFingerprint) -> bool:
        return (
            _identity(self)
            == (
                fingerprint.architecture,
                fingerprint.wavefront_size,
                fingerprint.rocm_abi,
                fingerprint.python_abi,
                fingerprint.pytorch_version,
            )
            and self.features <= frozenset(fingerprint.features)
        )

    def overlaps(self, other: EnvironmentConstraint) -> bool:
        return _identity(self) == _identity(other)

    def is_subset_of(self, other: EnvironmentConstraint) -> bool:
        return self.overlaps(other) and self.features >= other.features

    def is_strict_subset_of(self, other: EnvironmentConstraint) -> bool:
        return self.is_subset_of(other) and self.features != other.features

    def to_dict(self) -> dict[str, Any]:
        record = dict(zip(_REQUIRED, _identity(self)))
        record["features"] = sorted(self.features)
        return record
