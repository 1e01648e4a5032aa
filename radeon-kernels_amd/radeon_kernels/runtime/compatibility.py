"""Environment constraints of dispatch entries and kernel packs.

Reference semantics: src/radeon_kernels/runtime/compatibility.py:27-127.  A constraint is an
``EnvironmentKey`` (the five exact identity fields, checked by the same rules as a fingerprint's)
plus a set of required architecture features.  Read as the set of fingerprints it accepts:

* it matches a fingerprint with an equal key that has every required feature;
* two constraints intersect exactly when their keys are equal (features only narrow);
* ``a`` is inside ``b`` when the keys are equal and ``a`` requires every feature ``b`` does.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Mapping

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime import fields
from radeon_kernels.runtime.fingerprint import (
    EnvironmentFingerprint,
    EnvironmentKey,
    IdentityValueError,
    checked_features,
)


@dataclass(frozen=True)
class EnvironmentConstraint:
    key: EnvironmentKey
    features: frozenset[str] = frozenset()

    @classmethod
    def from_mapping(cls, value: Any, path: str) -> EnvironmentConstraint:
        raw = fields.mapping(value, path)
        fields.check_keys(raw, (*EnvironmentKey._fields, "features"), EnvironmentKey._fields, path)
        key = EnvironmentKey.checked(raw, lambda name, problem: ConfigError(f"{path}.{name}", problem))
        listed = raw.get("features", [])
        if not isinstance(listed, list):
            raise ConfigError(f"{path}.features", "expected a list")
        try:
            features = checked_features(listed)
        except (IdentityValueError, TypeError):
            raise ConfigError(f"{path}.features", "contains an invalid feature") from None
        return cls(key, features)

    @property
    def architecture(self) -> str:
        return self.key.architecture

    @property
    def wavefront_size(self) -> int:
        return self.key.wavefront_size

    @property
    def rocm_abi(self) -> str:
        return self.key.rocm_abi

    @property
    def python_abi(self) -> str:
        return self.key.python_abi

    @property
    def pytorch_version(self) -> str:
        return self.key.pytorch_version

    def matches(self, fingerprint: EnvironmentFingerprint) -> bool:
        return self.key == fingerprint.key and self.features.issubset(fingerprint.features)

    def overlaps(self, other: EnvironmentConstraint) -> bool:
        return self.key == other.key

    def is_subset_of(self, other: EnvironmentConstraint) -> bool:
        return self.key == other.key and self.features >= other.features

    def is_strict_subset_of(self, other: EnvironmentConstraint) -> bool:
        return self.is_subset_of(other) and not other.is_subset_of(self)

    def to_dict(self) -> dict[str, Any]:
        return {**self.key._asdict(), "features": sorted(self.features)}
