"""Identity of the executing ROCm environment.

Reference interface: src/radeon_kernels/runtime/fingerprint.py:37-128.  A dispatch entry or a kernel
pack applies to a process only when five identity fields are equal -- GPU architecture, wavefront
size, ROCm ABI (MAJOR.MINOR), CPython ABI tag and the exact PyTorch build string -- while
architecture features only narrow.  On MI355X the architecture is ``gfx950`` and the wavefront 64.

The five fields are defined once, as ``EnvironmentKey`` and the rule table ``_RULES`` (one checker
per field, each returning the normalised value or naming what it expected).  The fingerprint (what
this process is) and the environment constraint of manifests and packs (runtime/compatibility.py)
both build their key through that table, so they accept exactly the same values, and environment
matching is an equality of keys plus a feature-set inclusion.
"""

from __future__ import annotations

import re
import sys
from dataclasses import dataclass
from typing import Any, Callable, Iterable, Mapping, NamedTuple

from radeon_kernels.errors import RadeonKernelsError


class FingerprintError(RadeonKernelsError):
    """The local ROCm environment cannot be identified safely."""


class IdentityValueError(ValueError):
    """One identity value is invalid; the message says what was expected."""


def _architecture(value: Any) -> str:
    if isinstance(value, str) and re.fullmatch(r"gfx[0-9a-f]+", value):
        return value
    raise IdentityValueError("expected a gfx architecture")


def _wavefront(value: Any) -> int:
    if type(value) is int and value in (32, 64):
        return value
    raise IdentityValueError("expected 32 or 64")


def _rocm(value: Any) -> str:
    # "7.0.51831" -> "7.0" and "7.02.51831-rc1" -> "7.2": the ABI is the numeric major.minor prefix.
    found = re.match(r"(\d+)\.(\d+)", value.strip()) if isinstance(value, str) else None
    if found is None:
        raise IdentityValueError("expected MAJOR.MINOR")
    return f"{int(found[1])}.{int(found[2])}"


def _python_abi(value: Any) -> str:
    if isinstance(value, str) and re.fullmatch(r"cp\d{2,3}", value):
        return value
    raise IdentityValueError("expected a cpXY ABI tag")


def _pytorch(value: Any) -> str:
    if isinstance(value, str) and value:
        return value
    raise IdentityValueError("expected an exact build version")


_RULES: dict[str, Callable[[Any], Any]] = {
    "architecture": _architecture,
    "wavefront_size": _wavefront,
    "rocm_abi": _rocm,
    "python_abi": _python_abi,
    "pytorch_version": _pytorch,
}


def checked_features(values: Iterable[Any]) -> frozenset[str]:
    """Feature names: non-empty words of letters, digits and underscores."""

    features = frozenset(values)
    for item in features:
        if not (isinstance(item, str) and re.fullmatch(r"\w+", item, flags=re.ASCII)):
            raise IdentityValueError("contains an invalid feature")
    return features


class EnvironmentKey(NamedTuple):
    """The five exact-match identity fields, normalised."""

    architecture: str
    wavefront_size: int
    rocm_abi: str
    python_abi: str
    pytorch_version: str

    @classmethod
    def checked(cls, raw: Mapping[str, Any], failure: Callable[[str, str], Exception]) -> EnvironmentKey:
        """The key of ``raw``; an invalid field raises ``failure(field, expectation)``."""

        values = []
        for name, rule in _RULES.items():
            try:
                values.append(rule(raw[name]))
            except IdentityValueError as problem:
                raise failure(name, str(problem)) from None
        return cls(*values)


def normalize_rocm_abi(value: str) -> str:
    """``"7.0.51831"`` -> ``"7.0"``; leading zeros dropped; anything else is rejected."""

    try:
        return _rocm(value)
    except IdentityValueError as problem:
        raise FingerprintError(f"invalid ROCm version {value!r} ({problem})") from None


def _fingerprint_failure(name: str, problem: str) -> FingerprintError:
    return FingerprintError(f"invalid {name.replace('_', ' ')} ({problem})")


@dataclass(frozen=True)
class EnvironmentFingerprint:
    architecture: str
    wavefront_size: int
    rocm_abi: str
    python_abi: str
    pytorch_version: str
    features: tuple[str, ...] = ()

    def __post_init__(self) -> None:
        key = EnvironmentKey.checked({name: getattr(self, name) for name in EnvironmentKey._fields},
                                     _fingerprint_failure)
        for name, value in key._asdict().items():
            object.__setattr__(self, name, value)
        if isinstance(self.features, (str, bytes)):
            raise FingerprintError("features must be a collection of names")
        try:
            features = checked_features(self.features)
        except (IdentityValueError, TypeError) as problem:
            raise FingerprintError(f"invalid architecture features ({problem})") from None
        object.__setattr__(self, "features", tuple(sorted(features)))

    @property
    def key(self) -> EnvironmentKey:
        return EnvironmentKey(self.architecture, self.wavefront_size, self.rocm_abi, self.python_abi,
                              self.pytorch_version)

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any]) -> EnvironmentFingerprint:
        known = set(EnvironmentKey._fields) | {"features"}
        extra = sorted(set(value) - known)
        if extra:
            raise FingerprintError(f"unknown fingerprint fields: {extra}")
        if not set(EnvironmentKey._fields) <= set(value) or isinstance(value.get("features"), (str, bytes)):
            raise FingerprintError("fingerprint has missing or invalid fields")
        try:
            features = tuple(value.get("features", ()))
        except TypeError as error:
            raise FingerprintError("fingerprint has missing or invalid fields") from error
        return cls(**{name: value[name] for name in EnvironmentKey._fields}, features=features)

    @classmethod
    def detect(
        cls,
        *,
        torch_module: Any | None = None,
        device_index: int = 0,
        features: Iterable[str] = (),
        python_abi: str | None = None,
    ) -> EnvironmentFingerprint:
        """The fingerprint of GPU ``device_index`` as PyTorch reports it (PyTorch imported lazily)."""

        torch = torch_module
        if torch is None:
            try:
                import torch
            except ImportError as error:
                raise FingerprintError("PyTorch is required to detect the ROCm environment") from error
        if not torch.cuda.is_available():
            raise FingerprintError("no visible ROCm GPU")
        hip = getattr(torch.version, "hip", None)
        if not (isinstance(hip, str) and hip):
            raise FingerprintError("the installed PyTorch build does not report a ROCm version")
        device = torch.cuda.get_device_properties(device_index)
        wavefront = getattr(device, "warp_size", None)
        if type(wavefront) is not int:
            raise FingerprintError("PyTorch did not report the GPU wavefront size")
        # gcnArchName carries target features after the name: "gfx950:sramecc+:xnack-".
        architecture = str(getattr(device, "gcnArchName", "")).partition(":")[0]
        return cls(architecture=architecture, wavefront_size=wavefront, rocm_abi=hip,
                   python_abi=python_abi or "cp{}{}".format(*sys.version_info[:2]),
                   pytorch_version=str(torch.__version__), features=tuple(features))

    def to_dict(self) -> dict[str, Any]:
        return {**self.key._asdict(), "features": list(self.features)}
