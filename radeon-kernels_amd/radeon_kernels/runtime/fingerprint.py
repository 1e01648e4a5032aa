"""Identity of the executing ROCm environment.

Interface of src/radeon_kernels/runtime/fingerprint.py:37-128 in the reference: a dispatch entry
only matches a process whose GPU architecture, wavefront size, ROCm ABI (MAJOR.MINOR), CPython ABI
tag and exact PyTorch build string equal the entry's.  On MI355X the architecture is ``gfx950`` and
the wavefront size is 64.
"""

from __future__ import annotations

import re
import sys
from dataclasses import dataclass
from typing import Any, Iterable, Mapping

from radeon_kernels.errors import RadeonKernelsError

_ARCH = re.compile(r"gfx[0-9a-f]+")
_ROCM = re.compile(r"(\d+)\.(\d+)")
_PY_ABI = re.compile(r"cp\d{2,3}")
_FIELDS = ("architecture", "wavefront_size", "rocm_abi", "python_abi", "pytorch_version", "features")


class FingerprintError(RadeonKernelsError):
    """The local ROCm environment cannot be identified safely."""


def normalize_rocm_abi(value: str) -> str:
    """``"7.0.51831"`` -> ``"7.0"``; leading zeros dropped; anything else is rejected."""

    found = _ROCM.match(value.strip())
    if found is None:
        raise FingerprintError(f"invalid ROCm version: {value!r}")
    major, minor = (int(part) for part in found.groups())
    return f"{major}.{minor}"


def _normalized_features(values: Iterable[str]) -> tuple[str, ...]:
    seen: set[str] = set()
    for item in values:
        if not isinstance(item, str) or not item or not item.replace("_", "").isalnum():
            raise FingerprintError(f"invalid architecture feature: {item!r}")
        seen.add(item)
    return tuple(sorted(seen))


@dataclass(frozen=True)
class EnvironmentFingerprint:
    architecture: str
    wavefront_size: int
    rocm_abi: str
    python_abi: str
    pytorch_version: str
    features: tuple[str, ...] = ()

    def __post_init__(self) -> None:
        if not isinstance(self.architecture, str) or _ARCH.fullmatch(self.architecture) is None:
            raise FingerprintError(f"invalid AMDGPU architecture: {self.architecture!r}")
        if isinstance(self.wavefront_size, bool) or self.wavefront_size not in (32, 64):
            raise FingerprintError("wavefront size must be 32 or 64")
        object.__setattr__(self, "rocm_abi", normalize_rocm_abi(self.rocm_abi))
        if not isinstance(self.python_abi, str) or _PY_ABI.fullmatch(self.python_abi) is None:
            raise FingerprintError("Python ABI must use the cpXY form")
        if not self.pytorch_version:
            raise FingerprintError("PyTorch version must not be empty")
        object.__setattr__(self, "features", _normalized_features(self.features))

    @classmethod
    def from_mapping(cls, value: Mapping[str, Any]) -> EnvironmentFingerprint:
        extra = sorted(set(value) - set(_FIELDS))
        if extra:
            raise FingerprintError(f"unknown fingerprint fields: {extra}")
        features = value.get("features", ())
        if isinstance(features, (str, bytes)):
            raise FingerprintError("fingerprint has missing or invalid fields")
        try:
            return cls(
                architecture=value["architecture"],
                wavefront_size=value["wavefront_size"],
                rocm_abi=value["rocm_abi"],
                python_abi=value["python_abi"],
                pytorch_version=value["pytorch_version"],
                features=tuple(features),
            )
        except (KeyError, TypeError, AttributeError) as error:
            raise FingerprintError("fingerprint has missing or invalid fields") from error

    @classmethod
    def detect(
        cls,
        *,
        torch_module: Any | None = None,
        device_index: int = 0,
        features: Iterable[str] = (),
        python_abi: str | None = None,
    ) -> EnvironmentFingerprint:
        """Read the fingerprint of ``device_index`` from PyTorch (imported lazily)."""

        if torch_module is None:
            try:
                import torch as torch_module
            except ImportError as error:
                raise FingerprintError(
                    "PyTorch is required to detect the ROCm environment"
                ) from error
        if not torch_module.cuda.is_available():
            raise FingerprintError("no visible ROCm GPU")
        hip_version = getattr(torch_module.version, "hip", None)
        if not isinstance(hip_version, str) or not hip_version:
            raise FingerprintError("the installed PyTorch build does not report a ROCm version")
        properties = torch_module.cuda.get_device_properties(device_index)
        architecture = str(getattr(properties, "gcnArchName", "")).split(":", 1)[0]
        wavefront = getattr(properties, "warp_size", None)
        if isinstance(wavefront, bool) or not isinstance(wavefront, int):
            raise FingerprintError("PyTorch did not report the GPU wavefront size")
        return cls(
            architecture=architecture,
            wavefront_size=wavefront,
            rocm_abi=hip_version,
            python_abi=python_abi or f"cp{sys.version_info.major}{sys.version_info.minor}",
            pytorch_version=str(torch_module.__version__),
            features=tuple(features),
        )

    def to_dict(self) -> dict[str, Any]:
        return {
            "architecture": self.architecture,
            "wavefront_size": self.wavefront_size,
            "rocm_abi": self.rocm_abi,
            "python_abi": self.python_abi,
            "pytorch_version": self.pytorch_version,
            "features": list(self.features),
        }
