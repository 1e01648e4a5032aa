"""Verified loading of precompiled kernel artifacts.

Interface of src/radeon_kernels/runtime/loader.py:65-121 in the reference (path-escape and SHA-256
checks, ``python_extension`` import, ``hsaco`` needing a provider-specific launcher), with two
deliberate differences:

* the Python module name is the artifact's file stem (``lib/rk_pa_gfx950.so`` -> ``rk_pa_gfx950``),
  fixed at build time; the binary is never scanned for ``PyInit_`` symbols;
* an artifact is hashed once, when it is first loaded, and the resolved entrypoint is cached, so a
  dispatch call does not re-hash the shared object (the reference hashes it twice per call).
"""

from __future__ import annotations

import hashlib
import importlib.util
import sys
import threading
from dataclasses import dataclass
from pathlib import Path
from types import ModuleType
from typing import Any, Callable

from radeon_kernels.errors import RadeonKernelsError
from radeon_kernels.runtime.registry import ArtifactSpec


class ArtifactError(RadeonKernelsError):
    """Base class for precompiled kernel-pack failures."""


class ArtifactIntegrityError(ArtifactError):
    """An artifact path escapes its pack or its digest does not match."""


class ArtifactLoadError(ArtifactError):
    """A verified artifact cannot be loaded."""


def sha256_file(path: Path) -> str:
    digest = hashlib.sha256()
    with Path(path).open("rb") as stream:
        for chunk in iter(lambda: stream.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


def module_name_for(path: Path) -> str:
    """Module name of a python_extension artifact: the file name up to its first dot."""

    name = Path(path).name.split(".", 1)[0]
    if not name.isidentifier():
        raise ArtifactLoadError(f"artifact {Path(path).name} does not name a Python module")
    return name


@dataclass(frozen=True)
class LoadedEntrypoint:
    artifact: Path
    provider: str
    entrypoint: str
    callable: Callable[..., Any]


class PrecompiledArtifactLoader:
    """Loads artifacts of one pack root; each artifact is verified once per process."""

    def __init__(self, pack_root: Path) -> None:
        try:
            self._root = Path(pack_root).resolve(strict=True)
        except OSError as error:
            raise ArtifactIntegrityError(f"kernel pack root is unavailable: {pack_root}") from error
        if not self._root.is_dir():
            raise ArtifactIntegrityError(f"kernel pack root is not a directory: {pack_root}")
        self._modules: dict[Path, ModuleType] = {}
        self._entrypoints: dict[ArtifactSpec, LoadedEntrypoint] = {}
        self._lock = threading.Lock()

    @property
    def root(self) -> Path:
        return self._root

    def resolve_and_verify(self, artifact: ArtifactSpec) -> Path:
        candidate = (self._root / artifact.artifact).resolve()
        if not candidate.is_relative_to(self._root):
            raise ArtifactIntegrityError("artifact escapes the kernel pack root")
        if not candidate.is_file():
            raise ArtifactIntegrityError(f"artifact is missing: {artifact.artifact}")
        actual = sha256_file(candidate)
        if actual != artifact.sha256:
            raise ArtifactIntegrityError(
                f"artifact SHA-256 mismatch for {artifact.artifact}: expected {artifact.sha256}, got {actual}"
            )
        return candidate

    def load_module(self, artifact: ArtifactSpec) -> ModuleType:
        if artifact.format != "python_extension":
            raise ArtifactLoadError(f"artifact format {artifact.format!r} requires a provider-specific launcher")
        path = self.resolve_and_verify(artifact)
        with self._lock:
            module = self._modules.get(path)
            if module is not None:
                return module
            name = module_name_for(path)
            existing = sys.modules.get(name)
            if existing is not None and Path(getattr(existing, "__file__", "")).resolve() == path:
                self._modules[path] = existing
                return existing
            spec = importlib.util.spec_from_file_location(name, path)
            if spec is None or spec.loader is None:
                raise ArtifactLoadError(f"cannot create an import specification for {path.name}")
            try:
                # For a native extension, module_from_spec already dlopens the shared object.
                module = importlib.util.module_from_spec(spec)
                spec.loader.exec_module(module)
            except Exception as error:  # import of a shared object can raise anything
                raise ArtifactLoadError(f"failed to load {path.name}: {error}") from error
            sys.modules.setdefault(name, module)
            self._modules[path] = module
            return module

    def load_entrypoint(self, artifact: ArtifactSpec) -> LoadedEntrypoint:
        cached = self._entrypoints.get(artifact)
        if cached is not None:
            return cached
        module = self.load_module(artifact)
        function = getattr(module, artifact.entrypoint, None)
        if not callable(function):
            raise ArtifactLoadError(f"artifact {artifact.artifact} does not export callable {artifact.entrypoint!r}")
        loaded = LoadedEntrypoint(
            artifact=(self._root / artifact.artifact).resolve(),
            provider=artifact.provider,
            entrypoint=artifact.entrypoint,
            callable=function,
        )
        with self._lock:
            self._entrypoints.setdefault(artifact, loaded)
        return loaded
