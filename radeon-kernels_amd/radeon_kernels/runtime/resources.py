"""Built-in dispatch manifests shipped inside the package.

Counterpart of src/radeon_kernels/runtime/resources.py:19-43 in the reference: every ``*.json``
under ``radeon_kernels/dispatch`` is parsed strictly and registered by (operator, semantic
version).  The manifests here hold gfx950 entries only; they validate unchanged when appended to
the reference's own manifest because entries for different architectures never overlap.
"""

from __future__ import annotations

import json
from importlib.resources import files
from typing import Any, Iterator

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime.registry import DispatchManifest, DispatchRegistry


def manifest_documents(package: str = "radeon_kernels.dispatch") -> Iterator[tuple[str, Any]]:
    root = files(package)
    for resource in sorted(root.iterdir(), key=lambda item: item.name):
        if resource.name.endswith(".json"):
            try:
                yield str(resource), json.loads(resource.read_text(encoding="utf-8"))
            except json.JSONDecodeError as error:
                raise ConfigError(str(resource), f"invalid JSON: {error.msg}") from error


def builtin_dispatch_registry() -> DispatchRegistry:
    manifests = [DispatchManifest.from_mapping(document, path) for path, document in manifest_documents()]
    if not manifests:
        raise ConfigError("built-in dispatch", "contains no manifests")
    return DispatchRegistry(manifests)


def builtin_contract(operator: str, semantic_version: str) -> dict[str, Any]:
    """The operator contract document (``radeon_kernels/contracts/<operator>-<version>.json``)."""

    resource = files("radeon_kernels.contracts").joinpath(f"{operator}-{semantic_version}.json")
    return json.loads(resource.read_text(encoding="utf-8"))
