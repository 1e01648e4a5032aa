"""Provider that invokes a native (precompiled) dispatch winner.

Interface of src/radeon_kernels/providers/native.py:14-28 in the reference: the resolved
entrypoint is called as ``entrypoint(*arguments, **launch)`` with the entry's static launch
parameters; a ``None`` return is an error.  The provider holds no operator-specific policy.
"""

from __future__ import annotations

from typing import Any, Callable, Mapping

from radeon_kernels.errors import RadeonKernelsError
from radeon_kernels.runtime.loader import PrecompiledArtifactLoader
from radeon_kernels.runtime.registry import ArtifactSpec


class NativeProviderError(RadeonKernelsError):
    """An approved native launch cannot be executed safely."""


def resolve(loader: PrecompiledArtifactLoader, artifact: ArtifactSpec) -> Callable[..., Any]:
    """The winner's callable, loaded (and digest-checked) through ``loader``."""

    if artifact.provider != "native":
        raise NativeProviderError(f"unsupported native winner provider: {artifact.provider!r}")
    return loader.load_entrypoint(artifact).callable


def invoke(entrypoint: Callable[..., Any], launch: Mapping[str, str | int | float | bool], *arguments: Any) -> Any:
    result = entrypoint(*arguments, **launch)
    if result is None:
        raise NativeProviderError("native entrypoint returned no output")
    return result


def execute(
    loader: PrecompiledArtifactLoader,
    artifact: ArtifactSpec,
    launch: Mapping[str, str | int | float | bool],
    *arguments: Any,
) -> Any:
    return invoke(resolve(loader, artifact), dict(launch), *arguments)
