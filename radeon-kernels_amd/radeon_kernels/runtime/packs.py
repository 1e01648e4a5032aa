"""Kernel-pack discovery and resolution.

Reference interface: src/radeon_kernels/runtime/packs.py:20-147.

Roots, in order: the ``RADEON_KERNELS_PACK_PATH`` entries (``os.pathsep`` separated), the user data
directory, the interpreter prefix and, last, the in-tree pack directory the build writes
(``radeon-kernels_amd/packs``) -- that one is this build's addition, so a source checkout finds its
own gfx950 pack without installing it.  A root is a pack itself (it holds ``manifest.json``) or a
directory of packs.

Discovery is total: a pack that cannot be read or verified is recorded in ``rejected`` with its
reason, never raised.  Signatures are required by default (reference packs.py:88-113): a pack's
``manifest.json`` must carry a ``manifest.sig.json`` that verifies under the trusted keyring (the
built-in release keyring, plus the development keyring an opt-in environment variable names,
unless a keyring is given).

Accepted packs are indexed by (environment key, operator, semantic version).  Resolution looks up
the caller's key and then needs a pack whose required features the fingerprint has and whose
artifact record and evidence id equal the approved dispatch entry's exactly.
"""

from __future__ import annotations

import os
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, Mapping, Sequence

from radeon_kernels.errors import RadeonKernelsError
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint, EnvironmentKey
from radeon_kernels.runtime.pack import KernelPack, KernelPackArtifact
from radeon_kernels.runtime.registry import ArtifactSpec
from radeon_kernels.runtime.signing import (
    TrustedKeyring,
    default_trusted_keyring,
    verify_detached_file,
)

PACK_PATH_ENVIRONMENT_VARIABLE = "RADEON_KERNELS_PACK_PATH"
IN_TREE_PACK_ROOT = Path(__file__).resolve().parents[2] / "packs"


class PackResolutionError(RadeonKernelsError):
    """No discovered pack can satisfy an approved dispatch entry."""


@dataclass(frozen=True)
class ResolvedKernelPack:
    pack: KernelPack
    artifact: KernelPackArtifact


def default_pack_roots(
    *,
    environ: Mapping[str, str] | None = None,
    home: Path | None = None,
    prefix: Path | None = None,
    include_in_tree: bool = True,
) -> tuple[Path, ...]:
    listed = (os.environ if environ is None else environ).get(PACK_PATH_ENVIRONMENT_VARIABLE, "")
    roots = [Path(item).expanduser() for item in listed.split(os.pathsep) if item]
    roots += [(home or Path.home()) / ".local" / "share" / "radeon-kernels" / "packs",
              (prefix or Path(sys.prefix)) / "share" / "radeon-kernels" / "packs"]
    if include_in_tree:
        roots.append(IN_TREE_PACK_ROOT)
    return tuple(dict.fromkeys(root.absolute() for root in roots))  # first occurrence wins


def pack_directories(roots: Iterable[Path]) -> tuple[Path, ...]:
    """Every pack directory under ``roots``, resolved, in root order and without repeats."""

    def packs_in(root: Path) -> list[Path]:
        if (root / "manifest.json").is_file():
            return [root]
        if root.is_dir():
            return [child for child in sorted(root.iterdir()) if (child / "manifest.json").is_file()]
        return []

    found = (child.resolve() for root in roots for child in packs_in(Path(root).expanduser()))
    return tuple(dict.fromkeys(found))


class KernelPackRegistry:
    def __init__(self, packs: Sequence[KernelPack] = (), *, rejected: Sequence[str] = ()) -> None:
        self._packs = tuple(packs)
        self._rejected = tuple(rejected)
        self._index: dict[tuple[EnvironmentKey, str, str], list[tuple[KernelPack, KernelPackArtifact]]] = {}
        for pack in self._packs:
            for item in pack.artifacts:
                slot = (pack.environment.key, item.operator, item.semantic_version)
                self._index.setdefault(slot, []).append((pack, item))

    @classmethod
    def discover(
        cls,
        roots: Iterable[Path],
        *,
        require_signatures: bool = True,
        trusted_keys: TrustedKeyring | None = None,
    ) -> KernelPackRegistry:
        keyring = trusted_keys
        if require_signatures and keyring is None:
            keyring = default_trusted_keyring()
        packs, rejected = [], []
        for directory in pack_directories(roots):
            try:
                if require_signatures:
                    verify_detached_file(directory / "manifest.json", directory / "manifest.sig.json", keyring,
                                         signed_file="manifest.json")
                packs.append(KernelPack.from_directory(directory, verify_artifacts=False))
            except RadeonKernelsError as error:  # a malformed manifest or a failed signature
                rejected.append(f"{directory}: {error}")
        return cls(packs, rejected=rejected)

    @property
    def packs(self) -> tuple[KernelPack, ...]:
        return self._packs

    @property
    def rejected(self) -> tuple[str, ...]:
        return self._rejected

    def resolve(
        self,
        *,
        fingerprint: EnvironmentFingerprint,
        operator: str,
        semantic_version: str,
        artifact: ArtifactSpec,
        evidence_id: str,
    ) -> ResolvedKernelPack:
        for pack, item in self._index.get((fingerprint.key, operator, semantic_version), ()):
            if pack.matches(fingerprint) and item.artifact == artifact and item.evidence_id == evidence_id:
                return ResolvedKernelPack(pack=pack, artifact=item)
        ignored = f"; {len(self._rejected)} invalid pack(s) were ignored" if self._rejected else ""
        raise PackResolutionError(f"no installed kernel pack matches {operator} {semantic_version}, "
                                  f"{fingerprint.architecture}, ROCm {fingerprint.rocm_abi}{ignored}")
