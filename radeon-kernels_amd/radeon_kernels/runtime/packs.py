"""Kernel-pack discovery and resolution.

Interface of src/radeon_kernels/runtime/packs.py:20-147 in the reference: pack roots come from
``RADEON_KERNELS_PACK_PATH`` (os.pathsep separated), the user data directory and the interpreter
prefix; a root is either a pack itself (contains ``manifest.json``) or a directory of packs;
invalid packs are collected as ``rejected`` rather than raised; ``resolve`` needs a pack whose
environment matches the fingerprint and whose artifact record equals the dispatch winner exactly.

Signatures are required by default, as in the reference (packs.py:88-113): every pack's
``manifest.json`` must carry a ``manifest.sig.json`` that verifies under the trusted keyring
(radeon_kernels.runtime.signing; the built-in release keyring, plus the development keyring an
opt-in environment variable names, unless a keyring is given), else the pack is
rejected with the reason.

One deliberate difference: the in-tree pack directory written by the build
(``radeon-kernels_amd/packs``) is appended as the last default root, so a source checkout finds its
own gfx950 pack without installation.  The build signs that pack's manifest with its development key.
"""

from __future__ import annotations

import os
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, Mapping, Sequence

from radeon_kernels.errors import ConfigError, RadeonKernelsError
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.pack import KernelPack, KernelPackArtifact
from radeon_kernels.runtime.registry import ArtifactSpec
from radeon_kernels.runtime.signing import (
    SignatureVerificationError,
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
    environment = os.environ if environ is None else environ
    candidates = [Path(item).expanduser() for item in environment.get(PACK_PATH_ENVIRONMENT_VARIABLE, "").split(os.pathsep) if item]
    candidates.append((home or Path.home()) / ".local" / "share" / "radeon-kernels" / "packs")
    candidates.append((prefix or Path(sys.prefix)) / "share" / "radeon-kernels" / "packs")
    if include_in_tree:
        candidates.append(IN_TREE_PACK_ROOT)
    roots: list[Path] = []
    for candidate in candidates:
        absolute = candidate.absolute()
        if absolute not in roots:
            roots.append(absolute)
    return tuple(roots)


def pack_directories(roots: Iterable[Path]) -> tuple[Path, ...]:
    found: list[Path] = []
    for root in roots:
        root = Path(root).expanduser()
        if (root / "manifest.json").is_file():
            children: Sequence[Path] = (root,)
        elif root.is_dir():
            children = [child for child in sorted(root.iterdir()) if (child / "manifest.json").is_file()]
        else:
            children = ()
        for child in children:
            resolved = child.resolve()
            if resolved not in found:
                found.append(resolved)
    return tuple(found)


class KernelPackRegistry:
    def __init__(self, packs: Sequence[KernelPack] = (), *, rejected: Sequence[str] = ()) -> None:
        self._packs = tuple(packs)
        self._rejected = tuple(rejected)

    @classmethod
    def discover(
        cls,
        roots: Iterable[Path],
        *,
        require_signatures: bool = True,
        trusted_keys: TrustedKeyring | None = None,
    ) -> KernelPackRegistry:
        packs: list[KernelPack] = []
        rejected: list[str] = []
        keyring = trusted_keys
        if require_signatures and keyring is None:
            keyring = default_trusted_keyring()
        for directory in pack_directories(roots):
            try:
                if require_signatures:
                    verify_detached_file(directory / "manifest.json", directory / "manifest.sig.json", keyring,
                                         signed_file="manifest.json")
                packs.append(KernelPack.from_directory(directory, verify_artifacts=False))
            except (ConfigError, SignatureVerificationError, RadeonKernelsError) as error:
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
        for pack in self._packs:
            if not pack.matches(fingerprint):
                continue
            try:
                item = pack.get(operator, semantic_version)
            except ConfigError:
                continue
            if item.artifact == artifact and item.evidence_id == evidence_id:
                return ResolvedKernelPack(pack=pack, artifact=item)
        suffix = f"; {len(self._rejected)} invalid pack(s) were ignored" if self._rejected else ""
        raise PackResolutionError(
            f"no installed kernel pack matches {operator} {semantic_version}, "
            f"{fingerprint.architecture}, ROCm {fingerprint.rocm_abi}{suffix}"
        )
