"""Static dispatch: pick the highest-priority manifest entry matching (environment, signature).

Interface of src/radeon_kernels/runtime/dispatcher.py:11-100 in the reference.  Every selection,
matched or not, is written to the explain record (the operator runtime, which records the final
outcome of each call itself, asks for no intermediate record).  No search, tuning or compilation
happens here: an unmatched request gets the manifest's declared fallbacks.

Manifests are immutable once loaded and compiled into per-environment groups in priority order
(runtime/registry.py), so a decision walks only the caller's group and depends only on (operator,
version, fingerprint, signature); decisions are memoised on that key (the reference rescans every
entry per call).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Mapping

from radeon_kernels.runtime.explain import record_dispatch
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.registry import ArtifactSpec, DispatchRegistry


@dataclass(frozen=True)
class DispatchRequest:
    operator: str
    semantic_version: str
    signature: Mapping[str, Any]


@dataclass(frozen=True)
class DispatchDecision:
    operator: str
    semantic_version: str
    fingerprint: EnvironmentFingerprint
    entry_id: str | None
    winner: ArtifactSpec | None
    launch: Mapping[str, str | int | float | bool]
    fallbacks: tuple[str, ...]
    evidence_id: str | None
    reason: str

    @property
    def matched(self) -> bool:
        return self.winner is not None

    def to_dict(self) -> dict[str, Any]:
        winner = self.winner
        return {
            "operator": self.operator,
            "semantic_version": self.semantic_version,
            "architecture": self.fingerprint.architecture,
            "rocm_abi": self.fingerprint.rocm_abi,
            "python_abi": self.fingerprint.python_abi,
            "pytorch_version": self.fingerprint.pytorch_version,
            "entry_id": self.entry_id,
            "selected": None if winner is None else f"{winner.provider}/{winner.entrypoint}",
            "artifact": None if winner is None else winner.artifact,
            "launch": dict(self.launch),
            "fallbacks": list(self.fallbacks),
            "evidence_id": self.evidence_id,
            "reason": self.reason,
        }


class Dispatcher:
    _CACHE_LIMIT = 4096

    def __init__(self, registry: DispatchRegistry) -> None:
        self._registry = registry
        self._decisions: dict[Any, DispatchDecision] = {}

    def select(self, request: DispatchRequest, fingerprint: EnvironmentFingerprint, *,
               record: bool = True) -> DispatchDecision:
        try:
            key = (request.operator, request.semantic_version, fingerprint, tuple(request.signature.items()))
            decision = self._decisions.get(key)
        except TypeError:  # an unhashable signature value: decide without memoising
            key, decision = None, None
        if decision is None:
            decision = self._decide(request, fingerprint)
            if key is not None:
                if len(self._decisions) >= self._CACHE_LIMIT:
                    self._decisions.clear()
                self._decisions[key] = decision
        if record:
            record_dispatch(decision.to_dict(), owned=True)
        return decision

    def _decide(self, request: DispatchRequest, fingerprint: EnvironmentFingerprint) -> DispatchDecision:
        manifest = self._registry.get(request.operator, request.semantic_version)
        best = manifest.select(fingerprint, request.signature)
        if best is None:
            decision = DispatchDecision(
                operator=request.operator,
                semantic_version=request.semantic_version,
                fingerprint=fingerprint,
                entry_id=None,
                winner=None,
                launch={},
                fallbacks=manifest.default_fallbacks,
                evidence_id=None,
                reason="no compatible environment and workload region matched",
            )
        else:
            decision = DispatchDecision(
                operator=request.operator,
                semantic_version=request.semantic_version,
                fingerprint=fingerprint,
                entry_id=best.id,
                winner=best.winner,
                launch=best.launch,
                fallbacks=best.fallbacks,
                evidence_id=best.evidence_id,
                reason=f"matched dispatch entry {best.id!r} at priority {best.priority}",
            )
        return decision
