"""Shared static-dispatch executor for operators with a native winner and a torch fallback.

Behaviour of src/radeon_kernels/ops/_runtime.py:46-198 in the reference:

1. fingerprint the device (cached per device index);
2. select the dispatch entry (or the manifest's default fallbacks);
3. for a matched entry, resolve its pack, load the winner and call it with the entry's launch
   parameters; the decision is recorded as ``selected = "native/<entrypoint>"``;
4. if the winner cannot run (pack missing, artifact digest mismatch, provider error, or the
   entrypoint raising RuntimeError / TypeError / ValueError), demote to the declared ``torch``
   fallback and record ``"<reason>; winner unavailable: <error>; executed declared torch fallback"``;
5. with no usable fallback, record ``selected = "none"`` and raise OperatorDispatchError.

In addition to the reference, a demotion of a matched winner emits a NativeDemotionWarning so a
missing or broken native library never goes unnoticed, and ``strict_native=True`` turns such a
demotion into an error (used by acceptance checks that must prove the native path ran).

Call plans.  Steps 1-3 depend only on metadata the operator validated (dtypes, shapes, devices,
contiguity, autograd flags, scale) and on state that never changes once the runtime exists (the
dispatch manifests, the discovered packs, the loaded artifacts, the per-device fingerprint).  An
operator may therefore pass ``plan_key`` -- an exact, hashable description of everything its
validation and signature read from the call -- and after a successful native call the runtime keeps
the resolved entrypoint, its launch parameters and the explain record under that key.  A later call
with an equal key finds it through ``plan_for`` and ``run_plan`` calls the winner directly and stores
the same record.  Any error still demotes exactly as in step 4; a key never seen (or dropped when the table
is full) takes the full path.
"""

from __future__ import annotations

import warnings
from pathlib import Path
from threading import Lock
from typing import Any, Callable, Hashable, Iterable, Mapping

from radeon_kernels.errors import RadeonKernelsError
from radeon_kernels.providers import native
from radeon_kernels.runtime.dispatcher import DispatchDecision, DispatchRequest, Dispatcher
from radeon_kernels.runtime.explain import record_dispatch
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.loader import ArtifactError, PrecompiledArtifactLoader
from radeon_kernels.runtime.packs import KernelPackRegistry, PackResolutionError, default_pack_roots
from radeon_kernels.runtime.registry import DispatchRegistry
from radeon_kernels.runtime.resources import builtin_dispatch_registry

_DEMOTABLE = (
    PackResolutionError,
    ArtifactError,
    native.NativeProviderError,
    RuntimeError,
    TypeError,
    ValueError,
)


class OperatorDispatchError(RadeonKernelsError):
    """Neither a published winner nor the declared fallback can run."""


class NativeDemotionWarning(RuntimeWarning):
    """A matched native winner could not run and the declared fallback executed instead."""


def _record(decision: DispatchDecision, *, selected: str, artifact: str | None, evidence_id: str | None,
            reason: str) -> dict[str, Any]:
    record = decision.to_dict()
    record.update(selected=selected, artifact=artifact, evidence_id=evidence_id, reason=reason)
    record_dispatch(record, owned=True)
    return record


class _NativePlan:
    __slots__ = ("decision", "entrypoint", "launch", "record")

    def __init__(self, decision: DispatchDecision, entrypoint: Callable[..., Any], record: dict[str, Any]) -> None:
        self.decision = decision
        self.entrypoint = entrypoint
        self.launch = dict(decision.launch)
        self.record = record  # stored as the explain record of every planned call; never mutated


class OperatorRuntime:
    def __init__(
        self,
        *,
        registry: DispatchRegistry | None = None,
        pack_roots: Iterable[Path] | None = None,
        pack_registry: KernelPackRegistry | None = None,
        require_pack_signatures: bool = True,
        loader_factory: Callable[[Path], PrecompiledArtifactLoader] = PrecompiledArtifactLoader,
        fingerprint_detector: Callable[..., EnvironmentFingerprint] = EnvironmentFingerprint.detect,
        strict_native: bool = False,
    ) -> None:
        self._dispatcher = Dispatcher(registry if registry is not None else builtin_dispatch_registry())
        if pack_registry is None:
            roots = tuple(pack_roots) if pack_roots is not None else default_pack_roots()
            pack_registry = KernelPackRegistry.discover(roots, require_signatures=require_pack_signatures)
        self._packs = pack_registry
        self._loader_factory = loader_factory
        self._detect = fingerprint_detector
        self._strict = strict_native
        self._loaders: dict[Path, PrecompiledArtifactLoader] = {}
        self._fingerprints: dict[int, EnvironmentFingerprint] = {}
        self._plans: dict[Hashable, _NativePlan] = {}

    @property
    def pack_registry(self) -> KernelPackRegistry:
        return self._packs

    def fingerprint(self, torch_module: Any, device_index: int) -> EnvironmentFingerprint:
        cached = self._fingerprints.get(device_index)
        if cached is None:
            cached = self._detect(torch_module=torch_module, device_index=device_index)
            self._fingerprints[device_index] = cached
        return cached

    def _loader(self, root: Path) -> PrecompiledArtifactLoader:
        loader = self._loaders.get(root)
        if loader is None:
            loader = self._loaders.setdefault(root, self._loader_factory(root))
        return loader

    _PLAN_LIMIT = 1024

    def execute(
        self,
        *,
        operator: str,
        semantic_version: str,
        signature: Mapping[str, Any],
        device_index: int,
        torch_module: Any,
        native_arguments: tuple[Any, ...],
        fallback: Callable[[], Any],
        fallback_selected: str,
        plan_key: Hashable | None = None,
    ) -> Any:
        fingerprint = self.fingerprint(torch_module, device_index)
        decision = self._dispatcher.select(DispatchRequest(operator, semantic_version, signature), fingerprint,
                                           record=False)
        if not decision.matched:
            return self._run_fallback(decision, None, fallback, fallback_selected)
        winner = decision.winner
        try:
            resolved = self._packs.resolve(
                fingerprint=fingerprint,
                operator=decision.operator,
                semantic_version=decision.semantic_version,
                artifact=winner,
                evidence_id=decision.evidence_id,
            )
            entrypoint = native.resolve(self._loader(resolved.pack.root), winner)
            result = native.invoke(entrypoint, dict(decision.launch), *native_arguments)
        except _DEMOTABLE as error:
            return self._demote(decision, error, fallback, fallback_selected)
        record = _record(
            decision,
            selected=f"{winner.provider}/{winner.entrypoint}",
            artifact=winner.artifact,
            evidence_id=decision.evidence_id,
            reason=f"{decision.reason}; loaded pack {resolved.pack.pack_id} {resolved.pack.pack_version}",
        )
        if plan_key is not None:
            self._remember(plan_key, _NativePlan(decision, entrypoint, record))
        return result

    def plan_for(self, plan_key: Hashable | None) -> _NativePlan | None:
        """The plan kept for ``plan_key``, if a call with an equal key ran natively before."""

        if plan_key is None:
            return None
        try:
            return self._plans.get(plan_key)
        except TypeError:  # an unhashable component
            return None

    def run_plan(
        self,
        plan: _NativePlan,
        native_arguments: tuple[Any, ...],
        fallback: Callable[[], Any],
        fallback_selected: str,
    ) -> Any:
        """Call the planned winner; errors demote exactly as in ``execute``."""

        try:
            result = native.invoke(plan.entrypoint, plan.launch, *native_arguments)
        except _DEMOTABLE as error:
            return self._demote(plan.decision, error, fallback, fallback_selected)
        record_dispatch(plan.record, owned=True)
        return result

    def _remember(self, plan_key: Hashable, plan: _NativePlan) -> None:
        try:
            if plan_key not in self._plans and len(self._plans) >= self._PLAN_LIMIT:
                self._plans.clear()
            self._plans[plan_key] = plan
        except TypeError:
            pass

    def _demote(self, decision: DispatchDecision, error: Exception, fallback: Callable[[], Any],
                fallback_selected: str) -> Any:
        failure = str(error)
        winner = decision.winner
        if self._strict:
            _record(decision, selected="none", artifact=None, evidence_id=None,
                    reason=f"{decision.reason}; winner unavailable: {failure}; strict native mode")
            raise OperatorDispatchError(
                f"native winner for {decision.operator} {decision.semantic_version} failed: {failure}"
            ) from error
        warnings.warn(
            f"{decision.operator}: native winner {winner.entrypoint} unavailable ({failure}); "
            "running the declared fallback",
            NativeDemotionWarning,
            stacklevel=5,
        )
        return self._run_fallback(decision, failure, fallback, fallback_selected)

    def _run_fallback(self, decision: DispatchDecision, failure: str | None, fallback: Callable[[], Any],
                      fallback_selected: str) -> Any:
        reason = decision.reason if failure is None else f"{decision.reason}; winner unavailable: {failure}"
        if "torch" not in decision.fallbacks:
            _record(decision, selected="none", artifact=None, evidence_id=None,
                    reason=f"{reason}; no supported fallback is available")
            raise OperatorDispatchError(
                f"no approved implementation is available for {decision.operator} {decision.semantic_version}"
            )
        try:
            result = fallback()
        except Exception as error:
            _record(decision, selected="none", artifact=None, evidence_id=None, reason=f"torch fallback failed: {error}")
            raise
        _record(decision, selected=fallback_selected, artifact=None, evidence_id=None,
                reason=f"{reason}; executed declared torch fallback")
        return result


_DEFAULT: OperatorRuntime | None = None
_DEFAULT_LOCK = Lock()


def default_operator_runtime() -> OperatorRuntime:
    global _DEFAULT
    runtime = _DEFAULT
    if runtime is None:
        with _DEFAULT_LOCK:
            if _DEFAULT is None:
                _DEFAULT = OperatorRuntime()
            runtime = _DEFAULT
    return runtime


def reset_operator_runtime() -> None:
    global _DEFAULT
    with _DEFAULT_LOCK:
        _DEFAULT = None


__all__ = [
    "NativeDemotionWarning",
    "OperatorDispatchError",
    "OperatorRuntime",
    "default_operator_runtime",
    "reset_operator_runtime",
]
