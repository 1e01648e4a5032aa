"""Per-context record of the last dispatch decision.

Interface of src/radeon_kernels/runtime/explain.py:8-46 in the reference: the record lives in a
ContextVar (one per thread / async task) and ``explain_last_dispatch()`` renders seven lines --
operator, architecture, selected, artifact, evidence, fallbacks (joined by " -> ") and reason.
Records are copied on the way in and out, so callers cannot mutate the stored decision (a caller
that builds a fresh record for the purpose hands it over with ``owned=True`` and skips the inbound
copy; the reference deep-copies twice per dispatch).
"""

from __future__ import annotations

from contextvars import ContextVar
from copy import deepcopy
from typing import Any, Mapping

_LAST: ContextVar[dict[str, Any] | None] = ContextVar("radeon_kernels_last_dispatch", default=None)


def record_dispatch(value: Mapping[str, Any], *, owned: bool = False) -> None:
    """Store ``value`` as this context's last decision.

    ``owned=True`` promises that ``value`` is a dict built for this call whose nested containers
    nobody else holds, so it is stored without a copy.
    """

    _LAST.set(value if owned and type(value) is dict else deepcopy(dict(value)))


def get_last_dispatch() -> dict[str, Any] | None:
    value = _LAST.get()
    return None if value is None else deepcopy(value)


def clear_last_dispatch() -> None:
    _LAST.set(None)


def explain_last_dispatch() -> str:
    record = _LAST.get()
    if record is None:
        return "No Radeon kernel dispatch has been performed in this context."
    fallbacks = record.get("fallbacks") or []
    lines = (
        ("operator", record["operator"]),
        ("architecture", record["architecture"]),
        ("selected", record.get("selected") or "none"),
        ("artifact", record.get("artifact") or "none"),
        ("evidence", record.get("evidence_id") or "none"),
        ("fallbacks", " -> ".join(fallbacks) if fallbacks else "none"),
        ("reason", record["reason"]),
    )
    return "\n".join(f"{name}: {value}" for name, value in lines)
