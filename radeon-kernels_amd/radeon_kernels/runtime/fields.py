"""Typed readers for the strict JSON records of dispatch manifests and kernel packs.

A record is read against a declared field table: every key must be declared (``unknown fields``),
every required key present (``missing fields``), and each value goes through its reader, which
either returns the parsed value or raises ``ConfigError`` with the record path.  The document
formats are the reference's (schemas/dispatch.schema.json, schemas/kernel-pack.schema.json); the
messages are part of the contract the runtime tests pin.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from pathlib import PurePosixPath
from typing import Any, Callable, Mapping, Sequence

from radeon_kernels.errors import ConfigError

Reader = Callable[[Any, str], Any]

_IDENTIFIER = re.compile(r"[a-z][a-z0-9_.-]*")
_MAJOR_MINOR = re.compile(r"\d+\.\d+")
_SEMVER = re.compile(r"\d+\.\d+\.\d+")
_SHA256 = re.compile(r"[0-9a-f]{64}")


@dataclass(frozen=True)
class Field:
    name: str
    read: Reader
    required: bool = True
    default: Any = None


def mapping(value: Any, path: str) -> Mapping[str, Any]:
    if not isinstance(value, Mapping) or not all(isinstance(key, str) for key in value):
        raise ConfigError(path, "expected a mapping" if not isinstance(value, Mapping) else "keys must be strings")
    return value


def read_record(value: Any, fields: Sequence[Field], path: str) -> dict[str, Any]:
    """``{field name: parsed value}`` for a record declared by ``fields``."""

    raw = mapping(value, path)
    declared = {field.name: field for field in fields}
    unknown = sorted(key for key in raw if key not in declared)
    if unknown:
        raise ConfigError(path, f"unknown fields: {unknown}")
    missing = sorted(field.name for field in fields if field.required and field.name not in raw)
    if missing:
        raise ConfigError(path, f"missing fields: {missing}")
    return {name: (field.read(raw[name], f"{path}.{name}") if name in raw else field.default)
            for name, field in declared.items()}


def check_keys(raw: Mapping[str, Any], allowed: Sequence[str], required: Sequence[str], path: str) -> None:
    """The unknown / missing key checks of ``read_record`` on their own."""

    read_record(raw, [Field(name, lambda value, _path: value, name in required) for name in allowed], path)


def identifier(value: Any, path: str) -> str:
    if isinstance(value, str) and _IDENTIFIER.fullmatch(value):
        return value
    raise ConfigError(path, "expected a lowercase identifier")


def major_minor(value: Any, path: str) -> str:
    if isinstance(value, str) and _MAJOR_MINOR.fullmatch(value):
        return value
    raise ConfigError(path, "expected MAJOR.MINOR")


def pack_version(value: Any, path: str) -> str:
    if isinstance(value, str) and _SEMVER.fullmatch(value):
        return value
    raise ConfigError(path, "invalid version")


def scalar(value: Any, path: str) -> str | int | float | bool:
    if isinstance(value, (str, int, float, bool)):
        return value
    raise ConfigError(path, "expected a string, number or boolean")


def sha256(value: Any, path: str) -> str:
    if isinstance(value, str) and _SHA256.fullmatch(value):
        return value
    raise ConfigError(path, "expected a lowercase SHA-256")


def relative_path(value: Any, path: str) -> str:
    if not isinstance(value, str) or not value:
        raise ConfigError(path, "expected a relative path")
    pure = PurePosixPath(value)
    if pure.is_absolute() or ".." in pure.parts or pure.as_posix() != value:
        raise ConfigError(path, "must be a normalized relative path")
    return value


def code_identifier(value: Any, path: str) -> str:
    if isinstance(value, str) and value.isidentifier():
        return value
    raise ConfigError(path, "expected a Python/C identifier")


def non_negative_int(value: Any, path: str) -> int:
    if isinstance(value, int) and not isinstance(value, bool) and value >= 0:
        return value
    raise ConfigError(path, "expected a non-negative integer")


def one_of(*choices: str) -> Reader:
    def read(value: Any, path: str) -> str:
        if value in choices:
            return value
        raise ConfigError(path, f"expected {' or '.join(choices)}")

    return read


def identifier_list(*, non_empty: bool) -> Reader:
    """A list of distinct identifiers, as a tuple."""

    def read(value: Any, path: str) -> tuple[str, ...]:
        if not isinstance(value, list) or (non_empty and not value):
            raise ConfigError(path, "expected a non-empty list" if non_empty else "expected a list")
        items = tuple(identifier(item, path) for item in value)
        if len(set(items)) != len(items):
            raise ConfigError(path, "contains duplicates")
        return items

    return read


def scalar_mapping(value: Any, path: str) -> dict[str, str | int | float | bool]:
    """A mapping of identifier keys to scalars (an entry's launch parameters)."""

    out = {}
    for key, item in mapping(value, path).items():
        if not _IDENTIFIER.fullmatch(key):
            raise ConfigError(path, f"invalid parameter: {key!r}")
        out[key] = scalar(item, f"{path}.{key}")
    return out


def is_identifier(value: str) -> bool:
    return bool(_IDENTIFIER.fullmatch(value))
