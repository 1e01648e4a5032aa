"""A JSON-Schema (draft 2020-12) checker restricted to the keywords the reference's schemas use.

``jsonschema`` is not installed here.  This validator covers exactly the vocabulary of the
reference's schemas/*.schema.json: type, properties, required, additionalProperties,
propertyNames, minProperties, items, prefixItems, minItems, maxItems, uniqueItems, enum, const,
pattern, minLength, maxLength, minimum, maximum, exclusiveMinimum, oneOf and local ``$ref``
(``#/$defs/...``); ``format`` is annotation only, as in the draft's default.  An unknown keyword
raises, so a schema outside that vocabulary cannot pass silently.  The tests pin it by accepting
the reference's own signed records and rejecting planted violations of each keyword.
"""

from __future__ import annotations

import re
from typing import Any

_ANNOTATIONS = {"$schema", "$id", "$defs", "title", "description", "format"}
_TYPES = {
    "object": lambda v: isinstance(v, dict),
    "array": lambda v: isinstance(v, list),
    "string": lambda v: isinstance(v, str),
    "integer": lambda v: isinstance(v, int) and not isinstance(v, bool),
    "number": lambda v: isinstance(v, (int, float)) and not isinstance(v, bool),
    "boolean": lambda v: isinstance(v, bool),
    "null": lambda v: v is None,
}


def _resolve(root: dict, ref: str) -> dict:
    if not ref.startswith("#/"):
        raise ValueError(f"only local references are supported: {ref}")
    node: Any = root
    for part in ref[2:].split("/"):
        node = node[part]
    return node


def errors(instance: Any, schema: dict, root: dict | None = None, path: str = "$") -> list[str]:
    """All violations of ``schema`` by ``instance`` (empty when valid)."""

    root = schema if root is None else root
    found: list[str] = []
    for key, value in schema.items():
        if key in _ANNOTATIONS or key in ("properties", "additionalProperties"):
            continue
        if key == "$ref":
            found += errors(instance, _resolve(root, value), root, path)
        elif key == "type":
            kinds = value if isinstance(value, list) else [value]
            if not any(_TYPES[kind](instance) for kind in kinds):
                found.append(f"{path}: expected type {value}")
        elif key == "required":
            if isinstance(instance, dict):
                found += [f"{path}: missing {name!r}" for name in value if name not in instance]
        elif key == "propertyNames":
            if isinstance(instance, dict):
                for name in instance:
                    found += errors(name, value, root, f"{path}.<name {name!r}>")
        elif key == "minProperties":
            if isinstance(instance, dict) and len(instance) < value:
                found.append(f"{path}: fewer than {value} properties")
        elif key == "items":
            if isinstance(instance, list):
                start = len(schema.get("prefixItems", []))
                for index, item in enumerate(instance[start:], start):
                    found += errors(item, value, root, f"{path}[{index}]")
        elif key == "prefixItems":
            if isinstance(instance, list):
                for index, (item, sub) in enumerate(zip(instance, value)):
                    found += errors(item, sub, root, f"{path}[{index}]")
        elif key == "minItems":
            if isinstance(instance, list) and len(instance) < value:
                found.append(f"{path}: fewer than {value} items")
        elif key == "maxItems":
            if isinstance(instance, list) and len(instance) > value:
                found.append(f"{path}: more than {value} items")
        elif key == "uniqueItems":
            if value and isinstance(instance, list):
                seen = [repr(item) for item in instance]
                if len(set(seen)) != len(seen):
                    found.append(f"{path}: items are not unique")
        elif key == "enum":
            if not any(instance == option and type(instance) is type(option) for option in value):
                found.append(f"{path}: {instance!r} not in {value}")
        elif key == "const":
            if not (instance == value and type(instance) is type(value)):
                found.append(f"{path}: expected {value!r}")
        elif key == "pattern":
            if isinstance(instance, str) and re.search(value, instance) is None:
                found.append(f"{path}: {instance!r} does not match {value}")
        elif key == "minLength":
            if isinstance(instance, str) and len(instance) < value:
                found.append(f"{path}: shorter than {value}")
        elif key == "maxLength":
            if isinstance(instance, str) and len(instance) > value:
                found.append(f"{path}: longer than {value}")
        elif key == "minimum":
            if _TYPES["number"](instance) and instance < value:
                found.append(f"{path}: below {value}")
        elif key == "maximum":
            if _TYPES["number"](instance) and instance > value:
                found.append(f"{path}: above {value}")
        elif key == "exclusiveMinimum":
            if _TYPES["number"](instance) and instance <= value:
                found.append(f"{path}: not above {value}")
        elif key == "oneOf":
            matches = sum(not errors(instance, option, root, path) for option in value)
            if matches != 1:
                found.append(f"{path}: matches {matches} of the oneOf alternatives")
        else:
            raise ValueError(f"unsupported schema keyword {key!r}")
    if isinstance(instance, dict):
        properties = schema.get("properties", {})
        extra = schema.get("additionalProperties", True)
        for name, item in instance.items():
            if name in properties:
                found += errors(item, properties[name], root, f"{path}.{name}")
            elif extra is False:
                found.append(f"{path}: unexpected property {name!r}")
            elif isinstance(extra, dict):
                found += errors(item, extra, root, f"{path}.{name}")
    return found
