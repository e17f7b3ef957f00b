"""A small JSON Schema (draft 2020-12) checker for the keywords the reference's
report schemas use: $ref (local), type, const, enum, required, properties,
additionalProperties (false), items, minItems, minLength, minimum, maximum,
pattern, oneOf, allOf, if/then; `format` is not checked. Test helper, not a
test module (jsonschema is not installed in this image)."""
from __future__ import annotations

import re
from typing import Any


def _type_ok(value: Any, t: str) -> bool:
    if t == "null":
        return value is None
    if t == "boolean":
        return isinstance(value, bool)
    if t == "integer":
        return isinstance(value, int) and not isinstance(value, bool)
    if t == "number":
        return isinstance(value, (int, float)) and not isinstance(value, bool)
    if t == "string":
        return isinstance(value, str)
    if t == "array":
        return isinstance(value, list)
    if t == "object":
        return isinstance(value, dict)
    raise ValueError(f"unknown type {t}")


def _same(value: Any, expected: Any) -> bool:
    """JSON equality: booleans never equal numbers."""
    if isinstance(value, bool) or isinstance(expected, bool):
        return type(value) is type(expected) and value == expected
    return value == expected


def _resolve(root: dict, ref: str) -> dict:
    assert ref.startswith("#/"), ref
    node = root
    for part in ref[2:].split("/"):
        node = node[part]
    return node


def errors(schema: dict, value: Any, root: dict | None = None, path: str = "$") -> list[str]:
    root = schema if root is None else root
    out: list[str] = []
    if "$ref" in schema:
        out += errors(_resolve(root, schema["$ref"]), value, root, path)
    if "type" in schema:
        types = schema["type"] if isinstance(schema["type"], list) else [schema["type"]]
        if not any(_type_ok(value, t) for t in types):
            return out + [f"{path}: {value!r} is not of type {types}"]
    if "const" in schema and not _same(value, schema["const"]):
        out.append(f"{path}: {value!r} != const {schema['const']!r}")
    if "enum" in schema and not any(_same(value, e) for e in schema["enum"]):
        out.append(f"{path}: {value!r} not in enum {schema['enum']}")
    if isinstance(value, (int, float)) and not isinstance(value, bool):
        if "minimum" in schema and value < schema["minimum"]:
            out.append(f"{path}: {value} < minimum {schema['minimum']}")
        if "maximum" in schema and value > schema["maximum"]:
            out.append(f"{path}: {value} > maximum {schema['maximum']}")
    if isinstance(value, str):
        if "minLength" in schema and len(value) < schema["minLength"]:
            out.append(f"{path}: string shorter than {schema['minLength']}")
        if "pattern" in schema and not re.search(schema["pattern"], value):
            out.append(f"{path}: {value!r} does not match {schema['pattern']}")
    if isinstance(value, dict):
        for key in schema.get("required", []):
            if key not in value:
                out.append(f"{path}: missing required {key}")
        props = schema.get("properties", {})
        for key, sub in props.items():
            if key in value:
                out += errors(sub, value[key], root, f"{path}.{key}")
        if schema.get("additionalProperties") is False:
            for key in value:
                if key not in props:
                    out.append(f"{path}: unexpected property {key}")
    if isinstance(value, list):
        if "minItems" in schema and len(value) < schema["minItems"]:
            out.append(f"{path}: fewer than {schema['minItems']} items")
        if isinstance(schema.get("items"), dict):
            for i, item in enumerate(value):
                out += errors(schema["items"], item, root, f"{path}[{i}]")
    for sub in schema.get("allOf", []):
        out += errors(sub, value, root, path)
    if "oneOf" in schema:
        passing = sum(1 for sub in schema["oneOf"] if not errors(sub, value, root, path))
        if passing != 1:
            out.append(f"{path}: {passing} oneOf branches match (expected exactly 1)")
    if "if" in schema and not errors(schema["if"], value, root, path) and "then" in schema:
        out += errors(schema["then"], value, root, path)
    return out
