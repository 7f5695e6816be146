"""Validation error type and canonical JSON used by the sampling API.

Behaviour follows the reference's src/deepseekrpc/jsonutil.py:9-53: one
``ValidationError(ValueError)`` for every rejected input, strict bounded JSON
loading, sorted compact canonical JSON and its SHA-256 fingerprint, and the
exact-``int`` range check.
"""
from __future__ import annotations

import hashlib
import json
import math


class ValidationError(ValueError):
    """Every input the sampling path rejects raises this type."""


def _unique_pairs(items):
    seen = {}
    for key, value in items:
        if key in seen:
            raise ValidationError(f"duplicate JSON key: {key}")
        seen[key] = value
    return seen


def _reject_constant(_name):
    raise ValidationError("nonfinite JSON number")


def _finite_float(text):
    value = float(text)
    if not math.isfinite(value):
        raise ValidationError("JSON floating-point overflow")
    return value


def loads(data, *, limit: int):
    size = len(data.encode("utf-8")) if isinstance(data, str) else len(data)
    if size > limit:
        raise ValidationError("JSON byte limit exceeded")
    try:
        return json.loads(data, object_pairs_hook=_unique_pairs, parse_constant=_reject_constant,
                          parse_float=_finite_float)
    except (ValueError, UnicodeError, RecursionError) as exc:
        # Hook errors are ValueErrors too and are reported the same way.
        raise ValidationError("invalid or excessively nested JSON") from exc


def canonical(value) -> bytes:
    """Sorted keys, no whitespace, no NaN/inf: the bytes that are hashed."""
    return json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False).encode("utf-8")


def fingerprint(value) -> str:
    return hashlib.sha256(canonical(value)).hexdigest()


def integer(value, name: str, low: int, high: int) -> int:
    """An exact ``int`` (``bool`` and integral floats are rejected) in [low, high]."""
    if type(value) is not int or not low <= value <= high:
        raise ValidationError(f"{name} must be an integer in [{low}, {high}]")
    return value


def hex_id(value, size: int, name: str) -> str:
    """Lower-case hex identity of exactly ``size`` digits (reference protocol.py:57-60)."""
    if not isinstance(value, str) or len(value) != size or any(c not in "0123456789abcdef" for c in value):
        raise ValidationError(f"invalid {name} identity")
    return value
