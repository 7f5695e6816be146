"""Validation error type and the canonical JSON digest used by the sampling API.

Behaviour follows the reference's src/deepseekrpc/jsonutil.py:9-53 where the
sampling path touches it: one ``ValidationError(ValueError)`` for every
rejected input, sorted compact canonical JSON and its SHA-256 fingerprint
(the decision digest), and the exact-``int`` range check.
"""
from __future__ import annotations

import hashlib
import json


class ValidationError(ValueError):
    """Every input the sampling path rejects raises this type."""


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
