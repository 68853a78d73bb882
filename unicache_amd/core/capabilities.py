"""Operator capability record (fields of unicache/core/capabilities.py:11-34)."""

from __future__ import annotations

from dataclasses import dataclass

WILDCARD_CAPABILITY = "*"


@dataclass(frozen=True)
class CapabilityDescriptor:
    stages: frozenset[str] = frozenset({WILDCARD_CAPABILITY})
    phases: frozenset[str] = frozenset({WILDCARD_CAPABILITY})
    devices: frozenset[str] = frozenset({WILDCARD_CAPABILITY})
    layouts: frozenset[str] = frozenset({WILDCARD_CAPABILITY})
    requires: frozenset[str] = frozenset()
    produces_selection: bool = False
    stateful: bool = False
    mutation_scope: str = "none"
    physical_storage_mutation: bool = False
    accepts_quantized_input: bool = False
