"""Processing-operator base class and its execution context: the subset of
unicache/core/registry.py:28-131 the physical operators rely on."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

from .capabilities import CapabilityDescriptor
from .decisions import PhysicalCacheRequest


class ProcessingOperator:
    name: str = ""
    family: str = "generic"
    stages: set[str] = {"attention"}
    executable: bool = False
    capabilities: CapabilityDescriptor | None = None
    uses_final_attention: bool = False
    preserves_attention_dispatch: bool = False

    def capability_descriptor(self) -> CapabilityDescriptor:
        if self.capabilities is not None:
            return self.capabilities
        return CapabilityDescriptor(stages=frozenset(self.stages))

    def build_params(self, params: dict[str, Any]) -> dict[str, Any]:
        return dict(params)

    def execute(self, ctx: "OperatorExecutionContext") -> "OperatorExecutionContext":
        raise NotImplementedError(f"Operator {self.name} has no executable runtime implementation")

    def update_after_attention(self, ctx: "OperatorExecutionContext", attention_probs: Any) -> "OperatorExecutionContext":
        del attention_probs
        return ctx


@dataclass
class OperatorExecutionContext:
    """Tensor and runtime state handed to an operator.  ``runtime`` needs a
    ``kv_metadata`` dict and ``step`` a ``segment_id``."""

    runtime: Any
    step: Any
    params: dict[str, Any]
    q: Any
    k: Any
    v: Any
    attn_mask: Any
    key_type_ids: Any
    segment_mask: Any
    protected_mask: Any
    state: dict[Any, Any]
    record: Callable[[dict[str, float]], None]
    set_storage_snapshot: Callable[[dict[str, float]], None]
    metadata_state: dict[Any, Any] | None = None
    storage_num_kv_heads: int | None = None
    attention_probs: Any = None
    attention_prob_sources: Any = None
    attention_probs_override: Any = None
    attention_output: Any = None
    storage: Any = None
    decision: Any = None
    physical_request: PhysicalCacheRequest | None = None
    attention_keep_mask_override: Any = None
    extras: dict[str, Any] = field(default_factory=dict)
