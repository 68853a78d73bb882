"""The minimum of UniCache's plugin interfaces the physical operators use
(``unicache.core``): base classes and the physical request record."""

from .capabilities import CapabilityDescriptor
from .decisions import PhysicalCacheRequest
from .registry import OperatorExecutionContext, ProcessingOperator

__all__ = ["CapabilityDescriptor", "OperatorExecutionContext", "PhysicalCacheRequest", "ProcessingOperator"]
