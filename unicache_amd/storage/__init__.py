"""Physical storage of the UniCache engine on MI355X (drop-in for
``unicache.storage``'s physical layouts and tensor backend)."""

from .physical import (
    GQAH2OCache,
    PackedKIVICache,
    PhysicalLayerCache,
    PhysicalSegment,
    gqa_probability_value,
    gqa_query_key_logits,
    tensor_bytes,
)
from .tensor_backend import CacheMutationResult, TensorCacheStorageBackend

__all__ = [
    "CacheMutationResult",
    "TensorCacheStorageBackend",
    "GQAH2OCache",
    "PackedKIVICache",
    "PhysicalLayerCache",
    "PhysicalSegment",
    "gqa_probability_value",
    "gqa_query_key_logits",
    "tensor_bytes",
]
