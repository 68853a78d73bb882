"""Dense cache compaction and physical materialisation (drop-in for
``unicache/storage/tensor_backend.py``).

compact_and_materialize turns PhysicalCacheRequests into PackedKIVICache /
GQAH2OCache segments (HIP pack, H2O select and gather) and removes the
materialised tokens from the dense cache.  The keep-mask row compaction of
the remaining dense tokens runs as a HIP mask scan plus row copies.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from .. import _native as nat
from ..core.decisions import PhysicalCacheRequest
from .physical import GQAH2OCache, PackedKIVICache


def compact_rows(tensors: list[torch.Tensor | None], keep: torch.Tensor) -> list[torch.Tensor | None]:
    """tensor[keep] for every tensor (rows along dim 0, each row contiguous),
    in order, on the HIP scan + copy kernels (tensor_backend.py:66-77)."""

    device = nat.require_device(keep, *[t for t in tensors if t is not None], what="Dense cache compaction")
    n = int(keep.numel())
    mask = keep.to(device=device, dtype=torch.bool).contiguous()
    if mask.data_ptr() % 16:
        mask = mask.clone()
    dst = torch.empty(n, dtype=torch.int32, device=device)
    total = torch.zeros(1, dtype=torch.int64, device=device)
    stream = nat.stream(device)
    nat.call("uc_mask_scan", mask.data_ptr(), n, dst.data_ptr(), total.data_ptr(), stream)
    kept = int(total.item()) if n else 0
    out: list[torch.Tensor | None] = []
    for t in tensors:
        if t is None:
            out.append(None)
            continue
        if int(t.shape[0]) != n:
            raise ValueError("Keep mask does not match the cache token count")
        row = t[0] if n else t.new_empty(t.shape[1:])
        if n and not row.is_contiguous():
            t = t.contiguous()
        row_bytes = int(row.numel() * t.element_size())
        res = torch.empty((kept, *t.shape[1:]), dtype=t.dtype, device=device)
        if kept:
            nat.call("uc_compact_rows", t.data_ptr(), int(t.stride(0)) * t.element_size(), row_bytes,
                     dst.data_ptr(), n, res.data_ptr(), stream)
        out.append(res)
    return out


@dataclass
class CacheMutationResult:
    key: torch.Tensor
    value: torch.Tensor
    key_type_ids: torch.Tensor | None
    sample_lens: torch.Tensor
    original_bytes: int
    compacted_bytes: int
    physical_segments_by_sample: list[list[Any]] | None = None

    @property
    def bytes_saved(self) -> int:
        return self.original_bytes - self.compacted_bytes


def h2o_budget(segment_tokens: int, params: dict) -> tuple[int, int]:
    """(target, recent) of an H2O request (tensor_backend.py:199-210).
    Python's round() is round-half-to-even, as in UniCache."""

    target = params.get("budget", params.get("keep_k"))
    if target is None:
        ratio = float(params.get("target_budget_ratio", 1.0))
        target = max(1, int(round(int(segment_tokens) * ratio)))
    recent = params.get("recent_size")
    if recent is None:
        recent = int(round(int(target) * float(params.get("recent_budget_fraction", 0.25))))
    return int(target), int(recent)


class TensorCacheStorageBackend:
    """Compact a packed dense cache according to one keep mask per sample."""

    @staticmethod
    def compact(
        *,
        key: torch.Tensor,
        value: torch.Tensor,
        key_type_ids: torch.Tensor | None,
        sample_lens: torch.Tensor,
        keep_masks: list[torch.Tensor],
        sample_lengths: list[int] | None = None,
    ) -> CacheMutationResult:
        if key.shape != value.shape or key.dim() != 3:
            raise ValueError("Tensor cache backend expects matching [tokens, heads, head_dim] KV tensors")
        lengths = sample_lengths
        if lengths is None:
            lengths = [int(item) for item in sample_lens.to("cpu").tolist()]
        if sum(lengths) != int(key.shape[0]):
            raise ValueError("Packed sample lengths do not match the cache token count")
        if len(keep_masks) != len(lengths):
            raise ValueError("Tensor cache backend requires one keep mask per packed sample")
        if key_type_ids is not None and int(key_type_ids.numel()) != int(key.shape[0]):
            raise ValueError("key_type_ids do not match the cache token count")
        masks = []
        for length, keep_mask in zip(lengths, keep_masks):
            mask = keep_mask.to(device=key.device, dtype=torch.bool)
            if mask.dim() != 1 or int(mask.numel()) != length:
                raise ValueError("Keep mask does not match its packed sample length")
            masks.append(mask)
        full = torch.cat(masks) if masks else torch.zeros(0, dtype=torch.bool, device=key.device)
        same = key_type_ids is None or key_type_ids.device == key.device
        compacted_key, compacted_value, compacted_types = compact_rows(
            [key, value, key_type_ids if same else None], full)
        if not same:  # type ids kept on another device are indexed there, as the reference does
            compacted_types = key_type_ids[full.to(key_type_ids.device)]
        original_bytes = int(key.numel() * key.element_size() + value.numel() * value.element_size())
        compacted_bytes = int(
            compacted_key.numel() * compacted_key.element_size()
            + compacted_value.numel() * compacted_value.element_size()
        )
        compacted_lens = (
            torch.stack([m.sum(dtype=sample_lens.dtype) for m in masks]).to(
                device=sample_lens.device, dtype=sample_lens.dtype
            )
            if masks
            else sample_lens[:0]
        )
        return CacheMutationResult(
            key=compacted_key,
            value=compacted_value,
            key_type_ids=compacted_types,
            sample_lens=compacted_lens,
            original_bytes=original_bytes,
            compacted_bytes=compacted_bytes,
        )

    @staticmethod
    def compact_and_materialize(
        *,
        key: torch.Tensor,
        value: torch.Tensor,
        key_type_ids: torch.Tensor | None,
        sample_lens: torch.Tensor,
        keep_masks: list[torch.Tensor],
        physical_requests: list[list[PhysicalCacheRequest]],
        sample_lengths: list[int] | None = None,
    ) -> CacheMutationResult:
        """Build the requested physical segments per sample and remove their
        tokens from the dense KV (tensor_backend.py:102-239)."""

        lengths = sample_lengths
        if lengths is None:
            lengths = [int(item) for item in sample_lens.to("cpu").tolist()]
        if len(physical_requests) != len(lengths):
            raise ValueError("Physical requests require one list per packed sample")
        physical_by_sample: list[list[Any]] = []
        offset = 0
        for sample_idx, (length, requests) in enumerate(zip(lengths, physical_requests)):
            sample_key = key[offset: offset + length]
            sample_value = value[offset: offset + length]
            occupied = torch.zeros(length, device=key.device, dtype=torch.bool)
            segments: list[Any] = []
            normalized = []
            for request in requests:
                if request.token_count < length:
                    raise ValueError("PhysicalCacheRequest is shorter than the persistent cache sample")
                normalized.append((request, request.segment_mask[:length].to(device=key.device, dtype=torch.bool)))
            if len(normalized) > 1:
                claims = torch.stack([m for _, m in normalized], dim=0).sum(dim=0)
                if bool((claims > 1).any()):
                    raise ValueError(f"Overlapping physical requests in sample {sample_idx} are not allowed")
            for request, segment_mask in normalized:
                occupied |= segment_mask
                token_span = request.metadata.get("token_span")
                segment_slice = None
                if token_span is not None:
                    if not isinstance(token_span, (tuple, list)) or len(token_span) != 2:
                        raise ValueError("Physical token_span must be a (start, stop) pair")
                    span_start, span_stop = map(int, token_span)
                    if not 0 <= span_start < span_stop <= length:
                        raise ValueError("Physical token_span is outside its packed sample")
                    segment_slice = slice(span_start, span_stop)
                    segment_idx = torch.arange(span_start, span_stop, device=key.device, dtype=torch.long)
                else:
                    segment_idx = torch.nonzero(segment_mask, as_tuple=False).flatten()
                    if int(segment_idx.numel()) == 0:
                        continue
                metadata_type_id = request.metadata.get("token_type_id")
                type_id = int(metadata_type_id) if metadata_type_id is not None else -1
                if type_id < 0 and key_type_ids is not None:
                    segment_types = torch.unique(key_type_ids[offset: offset + length][segment_idx])
                    if int(segment_types.numel()) == 1:
                        type_id = int(segment_types.item())
                logical_ids = segment_idx.to(dtype=torch.int64)
                if segment_slice is None:
                    dense_key = sample_key[segment_idx].contiguous()
                    dense_value = sample_value[segment_idx].contiguous()
                else:
                    dense_key = sample_key[segment_slice]
                    dense_value = sample_value[segment_slice]
                if request.operator == "kivi_packed_quantization":
                    bits = int(request.params.get("bits", 4))
                    segment = PackedKIVICache.from_dense(
                        dense_key,
                        dense_value,
                        logical_token_ids=logical_ids,
                        token_type_id=type_id,
                        k_bits=int(request.params.get("k_bits", bits)),
                        v_bits=int(request.params.get("v_bits", bits)),
                        group_size=int(request.params.get("group_size", 64)),
                        residual_length=int(request.params.get("residual_length", 32)),
                        backend=str(request.params.get("backend", "cuda")),
                    )
                elif request.operator == "h2o_physical_gqa":
                    scores = request.per_kv_head_scores
                    if scores is None:
                        raise ValueError("Physical H2O request is missing per-KV-head scores")
                    scores = scores[:, :length].to(device=key.device, dtype=torch.float32)
                    segment_scores = scores[:, segment_idx]
                    target, recent = h2o_budget(int(segment_idx.numel()), request.params)
                    segment = GQAH2OCache.from_dense(
                        dense_key,
                        dense_value,
                        logical_token_ids=logical_ids,
                        token_type_id=type_id,
                        per_kv_head_scores=segment_scores,
                        target_tokens=target,
                        recent_tokens=recent,
                        selection_frozen=bool(request.params.get("selection_frozen", False)),
                    )
                else:
                    raise ValueError(f"Unknown physical cache request: {request.operator}")
                segments.append(segment)
            keep_masks[sample_idx] &= ~occupied
            physical_by_sample.append(segments)
            offset += length

        mutation = TensorCacheStorageBackend.compact(
            key=key,
            value=value,
            key_type_ids=key_type_ids,
            sample_lens=sample_lens,
            keep_masks=keep_masks,
            sample_lengths=lengths,
        )
        mutation.physical_segments_by_sample = physical_by_sample
        return mutation
