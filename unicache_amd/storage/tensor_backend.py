"""Dense cache compaction and physical materialisation (drop-in for
``unicache/storage/tensor_backend.py``).

``compact`` removes the tokens a keep mask drops from a packed multi-sample
dense cache; ``compact_and_materialize`` first turns PhysicalCacheRequests
into PackedKIVICache / GQAH2OCache segments (HIP pack, H2O select and gather)
and drops their tokens from the dense cache.  Row compaction runs as a HIP
mask scan plus row copies.

How a materialisation call is organised (own design; the reference builds
each sample's segments in turn with a host round trip per decision):

1. Host checks only: sample lengths, keep-mask shapes, request lengths,
   operator names and token spans.
2. Device work that needs no answer yet, queued in one pass: per-sample claim
   counts of the request masks (an overlap is a count above one), the keep
   masks with the claimed tokens cleared, the token count of every request
   given by mask only, the type-id bounds of every request whose type must be
   recovered, and the kept count of every sample.  All of these scalars land
   in one int64 vector.
3. One host read of that vector.  Errors are raised before any segment is
   built or any keep mask is touched.
4. Segments are built with known sizes: a request with a token span uses
   views of its rows; a request with a mask only is gathered by one mask scan
   and row copies.  The dense remainder is compacted with the kept totals
   already known, so it costs no further synchronisation.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from .. import _native as nat
from ..core.decisions import PhysicalCacheRequest
from .physical import GQAH2OCache, PackedKIVICache


# ------------------------------------------------------------ row kernels --
def _aligned_mask(keep: torch.Tensor, device: torch.device) -> torch.Tensor:
    mask = keep.to(device=device, dtype=torch.bool).contiguous()
    return mask.clone() if mask.data_ptr() % 16 else mask


def _scan(mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(dst [n] int32: destination row of each kept row or -1, total [1] int64
    on the device) of a 16-byte-aligned bool mask."""

    n = int(mask.numel())
    dst = torch.empty(n, dtype=torch.int32, device=mask.device)
    total = torch.empty(1, dtype=torch.int64, device=mask.device)  # the scan always writes it
    nat.call("uc_mask_scan", mask.data_ptr(), n, dst.data_ptr(), total.data_ptr(), nat.stream(mask.device))
    return dst, total


def _copy_rows(src: torch.Tensor, dst: torch.Tensor, kept: int) -> torch.Tensor:
    """The rows of src (dim 0) whose dst entry is >= 0, in order; `kept` is
    their number."""

    n = int(dst.numel())
    if int(src.shape[0]) != n:
        raise ValueError("Keep mask does not match the cache token count")
    if n and not src[0].is_contiguous():
        src = src.contiguous()
    out = torch.empty((kept, *src.shape[1:]), dtype=src.dtype, device=dst.device)
    if kept:
        row_bytes = int(src[0].numel()) * src.element_size()
        nat.call("uc_compact_rows", src.data_ptr(), int(src.stride(0)) * src.element_size(), row_bytes,
                 dst.data_ptr(), n, out.data_ptr(), nat.stream(dst.device))
    return out


def _copy_rows_many(srcs: list[torch.Tensor | None], dst: torch.Tensor, kept: int) -> list[torch.Tensor | None]:
    """_copy_rows for several tensors through one uc_compact_rows_multi call
    (one launch for the 16-byte-aligned ones)."""

    n = int(dst.numel())
    outs: list[torch.Tensor | None] = []
    copies = []
    for src in srcs:
        if src is None:
            outs.append(None)
            continue
        if int(src.shape[0]) != n:
            raise ValueError("Keep mask does not match the cache token count")
        if n and not src[0].is_contiguous():
            src = src.contiguous()
        out = torch.empty((kept, *src.shape[1:]), dtype=src.dtype, device=dst.device)
        outs.append(out)
        if kept:
            copies.append(nat.RowCopy(src.data_ptr(), int(src.stride(0)) * src.element_size(),
                                      int(src[0].numel()) * src.element_size(), out.data_ptr()))
    if copies:
        nat.call("uc_compact_rows_multi", (nat.RowCopy * len(copies))(*copies), len(copies), dst.data_ptr(), n,
                 nat.stream(dst.device))
    return outs


def compact_rows(tensors: list[torch.Tensor | None], keep: torch.Tensor,
                 kept: int | None = None) -> list[torch.Tensor | None]:
    """tensor[keep] for every tensor (rows along dim 0), in order, on the HIP
    scan + copy kernels (tensor_backend.py:66-77).  With `kept` (the number
    of True entries) given, no host synchronisation is needed."""

    device = nat.require_device(keep, *[t for t in tensors if t is not None], what="Dense cache compaction")
    mask = _aligned_mask(keep, device)
    dst, total = _scan(mask)
    if kept is None:
        kept = int(total.item()) if mask.numel() else 0
    return _copy_rows_many(tensors, dst, int(kept))


# --------------------------------------------------------------- results --
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


# ------------------------------------------------------------ validation --
def _sample_lengths(sample_lens: torch.Tensor, sample_lengths: list[int] | None) -> list[int]:
    if sample_lengths is not None:
        return [int(x) for x in sample_lengths]
    return [int(x) for x in sample_lens.to("cpu").tolist()]


def _check_cache(key, value, key_type_ids, lengths, keep_masks) -> None:
    if key.shape != value.shape or key.dim() != 3:
        raise ValueError("Tensor cache backend expects matching [tokens, heads, head_dim] KV tensors")
    if sum(lengths) != int(key.shape[0]):
        raise ValueError("Packed sample lengths do not match the cache token count")
    if len(keep_masks) != len(lengths):
        raise ValueError("Tensor cache backend requires one keep mask per packed sample")
    if key_type_ids is not None and int(key_type_ids.numel()) != int(key.shape[0]):
        raise ValueError("key_type_ids do not match the cache token count")
    for length, keep_mask in zip(lengths, keep_masks):
        if keep_mask.dim() != 1 or int(keep_mask.numel()) != length:
            raise ValueError("Keep mask does not match its packed sample length")


def _span_of(request: PhysicalCacheRequest, length: int) -> tuple[int, int] | None:
    span = request.metadata.get("token_span")
    if span is None:
        return None
    if not isinstance(span, (tuple, list)) or len(span) != 2:
        raise ValueError("Physical token_span must be a (start, stop) pair")
    start, stop = int(span[0]), int(span[1])
    if not 0 <= start < stop <= length:
        raise ValueError("Physical token_span is outside its packed sample")
    return start, stop


_OPERATORS = ("kivi_packed_quantization", "h2o_physical_gqa")


@dataclass
class _Planned:
    """One request of one sample, after the host checks."""

    request: PhysicalCacheRequest
    mask: torch.Tensor               # bool [length] on the cache device
    span: tuple[int, int] | None
    type_id: int                     # < 0: recover from key_type_ids
    count_slot: int = -1             # summary index of the token count (mask-only requests)
    type_slot: int = -1              # summary index of (min, max) type id


class _Summary:
    """Device int64 scalars collected for one host read."""

    def __init__(self) -> None:
        self.values: list[torch.Tensor] = []

    def add(self, value: torch.Tensor) -> int:
        self.values.append(value.reshape(()).to(torch.int64))
        return len(self.values) - 1

    def read(self) -> list[int]:
        return [int(v) for v in torch.stack(self.values).tolist()] if self.values else []


# ------------------------------------------------------------ the backend --
class TensorCacheStorageBackend:
    """Compact a packed dense cache according to one keep mask per sample."""

    @staticmethod
    def _compact_known(key, value, key_type_ids, sample_lens, masks, kept_per_sample):
        """The compaction with the kept count of every sample known."""

        full = torch.cat(masks) if masks else torch.zeros(0, dtype=torch.bool, device=key.device)
        total = sum(kept_per_sample)
        same = key_type_ids is None or key_type_ids.device == key.device
        compacted_key, compacted_value, compacted_types = compact_rows(
            [key, value, key_type_ids if same else None], full, kept=total)
        if not same:  # type ids kept on another device are indexed there, as the reference does
            compacted_types = key_type_ids[full.to(key_type_ids.device)]
        compacted_lens = torch.tensor(kept_per_sample, dtype=sample_lens.dtype, device=sample_lens.device)
        return CacheMutationResult(
            key=compacted_key,
            value=compacted_value,
            key_type_ids=compacted_types,
            sample_lens=compacted_lens,
            original_bytes=int(key.numel() * key.element_size() + value.numel() * value.element_size()),
            compacted_bytes=int(compacted_key.numel() * compacted_key.element_size()
                                + compacted_value.numel() * compacted_value.element_size()),
        )

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
        """Keep, per packed sample, the rows its mask marks (tensor_backend.py:32-100)."""

        lengths = _sample_lengths(sample_lens, sample_lengths)
        _check_cache(key, value, key_type_ids, lengths, keep_masks)
        device = nat.require_device(key, value, what="Dense cache compaction")
        masks = [m.to(device=device, dtype=torch.bool) for m in keep_masks]
        if len(masks) != 1 or key_type_ids is not None and key_type_ids.device != device:
            summary = _Summary()
            slots = [summary.add(m.sum()) for m in masks]
            counts = summary.read()
            return TensorCacheStorageBackend._compact_known(key, value, key_type_ids, sample_lens, masks,
                                                            [counts[s] for s in slots])
        # one sample: the mask scan's own total is the kept count (one host
        # read) and, cast on the device, the new sample length
        mask = _aligned_mask(masks[0], device)
        dst, total = _scan(mask)
        kept = int(total.item()) if mask.numel() else 0
        compacted_key, compacted_value, compacted_types = _copy_rows_many([key, value, key_type_ids], dst, kept)
        return CacheMutationResult(
            key=compacted_key,
            value=compacted_value,
            key_type_ids=compacted_types,
            sample_lens=total.to(device=sample_lens.device, dtype=sample_lens.dtype),
            original_bytes=int(key.numel() * key.element_size() + value.numel() * value.element_size()),
            compacted_bytes=int(compacted_key.numel() * compacted_key.element_size()
                                + compacted_value.numel() * compacted_value.element_size()),
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
        tokens from the dense KV (tensor_backend.py:102-239).  Errors are
        raised before any keep mask is modified."""

        lengths = _sample_lengths(sample_lens, sample_lengths)
        if len(physical_requests) != len(lengths):
            raise ValueError("Physical requests require one list per packed sample")
        _check_cache(key, value, key_type_ids, lengths, keep_masks)
        device = nat.require_device(key, value, what="Physical cache materialisation")
        offsets = [0]
        for length in lengths:
            offsets.append(offsets[-1] + length)

        # 1. host checks
        planned: list[list[_Planned]] = []
        for length, requests in zip(lengths, physical_requests):
            rows = []
            for request in requests:
                if request.token_count < length:
                    raise ValueError("PhysicalCacheRequest is shorter than the persistent cache sample")
                span = _span_of(request, length)
                if request.operator not in _OPERATORS:
                    raise ValueError(f"Unknown physical cache request: {request.operator}")
                given = request.metadata.get("token_type_id")
                rows.append(_Planned(request, request.segment_mask[:length].to(device=device, dtype=torch.bool),
                                     span, int(given) if given is not None else -1))
            planned.append(rows)

        # 2. device work, one summary vector
        summary = _Summary()
        types = key_type_ids.to(device) if key_type_ids is not None else None
        overlap_slots, kept_slots, new_masks = [], [], []
        for s, rows in enumerate(planned):
            claims = torch.zeros(lengths[s], dtype=torch.int32, device=device)
            for row in rows:
                claims += row.mask
                if row.span is None:
                    row.count_slot = summary.add(row.mask.sum())
                if row.type_id < 0 and types is not None:
                    seg_types = types[offsets[s]:offsets[s + 1]]
                    if row.span is not None:
                        lo = seg_types[row.span[0]:row.span[1]].amin()
                        hi = seg_types[row.span[0]:row.span[1]].amax()
                    else:
                        big = torch.iinfo(torch.int64).max
                        wide = seg_types.to(torch.int64)
                        lo = torch.where(row.mask, wide, big).amin()
                        hi = torch.where(row.mask, wide, -big).amax()
                    row.type_slot = summary.add(lo)
                    summary.add(hi)
            overlap_slots.append(summary.add(claims.amax() > 1) if len(rows) > 1 else -1)
            keep = keep_masks[s].to(device=device, dtype=torch.bool) & (claims == 0)
            new_masks.append(keep)
            kept_slots.append(summary.add(keep.sum()))

        # 3. one host read; every error before any mutation
        vals = summary.read()
        for s, slot in enumerate(overlap_slots):
            if slot >= 0 and vals[slot]:
                raise ValueError(f"Overlapping physical requests in sample {s} are not allowed")
        for s, rows in enumerate(planned):
            for row in rows:
                if row.request.operator == "h2o_physical_gqa" and row.request.per_kv_head_scores is None and (
                        row.span is not None or vals[row.count_slot] > 0):
                    raise ValueError("Physical H2O request is missing per-KV-head scores")

        # 4. segments, then the dense remainder; the H2O segments of every
        # sample are selected and gathered together in one launch
        physical_by_sample: list[list[Any]] = []
        h2o_specs: list[dict] = []
        h2o_slots: list[tuple[int, int]] = []
        for s, rows in enumerate(planned):
            sample_key = key[offsets[s]:offsets[s + 1]]
            sample_value = value[offsets[s]:offsets[s + 1]]
            segments = []
            for row in rows:
                count = row.span[1] - row.span[0] if row.span is not None else vals[row.count_slot]
                if count == 0:
                    continue
                type_id = row.type_id
                if type_id < 0 and row.type_slot >= 0 and vals[row.type_slot] == vals[row.type_slot + 1]:
                    type_id = vals[row.type_slot]
                built = _build_segment(row, sample_key, sample_value, lengths[s], count, type_id)
                if isinstance(built, dict):  # an H2O segment, built below with the others
                    h2o_slots.append((s, len(segments)))
                    h2o_specs.append(built)
                    built = None
                segments.append(built)
            physical_by_sample.append(segments)
        if h2o_specs:
            for (s, j), cache in zip(h2o_slots, GQAH2OCache.from_dense_segments(h2o_specs)):
                physical_by_sample[s][j] = cache
        for s, keep in enumerate(new_masks):
            if keep_masks[s].device == keep.device and keep_masks[s].dtype == torch.bool:
                keep_masks[s].copy_(keep)
            else:
                keep_masks[s] = keep.to(keep_masks[s].device)
        mutation = TensorCacheStorageBackend._compact_known(key, value, key_type_ids, sample_lens, new_masks,
                                                            [vals[k] for k in kept_slots])
        mutation.physical_segments_by_sample = physical_by_sample
        return mutation


def _build_segment(row: _Planned, sample_key, sample_value, length: int, count: int, type_id: int):
    """The physical segment of one request: rows by view (token span) or by
    one mask scan and row copies, then the KIVI pack; for an H2O request the
    keyword arguments of its GQAH2OCache.from_dense, which the caller builds
    together with the call's other H2O segments."""

    request, device = row.request, sample_key.device
    scores = None
    if request.operator == "h2o_physical_gqa":
        scores = request.per_kv_head_scores[:, :length].to(device=device, dtype=torch.float32)
    if row.span is not None:
        start, stop = row.span
        dense_key, dense_value = sample_key[start:stop], sample_value[start:stop]
        logical_ids = torch.arange(start, stop, device=device, dtype=torch.int64)
        if scores is not None:
            scores = scores[:, start:stop]
    else:
        mask = _aligned_mask(row.mask, device)
        dst, _ = _scan(mask)
        positions = torch.arange(length, device=device, dtype=torch.int64)
        dense_key, dense_value, logical_ids = _copy_rows_many([sample_key, sample_value, positions], dst, count)
        if scores is not None:
            scores = _copy_rows(scores.t(), dst, count).t()
    params = request.params
    if request.operator == "kivi_packed_quantization":
        bits = int(params.get("bits", 4))
        return PackedKIVICache.from_dense(
            dense_key, dense_value, logical_token_ids=logical_ids, token_type_id=type_id,
            k_bits=int(params.get("k_bits", bits)), v_bits=int(params.get("v_bits", bits)),
            group_size=int(params.get("group_size", 64)),
            residual_length=int(params.get("residual_length", 32)),
            backend=str(params.get("backend", "reference")),
        )
    target, recent = h2o_budget(count, params)
    # GQAH2OCache.from_dense's arguments (physical.py:493-547): the caller
    # builds every H2O segment of the call with one from_dense_segments
    return dict(key=dense_key, value=dense_value, logical_token_ids=logical_ids, token_type_id=type_id,
                per_kv_head_scores=scores, target_tokens=target, recent_tokens=recent,
                selection_frozen=bool(params.get("selection_frozen", False)))
