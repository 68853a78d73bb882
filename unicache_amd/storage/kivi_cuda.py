"""GPU dispatch of the physical KIVI engine, on MI355X HIP kernels.

Drop-in for ``unicache/storage/kivi_cuda.py``: same function names, arguments,
return layouts and exceptions.  Where UniCache binds the pinned KIVI CUDA GEMV
and Triton kernels, these functions call libunicache_hip.so.  The engine fails
closed: a missing library raises RuntimeError, never a CPU or torch fallback.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import TYPE_CHECKING, Callable

import torch

from .. import _native as nat
from .physical import _pack_native, gqa_probability_value, gqa_query_key_logits  # noqa: F401

if TYPE_CHECKING:
    from .physical import PackedKIVICache


def select_kivi_kernel_backend(query_length: int) -> str:
    """GEMV for decode and a tiled kernel for multi-query attention
    (kivi_cuda.py:26-34).  The names are UniCache's; on MI355X "official_gemv"
    is the split-K decode kernel and "triton_tiled" the multi-query path."""

    requested = os.environ.get("UNICACHE_KIVI_MULTI_QUERY_BACKEND", "auto").lower()
    if requested not in {"auto", "official_gemv", "triton_tiled"}:
        raise ValueError(f"Unknown KIVI multi-query backend: {requested}")
    if requested != "auto":
        return requested
    return "official_gemv" if int(query_length) == 1 else "triton_tiled"


def _check_native(cache: "PackedKIVICache", what: str) -> None:
    if not cache.kernel_native_layout:
        raise RuntimeError(f"{what} requires kernel-native layout")


def dequantize_kivi_chunk(
    cache: "PackedKIVICache",
    *,
    start: int,
    stop: int,
    dtype: torch.dtype,
    output_key: torch.Tensor | None = None,
    output_value: torch.Tensor | None = None,
    output_offset: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Restore packed tokens [start, stop) without a full bf16 replica,
    optionally into caller workspaces (kivi_cuda.py:58-93; kivi_triton.py:690-770)."""

    start = max(0, int(start))
    stop = min(int(stop), int(cache.quantized_tokens))
    if stop <= start:
        empty = cache.residual_key[:0].to(dtype)
        return empty, empty
    if not cache.kernel_native_layout or cache.k_bits != cache.v_bits:
        raise RuntimeError("Chunked KIVI dequantization requires native equal-bit KV")
    token_count = stop - start
    kv_heads, d_size = int(cache.key_code.shape[0]), int(cache.key_code.shape[1])
    output_offset = int(output_offset)
    if output_key is None or output_value is None:
        if output_key is not None or output_value is not None:
            raise ValueError("Both KIVI output buffers must be provided together")
        output_offset = 0
        output_key = torch.empty((token_count, kv_heads, d_size), device=cache.key_code.device, dtype=dtype)
        output_value = torch.empty_like(output_key)
    if (
        output_key.dim() != 3
        or output_value.shape != output_key.shape
        or tuple(output_key.shape[1:]) != (kv_heads, d_size)
        or output_key.device != cache.key_code.device
        or output_value.device != cache.key_code.device
        or output_key.dtype != dtype
        or output_value.dtype != dtype
        or output_offset < 0
        or output_offset + token_count > int(output_key.shape[0])
    ):
        raise ValueError("KIVI dequantization output workspace has an invalid layout")
    if output_key.stride() != output_value.stride():
        raise ValueError("KIVI dequantization output workspace has an invalid layout")
    cache.dequantize_into(output_key, output_value, start=start, stop=stop, output_offset=output_offset)
    chunk = slice(output_offset, output_offset + token_count)
    return output_key[chunk], output_value[chunk]


def _decode_summary(cache: "PackedKIVICache", query: torch.Tensor, *, include_residual: bool,
                    out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused split-K attention over the packed prefix (and optionally the
    residual) for a short query: (out [Lq, Hq, D], lse [Hq, Lq])."""

    device = nat.require_device(query, cache.key_code, what="Packed KIVI attention")
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    tr = cache.residual_tokens if include_residual else 0
    out = torch.empty((lq, hq, d), dtype=out_dtype, device=device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=device)
    item = cache.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                             residual_key_ptr=nat.ptr(cache.residual_key) if tr else None,
                             residual_value_ptr=nat.ptr(cache.residual_value) if tr else None, residual_tokens=tr)
    ws_bytes = nat.decode_workspace_bytes(1, cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq,
                                          cache.quantized_tokens, tr)
    ws = nat.workspace(device, ws_bytes)
    res_dtype = cache.residual_key.dtype if tr else q.dtype
    nat.call(
        "uc_kivi_attn_decode", item, cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq,
        nat.dtype_code(q.dtype), nat.dtype_code(res_dtype), nat.dtype_code(out_dtype),
        1.0 / math.sqrt(d), ws.data_ptr(), ws_bytes, nat.stream(device),
    )
    return out, lse


def _mq_summary(cache: "PackedKIVICache", query: torch.Tensor, *, include_residual: bool,
                out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Long-query fused attention (uc_kivi_attn_mq): the tiled multi-query
    kernel that UniCache reaches through backend "triton_tiled"."""

    device = nat.require_device(query, cache.key_code, what="Packed KIVI attention")
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    tr = cache.residual_tokens if include_residual else 0
    out = torch.empty((lq, hq, d), dtype=out_dtype, device=device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=device)
    item = cache.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                             residual_key_ptr=nat.ptr(cache.residual_key) if tr else None,
                             residual_value_ptr=nat.ptr(cache.residual_value) if tr else None, residual_tokens=tr)
    res_dtype = cache.residual_key.dtype if tr else q.dtype
    nat.call(
        "uc_kivi_attn_mq", item, cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq,
        nat.dtype_code(q.dtype), nat.dtype_code(res_dtype), nat.dtype_code(out_dtype),
        1.0 / math.sqrt(d), None, 0, nat.stream(device),
    )
    return out, lse


def _max_decode_query_len(cache: "PackedKIVICache", heads_q: int) -> int:
    return max(1, 16 // max(1, heads_q // cache.num_kv_heads))


def _mq_supported(cache: "PackedKIVICache", head_dim: int, include_residual: bool) -> bool:
    res_ok = not include_residual or not cache.residual_tokens or cache.residual_key.dtype in (
        torch.bfloat16, torch.float16)
    return head_dim == 128 and cache.group_size in (32, 64, 128) and res_ok and (
        not include_residual or not cache.residual_tokens or cache.residual_key.is_contiguous())


def packed_kivi_attention_summary(
    cache: "PackedKIVICache", query: torch.Tensor, *, include_residual: bool = True
) -> tuple[torch.Tensor, torch.Tensor]:
    """Normalised output [Lq, Hq, D] and natural-log LSE [Hq, Lq] of softmax
    attention over the packed prefix plus (by default) the residual, in one
    fused dequant-attention pass.  With include_residual=False this is
    packed_kivi_quantized_attention_summary."""

    if not cache.quantized_tokens:
        raise ValueError("Packed KIVI summary requires a non-empty quantized prefix")
    if cache.k_bits != cache.v_bits or cache.k_bits not in {2, 4}:
        raise ValueError("Packed KIVI fused summary supports equal 2-bit or 4-bit KV")
    _check_native(cache, "Packed KIVI fused summary")
    if query.dim() != 3 or int(query.shape[1]) % cache.num_kv_heads:
        raise ValueError("Packed KIVI attention requires query heads divisible by KV heads")
    if query.dtype not in (torch.bfloat16, torch.float16):
        query = query.to(torch.bfloat16)
    lq = int(query.shape[0])
    step = _max_decode_query_len(cache, int(query.shape[1]))
    if lq <= step:
        return _decode_summary(cache, query, include_residual=include_residual, out_dtype=query.dtype)
    if _mq_supported(cache, int(query.shape[2]), include_residual):
        return _mq_summary(cache, query, include_residual=include_residual, out_dtype=query.dtype)
    from .kivi_mq import packed_attention_mq

    return packed_attention_mq(cache, query, include_residual=include_residual)


def packed_summary_with_dense(
    cache: "PackedKIVICache", query: torch.Tensor, dense_key: torch.Tensor, dense_value: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """One fused attention pass over [packed prefix of `cache` | dense keys]:
    the dense [T, Hkv, D] tokens take the place of the cache's residual.  This
    is the first chunk of _run_fused_mixed_attention with the bf16 segments
    folded in (adapters/bagel.py:1812-1826).  (out [Lq, Hq, D], lse [Hq, Lq])."""

    if not cache.quantized_tokens:
        raise ValueError("Packed KIVI summary requires a non-empty quantized prefix")
    if cache.k_bits != cache.v_bits or cache.k_bits not in {2, 4}:
        raise ValueError("Packed KIVI fused summary supports equal 2-bit or 4-bit KV")
    _check_native(cache, "Packed KIVI fused summary")
    if dense_key.shape != dense_value.shape or dense_key.dim() != 3 or int(dense_key.shape[1]) != cache.num_kv_heads:
        raise ValueError("Dense segments must be matching [tokens, kv_heads, head_dim] tensors")
    if query.dtype not in (torch.bfloat16, torch.float16):
        query = query.to(torch.bfloat16)
    device = nat.require_device(query, cache.key_code, dense_key, dense_value, what="Mixed-segment attention")
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    dk, dv = dense_key.contiguous(), dense_value.contiguous()
    tr = int(dk.shape[0])
    out = torch.empty((lq, hq, d), dtype=q.dtype, device=device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=device)
    item = cache.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                             residual_key_ptr=dk.data_ptr() if tr else None,
                             residual_value_ptr=dv.data_ptr() if tr else None, residual_tokens=tr)
    res_code = nat.dtype_code(dk.dtype if tr else q.dtype)
    if lq <= _max_decode_query_len(cache, hq):
        ws_bytes = nat.decode_workspace_bytes(1, cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq,
                                              cache.quantized_tokens, tr)
        entry = "uc_kivi_attn_decode"
    else:
        if d != 128 or cache.group_size not in (32, 64, 128) or (tr and dk.dtype not in (torch.bfloat16,
                                                                                        torch.float16)):
            raise ValueError("Mixed-segment attention needs head_dim 128, group 32/64/128 and 16-bit dense KV")
        ws_bytes = 0  # the multi-query kernel needs no workspace
        entry = "uc_kivi_attn_mq"
    ws = nat.workspace(device, ws_bytes) if ws_bytes else None
    nat.call(
        entry, item, cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq, nat.dtype_code(q.dtype),
        res_code, nat.dtype_code(q.dtype), 1.0 / math.sqrt(d), nat.ptr(ws), ws_bytes, nat.stream(device),
    )
    return out, lse


MQ_MAX_BATCH = 8  # segments per uc_kivi_attn_mq_batch launch


def packed_batch_with_dense(items: list) -> None:
    """packed_summary_with_dense for several independent segments in one
    attention launch per MQ_MAX_BATCH of them (uc_kivi_attn_mq_batch):
    the per-sample loop of apply_static_physical_attention_batch
    (adapters/bagel.py:773-980) for samples whose layout is one packed prefix
    plus dense keys.  items: (cache, query [Lq, Hq, D], key_parts, value_parts,
    out [Lq, Hq, D][, lse [Hq, Lq] fp32]) where the parts are lists (possibly
    empty) of [T_j, Hkv, D] tensors whose concatenation is the item's dense
    keys / values; every out (contiguous, the query dtype) and lse is written
    in place.  The dense parts of all items are
    gathered by one concatenation per launch.  All items share bits, group
    size, heads, the 16-bit query dtype and the dense dtype (that of the first
    key part), and take the multi-query path (Lq above the decode limit); the
    results equal packed_summary_with_dense bit for bit."""

    if not items:
        return
    cache0, q0 = items[0][0], items[0][1]
    dtype = next((x.dtype for item in items for x in item[2]), q0.dtype)
    hq, d = int(q0.shape[1]), int(q0.shape[2])
    if d != 128 or cache0.group_size not in (32, 64, 128) or cache0.k_bits not in (2, 4):
        raise ValueError("Batched packed attention needs head_dim 128, group 32/64/128 and 2/4-bit codes")
    if q0.dtype not in (torch.bfloat16, torch.float16) or dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("Batched packed attention needs 16-bit queries and dense keys")
    for cache, query, kparts, vparts, out, *rest in items:
        lse = rest[0] if rest else None
        if lse is not None and (lse.dtype != torch.float32 or tuple(lse.shape) != (hq, int(query.shape[0]))
                                or not lse.is_contiguous()):
            raise ValueError("Batched packed attention: lse must be contiguous fp32 [Hq, Lq]")
        if (cache.k_bits, cache.v_bits, cache.group_size, cache.num_kv_heads) != (
                cache0.k_bits, cache0.k_bits, cache0.group_size, cache0.num_kv_heads):
            raise ValueError("Batched packed attention needs equal bits, group size and KV heads")
        if not cache.quantized_tokens:
            raise ValueError("Packed KIVI summary requires a non-empty quantized prefix")
        _check_native(cache, "Batched packed attention")
        if query.dtype != q0.dtype or out.dtype != q0.dtype:
            raise ValueError("Batched packed attention needs one query dtype")
        if tuple(query.shape[1:]) != (hq, d) or out.shape != query.shape or len(kparts) != len(vparts) or any(
                x.shape != y.shape or x.dim() != 3 or tuple(x.shape[1:]) != (cache.num_kv_heads, d)
                for x, y in zip(kparts, vparts)):
            raise ValueError("Batched packed attention: inconsistent query, output or dense shapes")
        if not (query.is_contiguous() and out.is_contiguous()):
            raise ValueError("Batched packed attention needs contiguous queries and outputs")
        if int(query.shape[0]) <= _max_decode_query_len(cache, hq):
            raise ValueError("Batched packed attention covers multi-query segments only")
        cache.native_packed_pointers(query.device)
    # every pointer that goes into the launch table, on one GPU, checked before any launch
    device = nat.require_device(
        *(t for cache, query, kparts, vparts, out, *rest in items
          for t in (query, out, *rest, *kparts, *vparts, cache.key_code, cache.key_scale, cache.key_minimum,
                    cache.value_code, cache.value_scale, cache.value_minimum)),
        what="Batched packed attention")
    for start in range(0, len(items), MQ_MAX_BATCH):
        chunk = items[start:start + MQ_MAX_BATCH]
        kparts = [x.to(dtype) for item in chunk for x in item[2]]
        vparts = [x.to(dtype) for item in chunk for x in item[3]]
        dk = torch.cat(kparts, dim=0) if kparts else None
        dv = torch.cat(vparts, dim=0) if vparts else None
        row_bytes = int(dk.stride(0)) * dk.element_size() if dk is not None else 0
        table = (nat.KiviItem * len(chunk))()
        lens = (ctypes.c_int64 * len(chunk))()
        row = 0
        for j, (cache, query, kparts, _, out, *rest) in enumerate(chunk):
            lse = rest[0] if rest else None
            tr = sum(int(x.shape[0]) for x in kparts)
            table[j] = cache.native_item(
                query.data_ptr(), out.data_ptr(), lse.data_ptr() if lse is not None else None,
                residual_key_ptr=dk.data_ptr() + row * row_bytes if tr else None,
                residual_value_ptr=dv.data_ptr() + row * row_bytes if tr else None, residual_tokens=tr)
            row += tr
            lens[j] = int(query.shape[0])
        nat.call(
            "uc_kivi_attn_mq_batch", table, lens, len(chunk), cache0.k_bits, cache0.group_size, hq,
            cache0.num_kv_heads, d, nat.dtype_code(q0.dtype), nat.dtype_code(dtype), nat.dtype_code(q0.dtype),
            1.0 / math.sqrt(d), None, 0, nat.stream(device),
        )


MQ_MAX_PACKED, MQ_MAX_DENSE = 8, 16  # segments per uc_kivi_attn_mq_segments launch


def _dense_segment(key: torch.Tensor, value: torch.Tensor):
    """uc_dense_segment of [T, Hkv, D] key/value views read in place: unit
    channel stride, token and head strides that are multiples of 8 elements
    (the same for key and value), 16-byte aligned; other layouts are copied.
    Returns (struct, tensors to keep alive)."""

    def in_place(x):
        return x.stride(2) == 1 and x.stride(0) % 8 == 0 and x.stride(1) % 8 == 0 and x.data_ptr() % 16 == 0

    if not (in_place(key) and in_place(value) and key.stride() == value.stride()):
        key, value = key.contiguous(), value.contiguous()
    seg = nat.DenseSegment(key.data_ptr(), value.data_ptr(), int(key.shape[0]), int(key.stride(0)),
                           int(key.stride(1)))
    return seg, (key, value)


def packed_segments_supported(packed: list, query: torch.Tensor, dense: list) -> bool:
    """Whether packed_segments_summary takes this layout: long 16-bit queries,
    head_dim 128, packed prefixes of equal 2- or 4-bit K/V, one group size and
    KV head count, 16-bit dense parts, within the per-launch segment limits."""

    if not packed or query.dim() != 3 or int(query.shape[2]) != 128 or query.dtype not in (torch.bfloat16,
                                                                                             torch.float16):
        return False
    first = packed[0]
    if first.k_bits not in (2, 4) or first.group_size not in (32, 64, 128):
        return False
    if any((s.k_bits, s.v_bits, s.group_size, s.num_kv_heads) != (first.k_bits, first.k_bits, first.group_size,
                                                                  first.num_kv_heads) or not s.kernel_native_layout
           for s in packed):
        return False
    if int(query.shape[0]) <= _max_decode_query_len(first, int(query.shape[1])):
        return False
    parts = [k for k, _ in dense] + [s.residual_key for s in packed if s.residual_tokens]
    if any(x.dtype not in (torch.bfloat16, torch.float16) for x in parts):
        return False
    n_dense = sum(1 for k, _ in dense if int(k.shape[0])) + sum(1 for s in packed if s.residual_tokens)
    return len(packed) <= MQ_MAX_PACKED and n_dense <= MQ_MAX_DENSE


def packed_segments_summary(packed: list, query: torch.Tensor, dense: list,
                            *, dense_dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One softmax of query [Lq, Hq, 128] over the packed prefixes and
    residuals of the PackedKIVICache segments `packed` and the dense
    (key, value) [T, Hkv, 128] segments `dense`, in one launch of the
    multi-query kernel (uc_kivi_attn_mq_segments): no concatenation of the
    dense parts, no per-prefix summaries, no merge.  This is the long-query
    form of _run_fused_mixed_attention (adapters/bagel.py:1598-1858).  Dense
    parts and residuals are attended in `dense_dtype` (default: the first dense
    part's dtype).  Returns (out [Lq, Hq, 128] in the query dtype, lse [Hq, Lq])."""

    if not packed_segments_supported(packed, query, dense):
        raise ValueError("Segment-table attention needs long 16-bit queries, head_dim 128, packed prefixes of "
                         "equal 2/4-bit K/V sharing group size and KV heads, 16-bit dense parts and at most "
                         f"{MQ_MAX_PACKED} prefixes and {MQ_MAX_DENSE} dense parts")
    first = packed[0]
    hkv = first.num_kv_heads
    for key, value in dense:
        if key.shape != value.shape or key.dim() != 3 or tuple(key.shape[1:]) != (hkv, 128):
            raise ValueError("Dense segments must be matching [tokens, kv_heads, 128] tensors")
    for cache in packed:
        if not cache.quantized_tokens:
            raise ValueError("Packed segments of a segment table need a quantized prefix")
    if dense_dtype is None:
        dense_dtype = next((k.dtype for k, _ in dense), None) or next(
            (s.residual_key.dtype for s in packed if s.residual_tokens), torch.bfloat16)
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    # every tensor whose address goes into the launch table, on one GPU, before any launch
    device = nat.require_device(
        q, *(t for pair in dense for t in pair),
        *(t for s in packed for t in (s.key_code, s.key_scale, s.key_minimum, s.value_code, s.value_scale,
                                      s.value_minimum, s.residual_key if s.residual_tokens else None,
                                      s.residual_value if s.residual_tokens else None)),
        what="Segment-table attention")
    keep = []
    dense_structs = []
    for key, value in dense:
        if int(key.shape[0]) == 0:
            continue
        seg, tensors = _dense_segment(key.to(dense_dtype), value.to(dense_dtype))
        dense_structs.append(seg)
        keep.append(tensors)
    items = (nat.KiviItem * len(packed))()
    for j, cache in enumerate(packed):
        tr = cache.residual_tokens
        rk, rv = cache.residual_key, cache.residual_value
        if tr and (rk.dtype != dense_dtype or not rk.is_contiguous() or not rv.is_contiguous()):
            rk, rv = rk.to(dense_dtype).contiguous(), rv.to(dense_dtype).contiguous()
            keep.append((rk, rv))
        items[j] = cache.native_item(None, None, None, residual_key_ptr=rk.data_ptr() if tr else None,
                                     residual_value_ptr=rv.data_ptr() if tr else None, residual_tokens=tr)
    table = (nat.DenseSegment * max(1, len(dense_structs)))(*dense_structs)
    out = torch.empty((lq, hq, d), dtype=q.dtype, device=device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=device)
    nat.call(
        "uc_kivi_attn_mq_segments", items, len(packed), table, len(dense_structs), q.data_ptr(), out.data_ptr(),
        lse.data_ptr(), first.k_bits, first.group_size, hq, hkv, d, lq, nat.dtype_code(q.dtype),
        nat.dtype_code(dense_dtype), nat.dtype_code(q.dtype), 1.0 / math.sqrt(d), nat.stream(device),
    )
    return out, lse


DECODE_MAX_SEGMENTS = 8  # items one uc_kivi_attn_decode_segments_host call takes


def decode_segments_supported(packed: list, query: torch.Tensor, dense: list) -> bool:
    """Whether decode_segments_summary takes this layout: decode-length 16-bit
    queries (at most 16 query rows per KV head), head_dim 128, native packed
    prefixes of equal 2/4-bit K/V sharing group size (32/64/128) and KV heads,
    dense parts and residuals of one 16-bit dtype in rows whose channels are
    contiguous, and at most 8 segments (each prefix with its residual, each
    non-empty dense part)."""

    if not packed or query.dim() != 3 or int(query.shape[2]) != 128 or query.dtype not in (torch.bfloat16,
                                                                                             torch.float16):
        return False
    first = packed[0]
    if first.k_bits not in (2, 4) or first.group_size not in (32, 64, 128):
        return False
    if any((s.k_bits, s.v_bits, s.group_size, s.num_kv_heads) != (first.k_bits, first.k_bits, first.group_size,
                                                                  first.num_kv_heads) or not s.kernel_native_layout
           for s in packed):
        return False
    if int(query.shape[0]) > _max_decode_query_len(first, int(query.shape[1])):
        return False
    parts = [(k, v) for k, v in dense if int(k.shape[0])] + [
        (s.residual_key, s.residual_value) for s in packed if s.residual_tokens]
    if len({k.dtype for k, _ in parts} | {v.dtype for _, v in parts}) > 1:
        return False
    if any(k.dtype not in (torch.bfloat16, torch.float16) or k.stride() != v.stride() or k.stride(2) != 1
           for k, v in parts):
        return False
    return len(packed) + sum(1 for k, _ in dense if int(k.shape[0])) <= DECODE_MAX_SEGMENTS


def decode_segments_summary(packed: list, query: torch.Tensor, dense: list) -> tuple[torch.Tensor, torch.Tensor]:
    """One softmax of a decode-length query [Lq, Hq, 128] over the packed
    prefixes (with their residuals) of the PackedKIVICache segments `packed`
    and the dense (key, value) [T, Hkv, 128] parts `dense` -- any token and
    head strides, so an H2O segment's [Hkv, R, 128] tensors enter transposed,
    as views -- in one launch of the split-K decode kernels
    (uc_kivi_attn_decode_segments_host): the segments are read where they lie,
    nothing is concatenated and no summaries are merged.  This is the decode
    form of _run_fused_mixed_attention (adapters/bagel.py:1598-1858).  Returns
    (out [Lq, Hq, 128] in the query dtype, lse [Hq, Lq])."""

    if not decode_segments_supported(packed, query, dense):
        raise ValueError("Decode segment attention needs decode-length 16-bit queries, head_dim 128, native packed "
                         "prefixes of equal 2/4-bit K/V sharing group size and KV heads, dense parts and residuals "
                         f"of one 16-bit dtype with contiguous channels, and at most {DECODE_MAX_SEGMENTS} segments")
    first = packed[0]
    hkv = first.num_kv_heads
    for key, value in dense:
        if key.shape != value.shape or key.dim() != 3 or tuple(key.shape[1:]) != (hkv, 128):
            raise ValueError("Dense segments must be matching [tokens, kv_heads, 128] tensors")
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    parts = [(k, v) for k, v in dense if int(k.shape[0])]
    device = nat.require_device(
        q, *(t for pair in parts for t in pair),
        *(t for s in packed for t in (s.key_code, s.residual_key if s.residual_tokens else None)),
        what="Decode segment attention")
    res_dtype = next((k.dtype for k, _ in parts), None) or next(
        (s.residual_key.dtype for s in packed if s.residual_tokens), q.dtype)
    out = torch.empty((lq, hq, d), dtype=q.dtype, device=device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=device)
    n = len(packed) + len(parts)
    items = (nat.KiviItem * n)()
    max_tq = max_tr = 0
    for j, cache in enumerate(packed):
        tr = cache.residual_tokens
        rk, rv = cache.residual_key, cache.residual_value
        items[j] = cache.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                     residual_key_ptr=rk.data_ptr() if tr else None,
                                     residual_value_ptr=rv.data_ptr() if tr else None, residual_tokens=tr)
        if tr:
            items[j].residual_token_stride, items[j].residual_head_stride = rk.stride(0), rk.stride(1)
        max_tq, max_tr = max(max_tq, cache.quantized_tokens), max(max_tr, tr)
    for j, (key, value) in enumerate(parts, start=len(packed)):
        t = int(key.shape[0])
        items[j] = nat.KiviItem(None, None, None, None, None, None, key.data_ptr(), value.data_ptr(), q.data_ptr(),
                                out.data_ptr(), lse.data_ptr(), 0, t, 0, key.stride(0), key.stride(1))
        max_tr = max(max_tr, t)
    ws_bytes = nat.decode_workspace_bytes(n, first.k_bits, first.group_size, hq, hkv, d, lq, max_tq, max_tr)
    workspace = nat.workspace(device, ws_bytes)
    nat.call("uc_kivi_attn_decode_segments_host", items, n, first.k_bits, first.group_size, hq, hkv, d, lq,
             nat.dtype_code(q.dtype), nat.dtype_code(res_dtype), nat.dtype_code(q.dtype), 1.0 / math.sqrt(d),
             workspace.data_ptr(), ws_bytes, nat.stream(device))
    return out, lse


def packed_table_summaries(entries: list, *, dense_dtype: torch.dtype) -> None:
    """Several independent long-query attentions in as few launches as the
    table limits allow (uc_kivi_attn_mq_table, 8 queries / 8 packed prefixes /
    16 dense parts per launch): entry = (query [Lq, Hq, 128], out [Lq, Hq, 128]
    in the query dtype, lse fp32 [Hq, Lq] or None, packed caches (each with a
    quantized prefix), dense (key, value) [T, Hkv, 128] parts).  Each entry is
    one softmax over its segments, read in place; every out / lse is written.
    All entries share the packed bits, group size, KV heads, query dtype and
    `dense_dtype`; results equal packed_segments_summary per entry bit for bit
    (dense-only entries: bits 2 / group 32 stand for the absent codes)."""

    if not entries:
        return
    q0 = entries[0][0]
    hq, d = int(q0.shape[1]), int(q0.shape[2])
    first = next((c for e in entries for c in e[3]), None)
    bits, group = (first.k_bits, first.group_size) if first is not None else (2, 32)
    if first is not None:
        hkv = first.num_kv_heads
    else:
        part = next((k for e in entries for k, _ in e[4] if k.dim() == 3), None)
        if part is None:
            raise ValueError("Table attention needs a packed cache or a dense [tokens, kv_heads, head_dim] part")
        hkv = int(part.shape[1])
    tensors = []
    for query, out, lse, caches, dense in entries:
        if query.dtype != q0.dtype or out.dtype != q0.dtype or tuple(query.shape[1:]) != (hq, d) or \
                out.shape != query.shape or not (query.is_contiguous() and out.is_contiguous()):
            raise ValueError("Table attention needs contiguous queries and outputs of one dtype and shape")
        if lse is not None and (lse.dtype != torch.float32 or tuple(lse.shape) != (hq, int(query.shape[0]))
                                or not lse.is_contiguous()):
            raise ValueError("Table attention: lse must be contiguous fp32 [Hq, Lq]")
        if caches and not packed_segments_supported(caches, query, dense):
            raise ValueError("Table attention: unsupported packed layout or query length")
        if not caches and (d != 128 or query.dtype not in (torch.bfloat16, torch.float16)
                           or any(k.dtype not in (torch.bfloat16, torch.float16) for k, _ in dense)):
            # the dtype and head_dim checks packed_segments_supported makes for
            # entries with caches (the kernel takes any query length)
            raise ValueError("Table attention: dense-only entries need 16-bit queries and parts, head_dim 128")
        for cache in caches:
            if (cache.k_bits, cache.v_bits, cache.group_size, cache.num_kv_heads) != (bits, bits, group, hkv):
                raise ValueError("Table attention needs equal bits, group size and KV heads")
            if not cache.quantized_tokens:
                raise ValueError("Packed segments of a segment table need a quantized prefix")
        for key, value in dense:
            if key.shape != value.shape or key.dim() != 3 or tuple(key.shape[1:]) != (hkv, d):
                raise ValueError("Dense segments must be matching [tokens, kv_heads, head_dim] tensors")
        tensors += [query, out, lse, *(t for pair in dense for t in pair)]
        for c in caches:
            tensors += [c.key_code, c.key_scale, c.key_minimum, c.value_code, c.value_scale, c.value_minimum]
            if c.residual_tokens:
                tensors += [c.residual_key, c.residual_value]
    device = nat.require_device(*tensors, what="Table attention")
    stream = nat.stream(device)
    i = 0
    while i < len(entries):
        # greedy chunk within the per-launch limits
        chunk, n_p, n_d = [], 0, 0
        while i < len(entries) and len(chunk) < MQ_MAX_BATCH:
            _, _, _, caches, dense = entries[i]
            need_p = len(caches)
            need_d = sum(1 for k, _ in dense if int(k.shape[0])) + sum(1 for c in caches if c.residual_tokens)
            if need_p > MQ_MAX_PACKED or need_d > MQ_MAX_DENSE:
                raise ValueError("Table attention: one query exceeds the per-launch segment limits")
            if n_p + need_p > MQ_MAX_PACKED or n_d + need_d > MQ_MAX_DENSE:
                break
            chunk.append(entries[i])
            n_p, n_d = n_p + need_p, n_d + need_d
            i += 1
        queries = (nat.MqQuery * len(chunk))()
        items = (nat.KiviItem * max(1, n_p))()
        dsegs = (nat.DenseSegment * max(1, n_d))()
        keep = []
        pi = di = 0
        for j, (query, out, lse, caches, dense) in enumerate(chunk):
            queries[j] = nat.MqQuery(query.data_ptr(), out.data_ptr(), nat.ptr(lse), int(query.shape[0]),
                                     pi, len(caches), di, 0)
            for cache in caches:
                tr = cache.residual_tokens
                rk, rv = cache.residual_key, cache.residual_value
                if tr and (rk.dtype != dense_dtype or not rk.is_contiguous() or not rv.is_contiguous()):
                    rk, rv = rk.to(dense_dtype).contiguous(), rv.to(dense_dtype).contiguous()
                    keep.append((rk, rv))
                items[pi] = cache.native_item(None, None, None, residual_key_ptr=rk.data_ptr() if tr else None,
                                              residual_value_ptr=rv.data_ptr() if tr else None, residual_tokens=tr)
                pi += 1
            n_dense = 0
            for key, value in dense:
                if int(key.shape[0]) == 0:
                    continue
                seg, kept = _dense_segment(key.to(dense_dtype), value.to(dense_dtype))
                dsegs[di + n_dense] = seg
                keep.append(kept)
                n_dense += 1
            queries[j].n_dense = n_dense
            di += n_dense
        nat.call(
            "uc_kivi_attn_mq_table", queries, len(chunk), items, pi, dsegs, di, bits, group, hq, hkv, d,
            nat.dtype_code(q0.dtype), nat.dtype_code(dense_dtype), nat.dtype_code(q0.dtype), 1.0 / math.sqrt(d),
            stream,
        )


def dense_attention_summary(
    query: torch.Tensor, key: torch.Tensor, value: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Softmax attention of query [Lq, Hq, D] over dense 16-bit keys/values
    [T, Hkv, D] in one pass of the packed kernels with an empty packed prefix:
    the bf16-only summary (flash_attention_summary, adapters/bagel.py:75-95).
    (out [Lq, Hq, D] in the query dtype, lse [Hq, Lq])."""

    if key.shape != value.shape or key.dim() != 3 or query.dim() != 3:
        raise ValueError("Dense attention expects query [Lq, Hq, D] and matching [T, Hkv, D] keys/values")
    lq, hq, d = map(int, query.shape)
    tokens, hkv = int(key.shape[0]), int(key.shape[1])
    if int(key.shape[2]) != d or hq % hkv:
        raise ValueError("Dense attention: head_dim must match and query heads divide by KV heads")
    if tokens == 0:
        raise ValueError("Dense attention needs at least one key")
    if key.dtype not in (torch.bfloat16, torch.float16) or value.dtype != key.dtype:
        raise ValueError("Dense attention needs bf16 or fp16 keys and values")
    if query.dtype not in (torch.bfloat16, torch.float16):
        query = query.to(torch.bfloat16)
    device = nat.require_device(query, key, value, what="Dense attention")
    q, dk, dv = query.contiguous(), key.contiguous(), value.contiguous()
    out = torch.empty((lq, hq, d), dtype=q.dtype, device=device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=device)
    item = nat.KiviItem(None, None, None, None, None, None, dk.data_ptr(), dv.data_ptr(), q.data_ptr(),
                        out.data_ptr(), lse.data_ptr(), 0, tokens, 0)
    bits, group = 2, 32  # no packed tokens: only the dense (residual) part is read
    if lq <= max(1, 16 // (hq // hkv)):
        ws_bytes = nat.decode_workspace_bytes(1, bits, group, hq, hkv, d, lq, 0, tokens)
        entry = "uc_kivi_attn_decode"
    else:
        if d != 128:
            raise ValueError("Dense attention over more than 16 query rows per KV head needs head_dim 128")
        ws_bytes = 0  # the multi-query kernel needs no workspace
        entry = "uc_kivi_attn_mq"
    ws = nat.workspace(device, ws_bytes) if ws_bytes else None
    nat.call(entry, item, bits, group, hq, hkv, d, lq, nat.dtype_code(q.dtype), nat.dtype_code(dk.dtype),
             nat.dtype_code(q.dtype), 1.0 / math.sqrt(d), nat.ptr(ws), ws_bytes, nat.stream(device))
    return out, lse


def packed_kivi_quantized_attention_summary(
    cache: "PackedKIVICache", query: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Normalised output and LSE for the packed quantized prefix
    (kivi_cuda.py:96-120)."""

    return packed_kivi_attention_summary(cache, query, include_residual=False)


def quantize_kivi_native(
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    k_bits: int,
    v_bits: int,
    group_size: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """KIVI's kernel-native packed layout in one HIP pass (kivi_cuda.py:157-190):
    keys grouped along tokens -> [Hkv, D, T*b/32] words, values grouped along
    channels -> [Hkv, T, D*b/32] words, fp16 scale/minimum.  The tensors have
    these shapes but token-major strides (views of [Hkv, T*b/32, D] and
    [Hkv, T/G, D] key storage), the layout the attention kernels read."""

    if key.shape != value.shape or key.dim() != 3:
        raise ValueError("KIVI native packing expects matching [tokens, heads, dim] KV")
    if key.device.type != "cuda":
        raise RuntimeError("KIVI native packing requires CUDA tensors")
    if k_bits not in {2, 4} or v_bits not in {2, 4}:
        raise ValueError("KIVI native packing supports 2-bit or 4-bit codes")
    return _pack_native(key, value, k_bits=int(k_bits), v_bits=int(v_bits), group_size=int(group_size))


def packed_kivi_attention_parts(
    cache: "PackedKIVICache",
    query: torch.Tensor,
) -> tuple[torch.Tensor, Callable[[torch.Tensor], torch.Tensor]]:
    """Scaled fp32 logits [Hq, Lq, Tq+Tr] over [packed | residual] and an AV
    closure returning [Hq, Lq, D] in the residual dtype (kivi_cuda.py:238-329)."""

    if query.device.type != "cuda":
        raise RuntimeError("Physical KIVI CUDA backend received a non-CUDA query")
    if cache.k_bits != cache.v_bits:
        raise ValueError("Official KIVI kernel path requires equal key/value bit widths")
    repeat = int(query.shape[1]) // cache.num_kv_heads
    if repeat * cache.num_kv_heads != int(query.shape[1]):
        raise ValueError("Query heads must be divisible by KIVI KV heads")
    if cache.quantized_tokens and cache.k_bits in {2, 4} and not cache.kernel_native_layout:
        raise RuntimeError("Physical KIVI CUDA cache is not stored in kernel-native layout")
    device = nat.require_device(query, cache.residual_key, what="Physical KIVI attention")
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    tq, tr = cache.quantized_tokens, cache.residual_tokens
    res = cache.residual_key
    stats_dtype = cache.key_scale.dtype if tq else torch.float16
    cap = cache.native_packed_pointers(device)[-1] if tq and cache.k_bits in (2, 4) else 0
    logits = torch.empty((hq, lq, tq + tr), dtype=torch.float32, device=device)
    nat.call(
        "uc_kivi_qk", q.data_ptr(), nat.dtype_code(q.dtype), lq, hq,
        nat.ptr(cache.key_code), nat.ptr(cache.key_scale), nat.ptr(cache.key_minimum),
        nat.dtype_code(stats_dtype), tq, cap, cache.k_bits, cache.group_size,
        res.data_ptr(), nat.dtype_code(res.dtype), tr, int(res.stride(0)), int(res.stride(1)),
        cache.num_kv_heads, d, 1.0 / math.sqrt(d), logits.data_ptr(), nat.stream(device),
    )

    def apply_value(probabilities: torch.Tensor) -> torch.Tensor:
        if tuple(probabilities.shape) != (hq, lq, tq + tr):
            raise ValueError("KIVI AV probabilities must be [query_heads, queries, tokens]")
        nat.require_device(probabilities, what="Physical KIVI AV")
        val = cache.residual_value
        out = torch.empty((hq, lq, d), dtype=val.dtype, device=device)
        ws = nat.workspace(device, nat.workspace_bytes(nat.UC_OP_KIVI_AV, 1, hq, lq, d, tq + tr))
        nat.call(
            "uc_kivi_av", probabilities.data_ptr(), nat.dtype_code(probabilities.dtype),
            *map(int, probabilities.stride()), lq, hq,
            nat.ptr(cache.value_code), nat.ptr(cache.value_scale), nat.ptr(cache.value_minimum),
            nat.dtype_code(stats_dtype), tq, cap, cache.v_bits, cache.group_size,
            val.data_ptr(), nat.dtype_code(val.dtype), tr, int(val.stride(0)), int(val.stride(1)),
            cache.num_kv_heads, d, out.data_ptr(), nat.dtype_code(val.dtype), ws.data_ptr(),
            nat.stream(device),
        )
        return out

    return logits, apply_value
