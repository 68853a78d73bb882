"""Segment-summary merge, fused mixed-segment attention and batched
physical attention of the BAGEL adapter on the MI355X kernels."""

from __future__ import annotations

import ctypes

import torch

from .. import _native as nat


def merge_attention_summaries(
    summaries: list[tuple[torch.Tensor, torch.Tensor]],
) -> tuple[torch.Tensor, torch.Tensor]:
    """Merge normalised segment outputs [Lq, Hq, D] by their per-row LSE
    [Hq, Lq] (adapters/bagel.py:57-72): lse = logsumexp_s lse_s and
    out = sum_s out_s * exp(lse_s - lse), accumulated in fp32 and returned in
    the first output's dtype."""

    if not summaries:
        raise ValueError("At least one attention summary is required")
    out0 = summaries[0][0]
    device = nat.require_device(*[o for o, _ in summaries], *[l for _, l in summaries],
                                what="Attention summary merge")
    lq, hq, d = map(int, out0.shape)
    same = all(o.dtype == out0.dtype for o, _ in summaries)
    work_dtype = out0.dtype if same else torch.float32
    outs = [o.to(work_dtype).contiguous() for o, _ in summaries]
    lses = [l.float().contiguous() for _, l in summaries]
    for o, l in zip(outs, lses):
        if tuple(o.shape) != (lq, hq, d) or tuple(l.shape) != (hq, lq):
            raise ValueError("Attention summaries must be out [Lq, Hq, D] and lse [Hq, Lq]")
    merged = torch.empty((lq, hq, d), dtype=work_dtype, device=device)
    total = torch.empty((hq, lq), dtype=torch.float32, device=device)
    n = len(outs)
    out_ptrs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    lse_ptrs = (ctypes.c_void_p * n)(*[l.data_ptr() for l in lses])
    nat.call(
        "uc_lse_merge", ctypes.cast(out_ptrs, ctypes.c_void_p), ctypes.cast(lse_ptrs, ctypes.c_void_p), n,
        nat.dtype_code(work_dtype), lq, hq, d, merged.data_ptr(), total.data_ptr(), nat.stream(device),
    )
    return merged.to(out0.dtype), total


def run_fused_mixed_attention(
    query: torch.Tensor,
    dense_key: torch.Tensor,
    dense_value: torch.Tensor,
    physical_segments: list,
    *,
    return_lse: bool = False,
):
    """Attention of query [Lq, Hq, D] over a mixed cache: the dense bf16 KV
    [T, Hkv, D], the retained tokens of GQAH2OCache segments, and the packed
    prefix plus residual of PackedKIVICache segments
    (_run_fused_mixed_attention, adapters/bagel.py:1598-1858).

    Long queries (image editing) take one launch over a segment table
    (packed_segments_summary): every packed prefix is dequantized inside the
    attention kernel and every bf16 part -- the dense KV, the H2O segments
    (read through their [Hkv, T, D] strides) and the residuals -- is read
    where it lies, in one softmax.  Decode-length queries take the split-K
    decode kernels over the same segments, read in place
    (decode_segments_summary).  Otherwise the bf16 keys are gathered in
    UniCache's order [dense, H2O..., residuals...] and attended in the same
    fused pass as the first packed segment's prefix; further packed prefixes
    get their own pass (all passes in one batched launch for long queries) and
    the summaries are merged by LSE.  Non-frozen H2O segments then receive
    exp(logit - global LSE) as bf16 probabilities and are trimmed to their
    budget.  Returns the output (and the global LSE [Hq, Lq] with
    return_lse=True)."""

    from ..storage.kivi_cuda import (_max_decode_query_len, decode_segments_summary, decode_segments_supported,
                                     packed_batch_with_dense, packed_kivi_quantized_attention_summary,
                                     packed_segments_summary, packed_segments_supported, packed_summary_with_dense)
    from ..storage.physical import GQAH2OCache, PackedKIVICache

    h2o = [s for s in physical_segments if isinstance(s, GQAH2OCache)]
    packed = [s for s in physical_segments if isinstance(s, PackedKIVICache)]
    with_prefix = [s for s in packed if s.quantized_tokens]
    if not with_prefix:
        raise RuntimeError("Fused mixed attention requires packed KIVI tokens")
    lq, hq, d = map(int, query.shape)
    first = with_prefix[0]
    dense_parts = [(dense_key, dense_value)] + [(s.key.transpose(0, 1), s.value.transpose(0, 1)) for s in h2o] + [
        (s.residual_key, s.residual_value) for s in packed if not s.quantized_tokens and s.residual_tokens]
    if dense_key.dtype in (torch.bfloat16, torch.float16) and packed_segments_supported(with_prefix, query,
                                                                                      dense_parts):
        output, global_lse = packed_segments_summary(with_prefix, query, dense_parts, dense_dtype=dense_key.dtype)
    elif decode_segments_supported(with_prefix, query, dense_parts):
        output, global_lse = decode_segments_summary(with_prefix, query, dense_parts)
    else:
        keys = [dense_key] + [s.key.transpose(0, 1) for s in h2o] + [
            s.residual_key for s in packed if s.residual_tokens]
        values = [dense_value] + [s.value.transpose(0, 1) for s in h2o] + [
            s.residual_value for s in packed if s.residual_tokens]
        all_key = torch.cat([k.to(dense_key.dtype) for k in keys], dim=0)
        all_value = torch.cat([v.to(dense_value.dtype) for v in values], dim=0)
        if (len(with_prefix) > 1 and query.dtype in (torch.bfloat16, torch.float16)
                and all_key.dtype in (torch.bfloat16, torch.float16) and all_value.dtype == all_key.dtype
                and d == 128 and first.group_size in (32, 64, 128) and first.k_bits in (2, 4)
                and lq > _max_decode_query_len(first, hq)
                and all((s.k_bits, s.v_bits, s.group_size, s.num_kv_heads) == (first.k_bits, first.k_bits,
                                                                              first.group_size, first.num_kv_heads)
                        for s in with_prefix)):
            # every packed prefix in one attention launch (the first with the
            # dense keys), the same summaries as one pass per prefix
            q = query.contiguous()
            summaries = [(torch.empty_like(q), torch.empty((hq, lq), dtype=torch.float32, device=q.device))
                         for _ in with_prefix]
            packed_batch_with_dense([(s, q, [all_key] if j == 0 else [], [all_value] if j == 0 else [], o, lse)
                                     for j, (s, (o, lse)) in enumerate(zip(with_prefix, summaries))])
        else:
            summaries = [packed_summary_with_dense(first, query, all_key, all_value)]
            summaries += [packed_kivi_quantized_attention_summary(s, query) for s in with_prefix[1:]]
        output, global_lse = summaries[0] if len(summaries) == 1 else merge_attention_summaries(summaries)
    for segment in h2o:
        if segment.selection_frozen:
            continue
        segment.update_scores_from_query(query, global_lse)
        segment.enforce_budget()
    return (output, global_lse) if return_lse else output


def run_batched_physical_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    physical_cache_by_sample: list,
) -> torch.Tensor:
    """Non-causal varlen attention of packed samples over their frozen physical
    layouts (apply_static_physical_attention_batch, adapters/bagel.py:773-980):
    sample i's queries q[cu_q[i]:cu_q[i+1]] attend to its current keys
    k[cu_k[i]:cu_k[i+1]], the retained tokens of its GQAH2OCache segments and
    the residual and packed prefix of its PackedKIVICache segments.  CFG
    branches packed with pack_naive_caches are such samples.

    Samples with packed prefixes whose queries exceed the decode limit run
    together over one segment table (packed_table_summaries: one launch per 8
    samples within the table limits): each sample's packed prefixes,
    residuals, current keys and H2O segments are read in place, no
    concatenation, and the rows of the output are written in place.  Other
    samples with a packed prefix are one fused pass each
    (run_fused_mixed_attention) and H2O-only samples one dense pass, so the
    packed prefixes are never dequantised into a varlen workspace.  Returns
    [total queries, Hq, D] in q's dtype.  H2O segments must be frozen, as in the
    reference fast path."""

    from ..storage.kivi_cuda import dense_attention_summary, packed_segments_supported, packed_table_summaries
    from ..storage.physical import GQAH2OCache, PackedKIVICache

    cu_q = [int(x) for x in (cu_seqlens_q.tolist() if torch.is_tensor(cu_seqlens_q) else cu_seqlens_q)]
    cu_k = [int(x) for x in (cu_seqlens_k.tolist() if torch.is_tensor(cu_seqlens_k) else cu_seqlens_k)]
    samples = len(physical_cache_by_sample)
    if len(cu_q) != samples + 1 or len(cu_k) != samples + 1:
        raise ValueError("cu_seqlens must have one more entry than physical_cache_by_sample")
    if cu_q[-1] != int(q.shape[0]) or cu_k[-1] != int(k.shape[0]) or k.shape != v.shape:
        raise ValueError("cu_seqlens must cover q and k; k and v must match")
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    hq, d = int(q.shape[1]), int(q.shape[2])
    qc = q.contiguous()
    tables: dict = {}  # (bits, group, kv heads) -> entries of packed_table_summaries
    for i, segments in enumerate(physical_cache_by_sample):
        if not segments:
            raise ValueError(f"Sample {i} has no physical segments")
        q_i = qc[cu_q[i]:cu_q[i + 1]]
        k_i, v_i = k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]]
        h2o = [s for s in segments if isinstance(s, GQAH2OCache)]
        packed = [s for s in segments if isinstance(s, PackedKIVICache)]
        if any(not s.selection_frozen for s in h2o):
            raise ValueError("Batched physical attention needs frozen H2O selections")
        if q_i.shape[0] == 0:
            continue
        with_prefix = [s for s in packed if s.quantized_tokens]
        out_i = out[cu_q[i]:cu_q[i + 1]]
        dense_parts = [(k_i, v_i)] + [(s.key.transpose(0, 1), s.value.transpose(0, 1)) for s in h2o] + [
            (s.residual_key, s.residual_value) for s in packed if not s.quantized_tokens and s.residual_tokens]
        if with_prefix and k.dtype in (torch.bfloat16, torch.float16) and packed_segments_supported(
                with_prefix, q_i, dense_parts):
            key = (with_prefix[0].k_bits, with_prefix[0].group_size, with_prefix[0].num_kv_heads)
            tables.setdefault(key, []).append((q_i, out_i, None, with_prefix, dense_parts))
            continue
        if with_prefix:
            out_i.copy_(run_fused_mixed_attention(q_i, k_i, v_i, list(segments)))
            continue
        keys = [k_i] + [s.key.transpose(0, 1) for s in h2o] + [s.residual_key for s in packed if s.residual_tokens]
        values = [v_i] + [s.value.transpose(0, 1) for s in h2o] + [
            s.residual_value for s in packed if s.residual_tokens]
        dk = torch.cat([x.to(k.dtype) for x in keys], dim=0)
        dv = torch.cat([x.to(v.dtype) for x in values], dim=0)
        out_i.copy_(dense_attention_summary(q_i, dk, dv)[0])
    for entries in tables.values():
        packed_table_summaries(entries, dense_dtype=k.dtype)
    return out

