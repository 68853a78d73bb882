"""Segment-summary merge of the BAGEL adapter on the MI355X kernels."""

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

    The bf16 keys are gathered in UniCache's order [dense, H2O..., residuals...]
    and attended in the same fused pass as the first packed segment's prefix;
    further packed prefixes get their own pass and the summaries are merged by
    LSE.  Non-frozen H2O segments then receive exp(logit - global LSE) as
    bf16 probabilities and are trimmed to their budget.  Returns the output
    (and the global LSE [Hq, Lq] with return_lse=True)."""

    from ..storage.kivi_cuda import packed_kivi_quantized_attention_summary, packed_summary_with_dense
    from ..storage.physical import GQAH2OCache, PackedKIVICache

    h2o = [s for s in physical_segments if isinstance(s, GQAH2OCache)]
    packed = [s for s in physical_segments if isinstance(s, PackedKIVICache)]
    with_prefix = [s for s in packed if s.quantized_tokens]
    if not with_prefix:
        raise RuntimeError("Fused mixed attention requires packed KIVI tokens")
    keys = [dense_key] + [s.key.transpose(0, 1) for s in h2o] + [s.residual_key for s in packed if s.residual_tokens]
    values = [dense_value] + [s.value.transpose(0, 1) for s in h2o] + [
        s.residual_value for s in packed if s.residual_tokens]
    all_key = torch.cat([k.to(dense_key.dtype) for k in keys], dim=0)
    all_value = torch.cat([v.to(dense_value.dtype) for v in values], dim=0)
    summaries = [packed_summary_with_dense(with_prefix[0], query, all_key, all_value)]
    summaries += [packed_kivi_quantized_attention_summary(s, query) for s in with_prefix[1:]]
    output, global_lse = summaries[0] if len(summaries) == 1 else merge_attention_summaries(summaries)
    for segment in h2o:
        if segment.selection_frozen:
            continue
        segment.update_scores_from_query(query, global_lse)
        segment.enforce_budget()
    return (output, global_lse) if return_lse else output
