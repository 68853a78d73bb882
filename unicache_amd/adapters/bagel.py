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
