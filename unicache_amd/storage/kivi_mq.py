"""Multi-query (editing) attention over a packed KIVI segment.

The Lq x group query rows are processed in slices small enough for the
split-K decode kernel (group * rows <= 16) and stitched together; each slice
reads the packed segment once.
"""

from __future__ import annotations

import torch

from .kivi_cuda import _decode_summary, _max_decode_query_len


def packed_attention_mq(cache, query: torch.Tensor, *, include_residual: bool = True):
    """(out [Lq, Hq, D], lse [Hq, Lq]) of attention over the packed prefix
    (plus the residual when include_residual)."""

    lq, hq, d = map(int, query.shape)
    step = _max_decode_query_len(cache, hq)
    out = torch.empty((lq, hq, d), dtype=query.dtype, device=query.device)
    lse = torch.empty((hq, lq), dtype=torch.float32, device=query.device)
    for start in range(0, lq, step):
        stop = min(lq, start + step)
        o, l = _decode_summary(cache, query[start:stop], include_residual=include_residual, out_dtype=query.dtype)
        out[start:stop].copy_(o)
        lse[:, start:stop].copy_(l)
    return out, lse
