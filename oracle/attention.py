"""numpy restatement of the GQA attention products over physical segments.

Logits and softmax are evaluated in float64 ("the fp32 dequant path" to well
within the tolerances the kernels are held to: 2e-2 max abs, 1e-3 mean abs).
"""

from __future__ import annotations

import math

import numpy as np

from .kivi import PackedSegment, dequantize, round_to


def gqa_logits(query, key) -> np.ndarray:
    """gqa_query_key_logits (physical.py:20-39): query [Lq, Hq, D], key
    [T, Hkv, D] -> [Hq, Lq, T]; query head h reads KV head h // (Hq/Hkv)."""

    q = np.asarray(query, dtype=np.float64)
    k = np.asarray(key, dtype=np.float64)
    lq, hq, d = q.shape
    t, hkv, _ = k.shape
    group = hq // hkv
    gq = q.transpose(1, 0, 2).reshape(hkv, group, lq, d)
    gk = k.transpose(1, 0, 2)[:, None]  # [Hkv, 1, T, D]
    return (gq @ gk.transpose(0, 1, 3, 2)).reshape(hq, lq, t)


def gqa_pv(probs, value) -> np.ndarray:
    """gqa_probability_value (physical.py:42-63): [Hq, Lq, T] x [T, Hkv, D]
    -> [Hq, Lq, D]."""

    p = np.asarray(probs, dtype=np.float64)
    v = np.asarray(value, dtype=np.float64)
    hq, lq, t = p.shape
    hkv = v.shape[1]
    group = hq // hkv
    gp = p.reshape(hkv, group, lq, t)
    gv = v.transpose(1, 0, 2)[:, None]
    return (gp @ gv).reshape(hq, lq, v.shape[-1])


def softmax(x, axis=-1):
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def logsumexp(x, axis=-1):
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    return (np.log(np.exp(x - m).sum(axis=axis, keepdims=True)) + m).squeeze(axis)


def attention_summary(query, key, value, scale=None):
    """Softmax attention of query [Lq, Hq, D] over dense key/value [T, Hkv, D]:
    (out [Lq, Hq, D], lse [Hq, Lq]) with the natural-log LSE of
    kivi_triton.py:366-382."""

    d = np.asarray(query).shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    logits = gqa_logits(query, key) * scale
    out = gqa_pv(softmax(logits), value)
    return out.transpose(1, 0, 2), logsumexp(logits)


def packed_logits(seg: PackedSegment, query, kv_dtype="bf16") -> np.ndarray:
    """packed_kivi_attention_parts logits (kivi_cuda.py:283-287 /
    physical.py:469-470): [Hq, Lq, Tq+Tr] over the dequantized segment,
    scaled by 1/sqrt(D)."""

    key, _ = dequantize(seg, kv_dtype)
    d = np.asarray(query).shape[-1]
    return gqa_logits(query, key) / math.sqrt(d)


def packed_pv(seg: PackedSegment, probs, kv_dtype="bf16") -> np.ndarray:
    """The apply_value closure of physical.py:472-473: P x dequantized V."""

    _, value = dequantize(seg, kv_dtype)
    return gqa_pv(probs, value)


def packed_summary(seg: PackedSegment, query, *, include_residual=True, kv_dtype="bf16"):
    """(out, lse) over the dequantized packed prefix (and residual)."""

    key, value = dequantize(seg, kv_dtype)
    if not include_residual:
        key, value = key[: seg.quantized_tokens], value[: seg.quantized_tokens]
    return attention_summary(query, key, value)


def merge_summaries(summaries, out_dtype="fp32"):
    """merge_attention_summaries (adapters/bagel.py:57-72):
    lse = logsumexp_s lse_s; out = sum_s out_s * exp(lse_s - lse)."""

    lses = np.stack([np.asarray(l, dtype=np.float64) for _, l in summaries], axis=0)
    total = logsumexp(lses, axis=0)
    out = np.zeros(np.asarray(summaries[0][0]).shape, dtype=np.float64)
    for seg_out, seg_lse in summaries:
        w = np.exp(np.asarray(seg_lse, dtype=np.float64) - total).T[:, :, None]
        out = out + np.asarray(seg_out, dtype=np.float64) * w
    return round_to(out.astype(np.float32), out_dtype), total.astype(np.float32)
