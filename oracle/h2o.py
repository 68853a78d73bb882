"""numpy restatement of H2O scoring, selection and GQA compaction."""

from __future__ import annotations

import math

import numpy as np

from .attention import gqa_logits, softmax
from .kivi import round_bf16


def scores_from_probs(probs, kv_heads: int) -> np.ndarray:
    """operators/physical.py:62-65 (and physical.py:607-609):
    P.float().sum(queries) -> [Hkv, group, T] -> sum(group)."""

    p = np.asarray(probs, dtype=np.float64)
    hq, _, t = p.shape
    return p.sum(axis=1).reshape(kv_heads, hq // kv_heads, t).sum(axis=1).astype(np.float32)


def scores_from_qk(query, key, scale=None) -> np.ndarray:
    """The adapter's probabilities (softmax of the 1/sqrt(D)-scaled fp32
    logits, cast to bf16; adapters/bagel.py:1205-1243) reduced per KV head."""

    d = np.asarray(query).shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    logits = (gqa_logits(query, key) * scale).astype(np.float32)
    probs = round_bf16(softmax(logits).astype(np.float32))
    return scores_from_probs(probs, np.asarray(key).shape[1])


def budget(segment_tokens: int, params: dict) -> tuple[int, int]:
    """(target, recent) of tensor_backend.py:199-210; Python round() is
    round-half-to-even."""

    target = params.get("budget", params.get("keep_k"))
    if target is None:
        ratio = float(params.get("target_budget_ratio", 1.0))
        target = max(1, int(round(int(segment_tokens) * ratio)))
    recent = params.get("recent_size")
    if recent is None:
        recent = int(round(int(target) * float(params.get("recent_budget_fraction", 0.25))))
    return int(target), int(recent)


def clamp_budget(tokens: int, target_tokens: int, recent_tokens: int) -> tuple[int, int, int]:
    """physical.py:511-515: (heavy_k, recent, heavy)."""

    target = min(tokens, max(1, int(target_tokens)))
    recent = min(target, max(0, int(recent_tokens)))
    heavy = target - recent
    history_end = tokens - recent
    return min(heavy, history_end), recent, heavy


def topk_lowest_index(row, k: int) -> np.ndarray:
    """Indices of the k largest entries of a 1-D score row, ties to the
    lowest index, NaN ranked above every number (torch.topk's NaN order),
    returned in ascending index order (physical.py:516-519 with the
    deterministic tie rule)."""

    row = np.asarray(row, dtype=np.float32)
    idx = np.arange(row.shape[0])
    nan = np.isnan(row)
    neg = np.where(nan, 0.0, -row.astype(np.float64))
    order = np.lexsort((idx, neg, ~nan))  # NaN first, then descending score, then index
    return np.sort(order[:k])


def select(scores, heavy_k: int, recent: int) -> np.ndarray:
    """[Hkv, heavy_k + recent]: heavy top-k of the history then the recent
    window (physical.py:516-532)."""

    s = np.asarray(scores, dtype=np.float32)
    heads, tokens = s.shape
    history_end = tokens - recent
    out = np.empty((heads, heavy_k + recent), dtype=np.int64)
    for h in range(heads):
        out[h, :heavy_k] = topk_lowest_index(s[h, :history_end], heavy_k) if heavy_k else []
        out[h, heavy_k:] = np.arange(history_end, tokens)
    return out


def gather(key, value, indices, logical_ids, scores):
    """physical.py:533-546: key/value [T, Hkv, D] -> [Hkv, R, D]; ids and
    scores gathered per head."""

    k = np.asarray(key)
    v = np.asarray(value)
    idx = np.asarray(indices)
    heads = idx.shape[0]
    ok = np.stack([k[idx[h], h] for h in range(heads)])
    ov = np.stack([v[idx[h], h] for h in range(heads)])
    ids = np.asarray(logical_ids)
    oid = np.stack([ids[idx[h]] if ids.ndim == 1 else ids[h, idx[h]] for h in range(heads)])
    osc = np.stack([np.asarray(scores, dtype=np.float32)[h, idx[h]] for h in range(heads)])
    return ok, ov, oid, osc


def from_dense(key, value, logical_ids, scores, target_tokens, recent_tokens):
    """GQAH2OCache.from_dense (physical.py:493-547) -> (key, value, ids,
    cumulative_scores, heavy, recent)."""

    tokens = np.asarray(key).shape[0]
    heavy_k, recent, heavy = clamp_budget(tokens, target_tokens, recent_tokens)
    idx = select(scores, heavy_k, recent)
    ok, ov, oid, osc = gather(key, value, idx, logical_ids, scores)
    return ok, ov, oid, osc, heavy, recent


def trim(key_hrd, value_hrd, ids_hr, scores_hr, target_tokens, recent_tokens):
    """GQAH2OCache.trim (physical.py:624-654) on [Hkv, R, D] storage."""

    retained = key_hrd.shape[1]
    target = min(retained, max(1, int(target_tokens)))
    if target >= retained:
        return key_hrd, value_hrd, ids_hr, scores_hr
    recent = min(target, max(0, int(recent_tokens)))
    heavy = target - recent
    history_end = retained - recent
    heavy_k = min(heavy, history_end) if heavy else 0
    idx = select(scores_hr, heavy_k, recent)
    heads = key_hrd.shape[0]
    take = lambda a: np.stack([a[h, idx[h]] for h in range(heads)])  # noqa: E731
    return take(key_hrd), take(value_hrd), take(ids_hr), take(np.asarray(scores_hr, dtype=np.float32))


def min_selection_margin(scores, heavy_k: int, recent: int) -> float:
    """Smallest gap, over heads, between the heavy_k-th and (heavy_k+1)-th
    largest history score: index equality between two summation orders is
    guaranteed when it exceeds their score difference."""

    s = np.asarray(scores, dtype=np.float64)
    history_end = s.shape[1] - recent
    gaps = []
    for h in range(s.shape[0]):
        row = np.sort(s[h, :history_end])[::-1]
        if 0 < heavy_k < row.shape[0]:
            gaps.append(row[heavy_k - 1] - row[heavy_k])
    return float(min(gaps)) if gaps else math.inf


def compact(key, value, type_ids, sample_lens, keep_masks):
    """tensor_backend.py:54-77: per packed sample, the rows its keep mask
    keeps, samples concatenated in order; returns (key, value, type_ids,
    kept per sample)."""

    k, v = np.asarray(key), np.asarray(value)
    ids = None if type_ids is None else np.asarray(type_ids)
    ok, ov, oi, lens = [], [], [], []
    off = 0
    for n, m in zip(sample_lens, keep_masks):
        m = np.asarray(m, dtype=bool)
        ok.append(k[off:off + n][m])
        ov.append(v[off:off + n][m])
        if ids is not None:
            oi.append(ids[off:off + n][m])
        lens.append(int(m.sum()))
        off += n
    cat = lambda xs, like: np.concatenate(xs) if xs else like[:0]
    return cat(ok, k), cat(ov, v), None if ids is None else cat(oi, ids), lens
