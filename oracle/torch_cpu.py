"""torch-CPU restatement of the hot path (KIVI pack / dequantize, GQA
attention, H2O scores, top-k and gather), vectorised over whole tensors.

Test infrastructure, like the rest of oracle/: bench.py times it on the GPU
box's host cores as the CPU baseline, and tests/test_oracle_torch_cpu.py checks
it against the numpy oracle (codes and stats bit-exact, attention to fp32
rounding).  The product path never imports it.

Layouts follow the kernel-native packed cache (kivi_cuda.py:157-190): keys as
[Hkv, D, T] grouped and packed along tokens, values as [Hkv, T, D] grouped and
packed along channels, fp16 stats.
"""

from __future__ import annotations

import math

import torch

EPS = torch.finfo(torch.float32).eps


# ----------------------------------------------------------------- codes --
def quantize_codes(data: torch.Tensor, *, bits: int, group_size: int):
    """physical.py:139-175 along the last dim (a multiple of group_size):
    (codes uint8, scale fp32, minimum fp32), stats [..., L/G].

      mn, mx = amin, amax of the group
      scale  = clamp_min((mx - mn) / (2^b - 1), eps)
      code   = clamp(round((x - mn) / scale), 0, 2^b - 1), NaN -> 0
    """

    x = data.float()
    g = x.reshape(*x.shape[:-1], -1, group_size)
    mn = g.amin(-1, keepdim=True)
    mx = g.amax(-1, keepdim=True)
    max_code = float((1 << bits) - 1)
    scale = ((mx - mn) / max_code).clamp_min(EPS)
    q = torch.round((g - mn) / scale).clamp_(0, max_code)
    codes = torch.nan_to_num(q, nan=0.0).to(torch.uint8).reshape(x.shape)
    return codes, scale.squeeze(-1), mn.squeeze(-1)


def pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """physical.py:66-85 along the last dim: code j of a word at bit j*bits."""

    per = 32 // bits
    c = codes.to(torch.int64).reshape(*codes.shape[:-1], -1, per)
    shifts = torch.arange(per, dtype=torch.int64) * bits
    words = (c << shifts).sum(-1)
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)


def unpack_codes(words: torch.Tensor, bits: int) -> torch.Tensor:
    """physical.py:88-104 along the last dim."""

    per = 32 // bits
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, dtype=torch.int64) * bits
    return ((w.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(*words.shape[:-1], -1)


def dequantize_grouped(words, scale, minimum, *, bits: int, group_size: int, out_dtype=torch.bfloat16):
    """physical.py:178-201 along the last dim: code * scale + minimum in fp32
    (two roundings), then the output cast."""

    codes = unpack_codes(words, bits).float()
    g = codes.reshape(*codes.shape[:-1], -1, group_size)
    out = g * scale.float().unsqueeze(-1) + minimum.float().unsqueeze(-1)
    return out.reshape(codes.shape).to(out_dtype)


# --------------------------------------------------------- packed caches --
def from_dense(key: torch.Tensor, value: torch.Tensor, *, bits: int, group_size: int, residual_length: int):
    """PackedKIVICache.from_dense (physical.py:228-332) into the native layout:
    a dict of the six packed tensors, the residual and the packed length."""

    tokens = int(key.shape[0])
    requested = min(tokens, max(0, int(residual_length)))
    tq = ((tokens - requested) // group_size) * group_size
    kc, ks, km = quantize_codes(key[:tq].permute(1, 2, 0), bits=bits, group_size=group_size)
    vc, vs, vm = quantize_codes(value[:tq].permute(1, 0, 2), bits=bits, group_size=group_size)
    return {
        "key_code": pack_codes(kc, bits), "key_scale": ks.half(), "key_minimum": km.half(),
        "value_code": pack_codes(vc, bits), "value_scale": vs.half(), "value_minimum": vm.half(),
        "residual_key": key[tq:].clone(), "residual_value": value[tq:].clone(),
        "quantized_tokens": tq, "bits": bits, "group_size": group_size,
    }


def dequantize(seg: dict, out_dtype=torch.bfloat16):
    """PackedKIVICache.dequantize (physical.py:379-423): [T, Hkv, D] K and V."""

    b, g = seg["bits"], seg["group_size"]
    key = dequantize_grouped(seg["key_code"], seg["key_scale"], seg["key_minimum"], bits=b, group_size=g,
                             out_dtype=out_dtype).permute(2, 0, 1)
    value = dequantize_grouped(seg["value_code"], seg["value_scale"], seg["value_minimum"], bits=b, group_size=g,
                               out_dtype=out_dtype).permute(1, 0, 2)
    return (torch.cat([key, seg["residual_key"].to(out_dtype)]),
            torch.cat([value, seg["residual_value"].to(out_dtype)]))


def flush(seg: dict, count: int) -> dict:
    """Quantize the first `count` residual tokens (a multiple of the group
    size) and append them to the packed prefix: the streaming flush whose
    result equals from_dense of the flushed prefix."""

    part = from_dense(seg["residual_key"][:count], seg["residual_value"][:count], bits=seg["bits"],
                      group_size=seg["group_size"], residual_length=0)
    out = dict(seg)
    for name, dim in (("key_code", 2), ("key_scale", 2), ("key_minimum", 2), ("value_code", 1),
                      ("value_scale", 1), ("value_minimum", 1)):
        out[name] = torch.cat([seg[name], part[name]], dim=dim)
    out["residual_key"] = seg["residual_key"][count:].clone()
    out["residual_value"] = seg["residual_value"][count:].clone()
    out["quantized_tokens"] = seg["quantized_tokens"] + count
    return out


# ------------------------------------------------------------- attention --
def gqa_logits(query: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """gqa_query_key_logits (physical.py:20-39): [Lq, Hq, D] x [T, Hkv, D] ->
    fp32 [Hq, Lq, T]."""

    lq, hq, d = query.shape
    hkv = key.shape[1]
    q = query.float().permute(1, 0, 2).reshape(hkv, (hq // hkv) * lq, d)
    return torch.bmm(q, key.float().permute(1, 2, 0)).reshape(hq, lq, -1)


def gqa_pv(probs: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """gqa_probability_value (physical.py:42-63): [Hq, Lq, T] x [T, Hkv, D]
    -> fp32 [Hq, Lq, D]."""

    hq, lq, t = probs.shape
    hkv = value.shape[1]
    p = probs.float().reshape(hkv, (hq // hkv) * lq, t)
    return torch.bmm(p, value.float().permute(1, 0, 2)).reshape(hq, lq, -1)


def attention_summary(query, key, value):
    """Softmax attention with the adapter's numerics (fp32 logits and softmax,
    bf16 probabilities; adapters/bagel.py:1205-1297): (out [Lq, Hq, D] fp32,
    natural-log lse [Hq, Lq])."""

    logits = gqa_logits(query, key) / math.sqrt(query.shape[-1])
    lse = torch.logsumexp(logits, dim=-1)
    probs = torch.exp(logits - lse.unsqueeze(-1)).to(torch.bfloat16)
    return gqa_pv(probs, value).permute(1, 0, 2), lse


def packed_decode(seg: dict, query: torch.Tensor):
    """The reference backend's packed attention (physical.py:452-475):
    dequantize the segment, then dense attention over [packed | residual]."""

    key, value = dequantize(seg, query.dtype)
    return attention_summary(query, key, value)


# ------------------------------------------------------------------- H2O --
def h2o_scores(query: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """Per-KV-head H2O scores from the adapter's bf16 probabilities
    (adapters/bagel.py:1205-1243; operators/physical.py:62-65): [Hkv, T]."""

    hkv = key.shape[1]
    logits = gqa_logits(query, key) / math.sqrt(query.shape[-1])
    probs = torch.softmax(logits, dim=-1).to(torch.bfloat16)
    hq, _, t = probs.shape
    return probs.float().sum(1).reshape(hkv, hq // hkv, t).sum(1)


def h2o_select_gather(scores, key, value, *, heavy_k: int, recent: int):
    """physical.py:516-546: heavy top-k of the history plus the recent window
    per KV head, then the gather into [Hkv, R, D] K and V."""

    hkv, t = scores.shape
    history = t - recent
    top = torch.topk(scores[:, :history], heavy_k, dim=-1).indices.sort(dim=-1).values
    window = torch.arange(history, t).expand(hkv, recent)
    idx = torch.cat([top, window], dim=-1)
    heads = torch.arange(hkv).unsqueeze(-1)
    return key[idx, heads], value[idx, heads], idx
