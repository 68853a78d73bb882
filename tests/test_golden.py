"""The known answers of UniCache's own tests (tests/golden/reference_cases.json)
against the oracle (CPU) and the product (GPU)."""

import json
import os

import numpy as np
import pytest
import torch

from oracle import h2o as H
from oracle import kivi as K

CASES = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


def test_oracle_h2o_select_known_answer():
    c = CASES["h2o_select_per_kv_head"]
    scores = np.asarray(c["scores"], dtype=np.float32)
    heavy_k, recent, _ = H.clamp_budget(c["tokens"], c["target_tokens"], c["recent_tokens"])
    idx = H.select(scores, heavy_k, recent)
    assert idx.tolist() == c["expected_ids"]


def test_oracle_split_and_budget_known_answers():
    c = CASES["residual_expansion"]
    assert K.split_tokens(c["tokens"], c["group_size"], c["residual_length"]) == (
        c["quantized_tokens"], c["residual_tokens"])
    for n, target, recent in CASES["h2o_budget_20pct"]:
        assert H.budget(n, {"target_budget_ratio": 0.2}) == (target, recent)


def test_oracle_native_layout_shapes():
    c = CASES["native_layout"]
    rng = np.random.default_rng(0)
    x = rng.standard_normal((c["tokens"], c["kv_heads"], c["head_dim"])).astype(np.float32)
    seg = K.from_dense(x, x, k_bits=c["bits"], v_bits=c["bits"], group_size=c["group_size"],
                       residual_length=c["residual_length"])
    assert list(seg.key_code.shape) == c["key_code"] and list(seg.key_scale.shape) == c["key_scale"]
    assert list(seg.value_code.shape) == c["value_code"] and list(seg.value_scale.shape) == c["value_scale"]


@pytest.mark.gpu
def test_product_known_answers(device):
    from unicache_amd.storage import GQAH2OCache, PackedKIVICache
    from unicache_amd.storage.tensor_backend import h2o_budget

    c = CASES["h2o_select_per_kv_head"]
    key = torch.arange(c["tokens"] * c["kv_heads"] * c["head_dim"], dtype=torch.float32).reshape(
        c["tokens"], c["kv_heads"], c["head_dim"]).to(torch.bfloat16).to(device)
    cache = GQAH2OCache.from_dense(key, key + 1000, logical_token_ids=torch.arange(c["tokens"]), token_type_id=1,
                                   per_kv_head_scores=torch.tensor(c["scores"]).to(device),
                                   target_tokens=c["target_tokens"], recent_tokens=c["recent_tokens"])
    assert cache.logical_token_ids.cpu().tolist() == c["expected_ids"]

    c = CASES["native_layout"]
    g = torch.Generator().manual_seed(6)
    x = torch.randn(c["tokens"], c["kv_heads"], c["head_dim"], generator=g).to(torch.bfloat16).to(device)
    p = PackedKIVICache.from_dense(x, x.clone(), logical_token_ids=torch.arange(c["tokens"]), token_type_id=3,
                                   k_bits=c["bits"], v_bits=c["bits"], group_size=c["group_size"],
                                   residual_length=c["residual_length"], backend="cuda")
    assert p.kernel_native_layout
    assert list(p.key_code.shape) == c["key_code"] and list(p.key_scale.shape) == c["key_scale"]
    assert list(p.value_code.shape) == c["value_code"] and list(p.value_scale.shape) == c["value_scale"]
    assert p.key_scale.dtype == getattr(torch, c["stats_dtype"]) == p.value_scale.dtype

    c = CASES["residual_expansion"]
    x = torch.randn(c["tokens"], c["kv_heads"], c["head_dim"], generator=g).to(torch.bfloat16).to(device)
    p = PackedKIVICache.from_dense(x, x.clone(), logical_token_ids=torch.arange(c["tokens"]), token_type_id=3,
                                   k_bits=c["bits"], v_bits=c["bits"], group_size=c["group_size"],
                                   residual_length=c["residual_length"], backend="cuda")
    assert (p.quantized_tokens, p.residual_tokens) == (c["quantized_tokens"], c["residual_tokens"])
    assert torch.equal(p.dequantize()[0][-c["residual_tokens"]:], x[-c["residual_tokens"]:])

    # test_physical.py:1099-1132 as written: head_dim 16, group 8, the reference backend
    c = CASES["monotonic"]
    x = torch.randn(c["tokens"], c["kv_heads"], c["head_dim"], generator=g).to(torch.bfloat16).to(device)
    k = c["kivi"]
    p = PackedKIVICache.from_dense(x, x.clone(), logical_token_ids=torch.arange(c["tokens"]), token_type_id=3,
                                   k_bits=k["bits"], v_bits=k["bits"], group_size=k["group_size"],
                                   residual_length=k["residual_length"], backend="reference")
    bits, group, ok = k["repack_down"]
    assert p.repack_monotonic(bits=bits, group_size=group) is ok and p.k_bits == bits and p.group_size == group
    bits, group, ok = k["repack_up"]
    assert p.repack_monotonic(bits=bits, group_size=group) is ok
    assert p.budget_shortfall_events == k["shortfall_events"]
    hc = c["h2o"]
    h = GQAH2OCache.from_dense(x, x.clone(), logical_token_ids=torch.arange(c["tokens"]), token_type_id=1,
                               per_kv_head_scores=torch.rand(c["kv_heads"], c["tokens"]).to(device),
                               target_tokens=hc["target_tokens"], recent_tokens=hc["recent_tokens"])
    for target, recent, effective, retained in hc["requests"]:
        assert h.request_budget(target, recent) == effective and h.retained_tokens == retained
    assert h.budget_shortfall_tokens == hc["shortfall_tokens"]
    for n, target, recent in CASES["h2o_budget_20pct"]:
        assert h2o_budget(n, {"target_budget_ratio": 0.2}) == (target, recent)
