"""The torch-CPU restatement that bench.py times as the CPU baseline, checked
against the numpy oracle: packed codes and fp16 stats bit-exact, dequantized
K/V bit-exact, attention and H2O scores to fp32 rounding, selection equal."""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import h2o as H
from oracle import kivi as K
from oracle import torch_cpu as T
from tests.helpers import f32, kv_pair, queries


@pytest.mark.parametrize("bits,group,tokens,residual", [(2, 32, 2048, 128), (4, 64, 640, 100), (2, 128, 512, 0)])
def test_pack_and_dequantize_match_oracle(bits, group, tokens, residual):
    key, value = kv_pair(tokens, seed=bits + group)
    seg = T.from_dense(key, value, bits=bits, group_size=group, residual_length=residual)
    ref = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=group, residual_length=residual)
    assert seg["quantized_tokens"] == ref.quantized_tokens
    for name in ("key_code", "value_code"):
        assert np.array_equal(seg[name].numpy().view(np.uint32), getattr(ref, name).view(np.uint32)), name
    for name in ("key_scale", "key_minimum", "value_scale", "value_minimum"):
        assert np.array_equal(f32(seg[name]), getattr(ref, name)), name
    dk, dv = T.dequantize(seg)
    rk, rv = K.dequantize(ref, "bf16")
    assert np.array_equal(f32(dk), rk) and np.array_equal(f32(dv), rv)


def test_flush_equals_packing_the_prefix():
    key, value = kv_pair(1024, seed=5)
    first = T.from_dense(key[:768], value[:768], bits=2, group_size=32, residual_length=256)
    flushed = T.flush(first, 128)
    whole = T.from_dense(key[:768], value[:768], bits=2, group_size=32, residual_length=128)
    assert flushed["quantized_tokens"] == whole["quantized_tokens"] == 640
    for name in ("key_code", "key_scale", "key_minimum", "value_code", "value_scale", "value_minimum",
                 "residual_key", "residual_value"):
        assert torch.equal(flushed[name], whole[name]), name


def test_attention_and_decode_match_oracle():
    key, value = kv_pair(1000, seed=7)
    q = queries(3, seed=8)
    out, lse = T.attention_summary(q, key, value)
    eo, el = A.attention_summary(f32(q), f32(key), f32(value))
    # bf16 probabilities (the adapter's cast) against the oracle's fp64 softmax
    assert np.abs(out.numpy() - eo).max() < 2e-2 and np.abs(out.numpy() - eo).mean() < 1e-3
    assert np.abs(lse.numpy() - el).max() < 1e-4
    seg = T.from_dense(key, value, bits=2, group_size=32, residual_length=128)
    ref = K.from_dense(f32(key), f32(value), k_bits=2, v_bits=2, group_size=32, residual_length=128)
    out, lse = T.packed_decode(seg, q)
    eo, el = A.packed_summary(ref, f32(q))
    assert np.abs(out.numpy() - eo).max() < 2e-2 and np.abs(lse.numpy() - el).max() < 1e-4


def test_h2o_scores_select_gather_match_oracle():
    key, value = kv_pair(512, seed=11, outliers=0)
    q = queries(64, seed=12)
    got = T.h2o_scores(q, key)
    exp = H.scores_from_qk(f32(q), f32(key))
    assert np.abs(got.numpy() - exp).max() < 1e-4
    heavy_k, recent, _ = H.clamp_budget(512, 100, 25)
    k, v, idx = T.h2o_select_gather(torch.from_numpy(exp), key, value, heavy_k=heavy_k, recent=recent)
    ref_idx = H.select(exp, heavy_k, recent)
    assert np.array_equal(idx.numpy(), ref_idx)
    ok, ov, _, _ = H.gather(f32(key), f32(value), ref_idx, np.arange(512), exp)
    assert np.array_equal(f32(k), ok) and np.array_equal(f32(v), ov)
