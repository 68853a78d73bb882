"""The first-denoise-step materialisation path on the GPU: the two physical
operators emit PhysicalCacheRequests (operators/physical.py:51-101,
146-178) and TensorCacheStorageBackend.compact_and_materialize turns them
into packed KIVI / H2O segments and compacts the dense remainder
(tensor_backend.py:102-239).  Segments and remainder are compared bit for bit
with the oracle's from_dense / select / gather / compact on the same rows."""

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import h2o as H
from oracle import kivi as K
from tests.helpers import f32, kv_pair, queries
from unicache_amd.core.registry import OperatorExecutionContext
from unicache_amd.operators.physical import H2OPhysicalGQAOperator, KIVIPackedQuantizationOperator
from unicache_amd.storage import GQAH2OCache, PackedKIVICache
from unicache_amd.storage.tensor_backend import TensorCacheStorageBackend

pytestmark = pytest.mark.gpu


def _ctx(op, params, key, value, mask, *, type_id=None, span=None, heads_kv=None):
    records = {}

    def record(values):
        for k, v in values.items():
            records[k] = records.get(k, 0) + v

    meta = {"current_segment_type_id": type_id, "current_segment_span": span}
    ctx = OperatorExecutionContext(
        runtime=SimpleNamespace(kv_metadata=meta), step=SimpleNamespace(segment_id="seg"),
        params=op.build_params(params), q=None, k=key, v=value, attn_mask=None, key_type_ids=None,
        segment_mask=mask, protected_mask=None, state={}, record=record, set_storage_snapshot=lambda _: None,
        storage_num_kv_heads=heads_kv,
    )
    return ctx, records


def _probs(query, key):
    """bf16 softmax of the scaled fp32 logits over every key, [Hq, Lq, T]
    (the adapter's probabilities, adapters/bagel.py:1205-1243)."""

    hq, hkv = int(query.shape[1]), int(key.shape[1])
    q = query.float().permute(1, 0, 2)                                  # [Hq, Lq, D]
    k = key.float().repeat_interleave(hq // hkv, dim=1).permute(1, 2, 0).contiguous()  # [Hq, D, T]
    logits = torch.bmm(q, k) / math.sqrt(query.shape[-1])
    return torch.softmax(logits, dim=-1).to(torch.bfloat16)


def _bits16(t):
    return t.detach().cpu().view(torch.int16).numpy()


def _assert_kivi(seg, key_rows, value_rows, ids, params, *, native):
    bits = params["bits"]
    exp = K.from_dense(f32(key_rows), f32(value_rows), k_bits=bits, v_bits=bits, group_size=params["group_size"],
                       residual_length=params["residual_length"], native=native)
    assert isinstance(seg, PackedKIVICache)
    assert seg.kernel_native_layout == exp.native and seg.quantized_tokens == exp.quantized_tokens
    for name in ("key_code", "value_code"):
        got = getattr(seg, name).cpu().numpy()
        assert np.array_equal(got.view(np.int32) if got.dtype != np.uint8 else got, getattr(exp, name)), name
    for name in ("key_scale", "key_minimum", "value_scale", "value_minimum"):
        assert np.array_equal(f32(getattr(seg, name)), getattr(exp, name)), name
    assert np.array_equal(f32(seg.residual_key), exp.residual_key)
    assert np.array_equal(f32(seg.residual_value), exp.residual_value)
    assert seg.logical_token_ids.cpu().tolist() == list(ids)


def _assert_h2o(seg, key_rows, value_rows, ids, scores, params):
    target, recent = H.budget(len(ids), params)
    ek, ev, eid, esc, heavy, erecent = H.from_dense(_bits16(key_rows), _bits16(value_rows), np.asarray(ids),
                                                    scores, target, recent)
    assert isinstance(seg, GQAH2OCache)
    assert (seg.heavy_tokens, seg.recent_tokens) == (heavy, erecent)
    assert np.array_equal(_bits16(seg.key), ek) and np.array_equal(_bits16(seg.value), ev)
    assert np.array_equal(seg.logical_token_ids.cpu().numpy(), eid)
    assert np.array_equal(seg.cumulative_scores.cpu().numpy(), esc)


def test_h2o_request_reference_counts(device):
    # test_physical.py:1217-1270: 16 tokens (12 instruction of type 1, 4 of
    # type 4), 2 KV heads, head_dim 8, ratio 0.5 -> 6 retained, 4 left dense
    torch.manual_seed(2)
    key = torch.randn(16, 2, 8, dtype=torch.bfloat16)
    value = torch.randn_like(key)
    types = torch.tensor([1] * 12 + [4] * 4)
    query = torch.randn(3, 4, 8, dtype=torch.bfloat16)
    key_d, value_d, types_d = key.to(device), value.to(device), types.to(device)
    op = H2OPhysicalGQAOperator()
    params = {"target_budget_ratio": 0.5, "recent_budget_fraction": 0.25, "selection_frozen": True}
    ctx, records = _ctx(op, params, key_d, value_d, types_d == 1, type_id=1, span=(0, 12), heads_kv=2)
    probs = _probs(query.to(device), key_d)
    op.update_after_attention(ctx, probs)
    request = ctx.physical_request
    assert request.operator == "h2o_physical_gqa" and request.token_count == 16
    assert records == {"physical_h2o_requests": 1, "physical_h2o_source_tokens": 12,
                       "physical_h2o_target_tokens_per_kv_head": 6}
    scores = request.per_kv_head_scores.cpu().numpy()
    exp_scores = H.scores_from_probs(f32(probs), 2)
    assert np.abs(scores - exp_scores).max() <= 1e-5 * max(1.0, float(np.abs(exp_scores).max()))
    keep = [torch.ones(16, dtype=torch.bool, device=device)]
    mutation = TensorCacheStorageBackend.compact_and_materialize(
        key=key_d, value=value_d, key_type_ids=types_d, sample_lens=torch.tensor([16], device=device),
        keep_masks=keep, physical_requests=[[request]])
    assert mutation.key.shape[0] == 4
    h2o = mutation.physical_segments_by_sample[0][0]
    assert isinstance(h2o, GQAH2OCache)
    assert h2o.token_type_id == 1 and h2o.retained_tokens == 6 and h2o.selection_frozen
    _assert_h2o(h2o, key[:12], value[:12], range(12), scores[:, :12], ctx.params)
    assert torch.equal(mutation.key.cpu(), key[12:]) and torch.equal(mutation.value.cpu(), value[12:])
    assert mutation.key_type_ids.cpu().tolist() == [4] * 4 and mutation.sample_lens.cpu().tolist() == [4]
    assert keep[0].cpu().tolist() == [False] * 12 + [True] * 4  # the caller's mask is updated in place


def test_two_samples_spans_masks_and_type_recovery(device):
    # sample 0: instruction [0, 100) -> H2O (span), VAE [100, 500) -> KIVI
    #           2-bit (span), text [500, 600) stays dense
    # sample 1: KIVI over the tokens t % 3 != 0 of [0, 300) and H2O over
    #           t % 3 == 0 (masks only, type ids recovered from the cache), the
    #           rest dense with tokens 320..322 dropped by the keep mask
    lens = [600, 333]
    key, value = kv_pair(sum(lens), seed=11)
    types = torch.cat([torch.full((100,), 1), torch.full((400,), 3), torch.zeros(100, dtype=torch.long),
                       torch.full((300,), 3), torch.zeros(33, dtype=torch.long)])
    pos1 = torch.arange(333)
    types[600:900][pos1[:300] % 3 == 0] = 1
    types[600:900][(pos1[:300] % 3 == 0) & (pos1[:300] % 2 == 0)] = 2  # H2O rows of two types: no recovery
    key_d, value_d, types_d = key.to(device), value.to(device), types.to(device)
    kivi, h2o = KIVIPackedQuantizationOperator(), H2OPhysicalGQAOperator()
    kivi_params = {"bits": 2, "group_size": 32, "residual_length": 128}
    h2o_params = {"target_budget_ratio": 0.2, "recent_budget_fraction": 0.25}

    requests, expected = [[], []], [[], []]
    # sample 0
    k0, v0 = key_d[:600], value_d[:600]
    span_mask = lambda a, b, n: (torch.arange(n, device=device) >= a) & (torch.arange(n, device=device) < b)  # noqa
    ctx, _ = _ctx(h2o, h2o_params, k0, v0, span_mask(0, 100, 600), type_id=1, span=(0, 100), heads_kv=4)
    q0 = queries(64, seed=12).to(device)
    h2o.update_after_attention(ctx, _probs(q0, k0))
    requests[0].append(ctx.physical_request)
    ctx, rec = _ctx(kivi, kivi_params, k0, v0, span_mask(100, 500, 600), type_id=3, span=(100, 500))
    kivi.execute(ctx)
    assert rec["physical_kivi_quantized_tokens"] == 400 - 128 and ctx.params["backend"] == "cuda"
    requests[0].append(ctx.physical_request)
    # sample 1
    k1, v1 = key_d[600:], value_d[600:]
    kmask = (torch.arange(333, device=device) < 300) & (torch.arange(333, device=device) % 3 != 0)
    hmask = (torch.arange(333, device=device) < 300) & (torch.arange(333, device=device) % 3 == 0)
    ctx, _ = _ctx(kivi, kivi_params, k1, v1, kmask)
    kivi.execute(ctx)
    requests[1].append(ctx.physical_request)
    ctx, _ = _ctx(h2o, h2o_params, k1, v1, hmask, heads_kv=4)
    h2o.update_after_attention(ctx, _probs(queries(16, seed=13).to(device), k1))
    requests[1].append(ctx.physical_request)

    keep = [torch.ones(600, dtype=torch.bool), torch.ones(333, dtype=torch.bool)]
    keep[1][320:323] = False
    keep_d = [m.to(device) for m in keep]
    mutation = TensorCacheStorageBackend.compact_and_materialize(
        key=key_d, value=value_d, key_type_ids=types_d, sample_lens=torch.tensor(lens, device=device),
        keep_masks=keep_d, physical_requests=requests)

    segs0, segs1 = mutation.physical_segments_by_sample
    sc0 = requests[0][0].per_kv_head_scores.cpu().numpy()
    _assert_h2o(segs0[0], key[:100], value[:100], range(100), sc0[:, :100], h2o.build_params(h2o_params))
    assert segs0[0].token_type_id == 1 and segs0[0].retained_tokens == 20
    kp = kivi.build_params(kivi_params)
    _assert_kivi(segs0[1], key[100:500], value[100:500], range(100, 500), kp, native=True)
    assert segs0[1].token_type_id == 3
    kidx = [t for t in range(300) if t % 3]
    hidx = [t for t in range(300) if t % 3 == 0]
    _assert_kivi(segs1[0], key[600:][kidx], value[600:][kidx], kidx, kp, native=True)
    assert segs1[0].token_type_id == 3  # recovered: every row of the mask has type 3
    sc1 = requests[1][1].per_kv_head_scores.cpu().numpy()
    _assert_h2o(segs1[1], key[600:][hidx], value[600:][hidx], hidx, sc1[:, hidx], h2o.build_params(h2o_params))
    assert segs1[1].token_type_id == -1  # rows of types 1 and 2: no single type

    occupied = [np.arange(600) < 500, np.arange(333) < 300]
    final = [keep[0].numpy() & ~occupied[0], keep[1].numpy() & ~occupied[1]]
    ek, ev, ei, elens = H.compact(_bits16(key), _bits16(value), types.numpy(), lens, final)
    assert np.array_equal(_bits16(mutation.key), ek) and np.array_equal(_bits16(mutation.value), ev)
    assert np.array_equal(mutation.key_type_ids.cpu().numpy(), ei)
    assert mutation.sample_lens.cpu().tolist() == elens == [100, 30]
    assert [m.cpu().numpy().tolist() for m in keep_d] == [f.tolist() for f in final]


def test_reference_backend_request(device):
    # a request with backend "reference" (UniCache's default layout: codes
    # along tokens / channels, stats in the input dtype), 4-bit G=64 R=32
    key, value = kv_pair(300, seed=21)
    key_d, value_d = key.to(device), value.to(device)
    op = KIVIPackedQuantizationOperator()
    params = {"bits": 4, "group_size": 64, "backend": "reference"}
    mask = torch.ones(300, dtype=torch.bool, device=device)
    ctx, _ = _ctx(op, params, key_d, value_d, mask, type_id=3, span=(0, 300))
    op.execute(ctx)
    mutation = TensorCacheStorageBackend.compact_and_materialize(
        key=key_d, value=value_d, key_type_ids=None, sample_lens=torch.tensor([300], device=device),
        keep_masks=[torch.ones(300, dtype=torch.bool, device=device)], physical_requests=[[ctx.physical_request]])
    seg = mutation.physical_segments_by_sample[0][0]
    assert seg.backend == "reference" and not seg.kernel_native_layout
    assert seg.key_scale.dtype == torch.bfloat16 and tuple(seg.key_code.shape) == (256 * 4 // 32, 4, 128)
    _assert_kivi(seg, key, value, range(300), op.build_params(params), native=False)
    assert mutation.key.shape[0] == 0
    # attention_parts of the reference backend: dequantize, then QK / PV
    q = queries(5, seed=22).to(device)
    logits, apply_value = seg.attention_parts(q)
    exp = K.from_dense(f32(key), f32(value), k_bits=4, v_bits=4, group_size=64, residual_length=32, native=False)
    el = A.packed_logits(exp, f32(q))
    assert np.abs(f32(logits) - el).max() <= 2e-2
    probs = torch.softmax(logits, dim=-1)
    out = apply_value(probs)
    eo = A.packed_pv(exp, f32(probs))
    assert np.abs(f32(out) - eo).max() <= 2e-2


def _request(operator, mask, *, span=None, scores=None, params=None):
    from unicache_amd.core.decisions import PhysicalCacheRequest

    return PhysicalCacheRequest(operator=operator, segment_id="s", token_count=int(mask.numel()),
                                segment_mask=mask, params=params or {"bits": 2, "group_size": 32},
                                per_kv_head_scores=scores, metadata={"token_span": span})


def test_materialize_errors_leave_masks_untouched(device):
    key, value = kv_pair(64, seed=5)
    key_d, value_d = key.to(device), value.to(device)
    ar = torch.arange(32, device=device)
    m_lo, m_mid = ar < 16, (ar >= 8) & (ar < 24)
    keep = [torch.ones(32, dtype=torch.bool, device=device), torch.ones(32, dtype=torch.bool, device=device)]

    def run(requests):
        return TensorCacheStorageBackend.compact_and_materialize(
            key=key_d, value=value_d, key_type_ids=None, sample_lens=torch.tensor([32, 32], device=device),
            keep_masks=keep, physical_requests=requests)

    kv = "kivi_packed_quantization"
    ok = [_request(kv, ar < 32, span=(0, 32))]
    with pytest.raises(ValueError, match="Overlapping physical requests in sample 1"):
        run([ok, [_request(kv, m_lo), _request(kv, m_mid)]])
    with pytest.raises(ValueError, match="outside its packed sample"):
        run([ok, [_request(kv, m_lo, span=(16, 40))]])
    with pytest.raises(ValueError, match="outside its packed sample"):
        run([ok, [_request(kv, m_lo, span=(5, 5))]])
    with pytest.raises(ValueError, match="pair"):
        run([ok, [_request(kv, m_lo, span=(0, 4, 8))]])
    with pytest.raises(ValueError, match="shorter than"):
        run([ok, [_request(kv, torch.ones(20, dtype=torch.bool, device=device))]])
    with pytest.raises(ValueError, match="Unknown physical cache request"):
        run([ok, [_request("snapkv", m_lo)]])
    with pytest.raises(ValueError, match="missing per-KV-head scores"):
        run([ok, [_request("h2o_physical_gqa", m_lo)]])
    with pytest.raises(ValueError, match="one list per packed sample"):
        run([ok])
    assert all(bool(m.all()) for m in keep)
    # an empty mask-only request builds nothing; disjoint requests go through
    res = run([ok, [_request(kv, ar < 0), _request(kv, m_lo)]])
    assert [len(s) for s in res.physical_segments_by_sample] == [1, 1]
    assert res.sample_lens.cpu().tolist() == [0, 16]
