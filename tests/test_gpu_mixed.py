"""GPU parity of mixed-segment attention (_run_fused_mixed_attention,
adapters/bagel.py:1598-1858): dense + H2O + packed segments in one call
against the fp32 oracle softmax over the concatenated (dequantized) keys, and
the H2O update against exp(logit - global LSE) rounded to bf16."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import h2o as H
from oracle import kivi as K
from oracle.kivi import round_bf16
from tests.helpers import assert_close, f32, kv_pair, queries
from unicache_amd.adapters.bagel import run_fused_mixed_attention
from unicache_amd.storage import GQAH2OCache, PackedKIVICache

pytestmark = pytest.mark.gpu


def _segments(device, *, second_packed):
    dk, dv = kv_pair(64, seed=21)
    hk, hv = kv_pair(300, seed=22)
    h2o_live = GQAH2OCache.from_dense(hk.to(device), hv.to(device), logical_token_ids=torch.arange(300),
                                      token_type_id=1, per_kv_head_scores=torch.rand(4, 300).to(device),
                                      target_tokens=60, recent_tokens=15)
    fk, fv = kv_pair(200, seed=23)
    h2o_frozen = GQAH2OCache.from_dense(fk.to(device), fv.to(device), logical_token_ids=torch.arange(200),
                                        token_type_id=2, per_kv_head_scores=torch.rand(4, 200).to(device),
                                        target_tokens=40, recent_tokens=10, selection_frozen=True)
    pk, pv = kv_pair(1000, seed=24)
    packed = [PackedKIVICache.from_dense(pk.to(device), pv.to(device), logical_token_ids=torch.arange(1000),
                                         token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=128,
                                         backend="cuda")]
    segs = [K.from_dense(f32(pk), f32(pv), k_bits=2, v_bits=2, group_size=32, residual_length=128)]
    if second_packed:
        # "mixed": a 4-bit / group-64 prefix (its own pass); "same": a second
        # 2-bit / group-32 prefix (both prefixes in one batched launch when the
        # queries are long)
        bits, group, resid = (4, 64, 32) if second_packed == "mixed" else (2, 32, 128)
        sk, sv = kv_pair(700, seed=25)
        packed.append(PackedKIVICache.from_dense(sk.to(device), sv.to(device), logical_token_ids=torch.arange(700),
                                                 token_type_id=4, k_bits=bits, v_bits=bits, group_size=group,
                                                 residual_length=resid, backend="cuda"))
        segs.append(K.from_dense(f32(sk), f32(sv), k_bits=bits, v_bits=bits, group_size=group,
                                 residual_length=resid))
    return (dk, dv), [h2o_live, h2o_frozen], packed, segs


def _oracle_keys(dense, h2o, segs):
    """[dense, H2O..., residuals...] then the packed prefixes: one softmax over
    all of them is what the LSE merge of UniCache's segments computes."""

    ks, vs = [f32(dense[0])], [f32(dense[1])]
    for s in h2o:
        ks.append(np.transpose(f32(s.key), (1, 0, 2)))
        vs.append(np.transpose(f32(s.value), (1, 0, 2)))
    for seg in segs:
        ks.append(np.asarray(seg.residual_key, dtype=np.float32))
        vs.append(np.asarray(seg.residual_value, dtype=np.float32))
    for seg in segs:
        k, v = K.dequantize(seg, "fp32")
        ks.append(k[: seg.quantized_tokens])
        vs.append(v[: seg.quantized_tokens])
    return np.concatenate(ks), np.concatenate(vs)


@pytest.mark.parametrize("lq", [1, 40])
@pytest.mark.parametrize("second_packed", [None, "mixed", "same"])
def test_mixed_attention_matches_global_softmax(device, lq, second_packed):
    dense, h2o, packed, segs = _segments(device, second_packed=second_packed)
    q = queries(lq, seed=30 + lq)
    live = h2o[0]
    before = live.cumulative_scores.clone().cpu().numpy()
    live_key = np.transpose(f32(live.key), (1, 0, 2))
    ek, ev = _oracle_keys(dense, h2o, segs)
    eo, el = A.attention_summary(f32(q), ek, ev)
    out, lse = run_fused_mixed_attention(q.to(device), dense[0].to(device), dense[1].to(device),
                                         [*h2o, *packed], return_lse=True)
    assert out.shape == (lq, 28, 128) and out.dtype == torch.bfloat16
    assert_close(f32(out), eo, what="mixed out")
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what="mixed lse")
    # the live H2O segment received bf16(exp(logit - global lse)) per retained key
    logits = A.gqa_logits(f32(q), live_key) / math.sqrt(128)
    probs = round_bf16(np.exp(logits - f32(lse)[:, :, None]).astype(np.float32))
    expect = before + H.scores_from_probs(probs, 4)
    got = live.cumulative_scores.cpu().numpy()
    assert np.abs(got - expect).max() <= 2e-3 * max(1.0, float(np.abs(expect).max()))
    # the frozen one is untouched
    assert h2o[1].retained_tokens == 40


@pytest.mark.parametrize("lq", [1, 2])
def test_decode_length_mixed_attention_reads_segments_in_place(device, lq):
    # decode-length queries go to the split-K decode kernels over the segments
    # where they lie: the dense KV, both H2O segments through their [Hkv, R, D]
    # strides, two packed prefixes with their residuals -- no concatenation
    from unittest import mock

    from unicache_amd.storage.kivi_cuda import decode_segments_summary

    dense, h2o, packed, segs = _segments(device, second_packed="same")
    for s in h2o:
        s.selection_frozen = True
    q = queries(lq, seed=60 + lq)
    ek, ev = _oracle_keys(dense, h2o, segs)
    eo, el = A.attention_summary(f32(q), ek, ev)
    dk, dv, qd = dense[0].to(device), dense[1].to(device), q.to(device)
    with mock.patch("torch.cat", side_effect=AssertionError("concatenated")):
        out, lse = run_fused_mixed_attention(qd, dk, dv, [*h2o, *packed], return_lse=True)
    assert_close(f32(out), eo, what=f"decode mixed out Lq {lq}")
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what=f"decode mixed lse Lq {lq}")
    # the same call through the function itself, with a head-major part
    parts = [(dk, dv)] + [(s.key.transpose(0, 1), s.value.transpose(0, 1)) for s in h2o]
    o2, l2 = decode_segments_summary(packed, qd, parts)
    assert torch.equal(o2, out) and torch.equal(l2, lse)
    with pytest.raises(ValueError):
        decode_segments_summary(packed, qd, parts + [(dk.float(), dv.float())])


def test_mixed_attention_requires_packed(device):
    dk, dv = kv_pair(16, seed=1)
    with pytest.raises(RuntimeError):
        run_fused_mixed_attention(queries(1).to(device), dk.to(device), dv.to(device), [])


def test_segment_table_decode_matches_global_softmax(device):
    # group 0: packed + dense; group 1: packed only (padded to two segments);
    # group 2: two packed segments and no dense one
    from unicache_amd.storage.decode import MixedDecodeBatch

    def packed(tokens, seed):
        k, v = kv_pair(tokens, seed=seed)
        c = PackedKIVICache.from_dense(k.to(device), v.to(device), logical_token_ids=torch.arange(tokens),
                                       token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=128,
                                       backend="cuda")
        return c, K.from_dense(f32(k), f32(v), k_bits=2, v_bits=2, group_size=32, residual_length=128)

    (c0, s0), (c1, s1), (c2, s2), (c3, s3) = packed(2200, 41), packed(700, 42), packed(1500, 43), packed(300, 44)
    dk, dv = kv_pair(333, seed=45)
    groups = [[c0, (dk.to(device), dv.to(device))], [c1], [c2, c3]]
    qs = [queries(1, seed=50 + i).to(device) for i in range(3)]
    batch = MixedDecodeBatch(groups, qs)

    def check(expect_segs, dense, i):
        ks, vs = [], []
        for seg in expect_segs:
            k, v = K.dequantize(seg, "fp32")
            ks.append(k)
            vs.append(v)
        if dense is not None:
            ks.append(f32(dense[0]))
            vs.append(f32(dense[1]))
        eo, el = A.attention_summary(f32(qs[i]), np.concatenate(ks), np.concatenate(vs))
        assert_close(f32(batch.outputs[i]), eo, what=f"group {i} out")
        assert_close(f32(batch.lses[i]), el, max_abs=1e-2, mean_abs=1e-3, what=f"group {i} lse")

    batch.run()
    check([s0], (dk, dv), 0)
    check([s1], None, 1)
    check([s2, s3], None, 2)
    # a streaming append to group 1's residual, then refresh
    nk, nv = kv_pair(5, seed=46)
    c1.append(nk.to(device), nv.to(device), logical_token_ids=torch.arange(700, 705))
    with pytest.raises(RuntimeError, match="refresh"):  # the table still points at the old residual
        batch.run()
    batch.refresh()
    batch.run()
    s1.residual_key = np.concatenate([s1.residual_key, f32(nk)])
    s1.residual_value = np.concatenate([s1.residual_value, f32(nv)])
    check([s1], None, 1)


def test_batched_physical_attention_per_sample_softmax(device):
    # apply_static_physical_attention_batch (adapters/bagel.py:773-980): four
    # varlen samples (CFG branches) over frozen layouts -- mixed with a long and
    # a one-token query, H2O-only (dense pass) with both query lengths
    from unicache_amd.adapters import run_batched_physical_attention

    ak, av = kv_pair(300, seed=41)
    h2o_a = GQAH2OCache.from_dense(ak.to(device), av.to(device), logical_token_ids=torch.arange(300), token_type_id=1,
                                   per_kv_head_scores=torch.rand(4, 300).to(device), target_tokens=60,
                                   recent_tokens=15, selection_frozen=True)
    bk, bv = kv_pair(200, seed=42)
    h2o_b = GQAH2OCache.from_dense(bk.to(device), bv.to(device), logical_token_ids=torch.arange(200), token_type_id=2,
                                   per_kv_head_scores=torch.rand(4, 200).to(device), target_tokens=50,
                                   recent_tokens=10, selection_frozen=True)
    pk, pv = kv_pair(1000, seed=43)
    packed = PackedKIVICache.from_dense(pk.to(device), pv.to(device), logical_token_ids=torch.arange(1000),
                                        token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=128,
                                        backend="cuda")
    seg = K.from_dense(f32(pk), f32(pv), k_bits=2, v_bits=2, group_size=32, residual_length=128)
    layouts = [([h2o_a, packed], [seg]), ([h2o_b], []), ([h2o_b], []), ([packed], [seg])]
    q_lens, k_lens = [40, 1, 40, 1], [64, 16, 32, 8]
    q = queries(sum(q_lens), seed=44)
    k, v = kv_pair(sum(k_lens), seed=45)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)])
    cu_k = np.concatenate([[0], np.cumsum(k_lens)])
    out = run_batched_physical_attention(q.to(device), k.to(device), v.to(device), torch.tensor(cu_q).to(device),
                                         torch.tensor(cu_k).to(device), [lay[0] for lay in layouts])
    assert out.shape == (sum(q_lens), 28, 128) and out.dtype == torch.bfloat16
    for i, (segments, segs) in enumerate(layouts):
        h2o = [s for s in segments if isinstance(s, GQAH2OCache)]
        dense = (k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]])
        ek, ev = _oracle_keys(dense, h2o, segs)
        eo, _ = A.attention_summary(f32(q[cu_q[i]:cu_q[i + 1]]), ek, ev)
        assert_close(f32(out[cu_q[i]:cu_q[i + 1]]), eo, what=f"sample {i}")
    with pytest.raises(ValueError):
        run_batched_physical_attention(q.to(device), k.to(device), v.to(device), cu_q[:-1], cu_k,
                                       [lay[0] for lay in layouts[:-1]])


def test_batched_packed_launch_matches_per_sample_passes(device):
    # samples with a packed prefix plus dense keys share one table launch per 8
    # (uc_kivi_attn_mq_table); the results equal one segment-table call per
    # sample over the same segments bit for bit.  Ten samples: two launches for the
    # 2-bit / group-32 caches (chunks of 8 and 1) and one for the 4-bit /
    # group-64 cache; ragged query and current-key lengths.
    from unicache_amd.adapters import run_batched_physical_attention
    from unicache_amd.storage.kivi_cuda import packed_segments_summary

    caches = []
    for j, (n, bits, group) in enumerate([(1000, 2, 32), (600, 2, 32), (1100, 4, 64)]):
        ck, cv = kv_pair(n, seed=60 + j)
        caches.append(PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(n),
                                                 token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                                 residual_length=128, backend="cuda"))
    pick = [0, 1, 0, 2, 1, 0, 0, 1, 0, 1]
    q_lens = [40, 300, 3, 129, 64, 200, 17, 96, 250, 5]
    k_lens = [64, 0, 16, 128, 31, 200, 8, 100, 1, 77]
    q = queries(sum(q_lens), seed=70).to(device)
    k, v = (x.to(device) for x in kv_pair(sum(k_lens), seed=71))
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).tolist()
    out = run_batched_physical_attention(q, k, v, cu_q, cu_k, [[caches[c]] for c in pick])
    for i, c in enumerate(pick):
        q_i = q[cu_q[i]:cu_q[i + 1]]
        if q_i.shape[0] * 7 <= 16:  # decode-length samples take the fused decode pass
            continue
        want, _ = packed_segments_summary([caches[c]], q_i, [(k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]])])
        assert torch.equal(out[cu_q[i]:cu_q[i + 1]], want), f"sample {i}"


def test_batched_table_with_several_prefixes_per_sample(device):
    # five long-query samples, each over two packed prefixes, an H2O segment and
    # its own current keys: ten prefixes exceed one table launch (8 per call),
    # so the batch runs as two launches; every sample is one softmax over all of
    # its segments (one cache without a residual window), compared with the oracle
    from unicache_amd.adapters import run_batched_physical_attention

    caches, segs = [], []
    for j, n in enumerate((640, 1000, 480)):
        ck, cv = kv_pair(n, seed=90 + j)
        caches.append(PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(n),
                                                 token_type_id=3, k_bits=2, v_bits=2, group_size=32,
                                                 residual_length=128 if j != 1 else 0, backend="cuda"))
        segs.append(K.from_dense(f32(ck), f32(cv), k_bits=2, v_bits=2, group_size=32,
                                 residual_length=128 if j != 1 else 0))
    hk, hv = kv_pair(300, seed=95)
    h2o = GQAH2OCache.from_dense(hk.to(device), hv.to(device), logical_token_ids=torch.arange(300), token_type_id=1,
                                 per_kv_head_scores=torch.rand(4, 300).to(device), target_tokens=60,
                                 recent_tokens=15, selection_frozen=True)
    picks = [(0, 1), (2, 0), (1, 2), (0, 2), (1, 0)]
    q_lens, k_lens = [40, 130, 17, 64, 200], [64, 0, 33, 128, 7]
    q = queries(sum(q_lens), seed=96)
    k, v = kv_pair(sum(k_lens), seed=97)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)])
    cu_k = np.concatenate([[0], np.cumsum(k_lens)])
    layouts = [[h2o, caches[a], caches[b]] for a, b in picks]
    out = run_batched_physical_attention(q.to(device), k.to(device), v.to(device), torch.tensor(cu_q).to(device),
                                         torch.tensor(cu_k).to(device), layouts)
    for i, (a, b) in enumerate(picks):
        dense = (k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]])
        ek, ev = _oracle_keys(dense, [h2o], [segs[a], segs[b]])
        eo, _ = A.attention_summary(f32(q[cu_q[i]:cu_q[i + 1]]), ek, ev)
        assert_close(f32(out[cu_q[i]:cu_q[i + 1]]), eo, what=f"sample {i}")


def test_table_launch_writes_each_querys_lse(device):
    # uc_kivi_attn_mq_table with an LSE per query: two queries of different
    # lengths over their own prefixes and dense parts in one launch equal one
    # segment-table call each, outputs and natural-log LSEs bit for bit
    from unicache_amd.storage.kivi_cuda import packed_segments_summary, packed_table_summaries

    caches = []
    for j, n in enumerate((700, 1000)):
        ck, cv = kv_pair(n, seed=110 + j)
        caches.append(PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(n),
                                                 token_type_id=3, k_bits=2, v_bits=2, group_size=32,
                                                 residual_length=128, backend="cuda"))
    entries, wants = [], []
    for i, (lq, nd, picks) in enumerate([(96, 150, (0,)), (300, 64, (1, 0))]):
        q = queries(lq, seed=120 + i).to(device)
        k, v = (x.to(device) for x in kv_pair(nd, seed=130 + i))
        segs = [caches[c] for c in picks]
        wants.append(packed_segments_summary(segs, q, [(k, v)]))
        out = torch.empty_like(q)
        lse = torch.empty(q.shape[1], lq, dtype=torch.float32, device=device)
        entries.append((q, out, lse, segs, [(k, v)]))
    packed_table_summaries(entries, dense_dtype=torch.bfloat16)
    for i, ((_, out, lse, _, _), (want_o, want_l)) in enumerate(zip(entries, wants)):
        assert torch.equal(out, want_o), f"query {i} output"
        assert torch.equal(lse, want_l), f"query {i} lse"


def test_segment_table_matches_separate_passes(device):
    # two packed prefixes with long queries: one segment-table launch (both
    # prefixes, both residuals and the dense keys read in place) against one
    # pass per prefix plus the LSE merge, and both against the oracle
    from unicache_amd.adapters.bagel import merge_attention_summaries
    from unicache_amd.storage.kivi_cuda import packed_kivi_quantized_attention_summary, packed_summary_with_dense

    segments, segs = [], []
    for j, n in enumerate((1000, 700)):
        ck, cv = kv_pair(n, seed=80 + j)
        segments.append(PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(n),
                                                   token_type_id=3, k_bits=2, v_bits=2, group_size=32,
                                                   residual_length=128, backend="cuda"))
        segs.append(K.from_dense(f32(ck), f32(cv), k_bits=2, v_bits=2, group_size=32, residual_length=128))
    q = queries(150, seed=82).to(device)
    dk, dv = (x.to(device) for x in kv_pair(90, seed=83))
    out, lse = run_fused_mixed_attention(q, dk, dv, segments, return_lse=True)
    keys = torch.cat([dk] + [s.residual_key for s in segments if s.residual_tokens], dim=0)
    values = torch.cat([dv] + [s.residual_value for s in segments if s.residual_tokens], dim=0)
    parts = [packed_summary_with_dense(segments[0], q, keys, values),
             packed_kivi_quantized_attention_summary(segments[1], q)]
    want, want_lse = merge_attention_summaries(parts)
    assert_close(f32(out), f32(want), what="table vs passes")
    assert_close(f32(lse), f32(want_lse), max_abs=1e-2, mean_abs=1e-3, what="table vs passes lse")
    ek, ev = _oracle_keys((dk, dv), [], segs)
    eo, el = A.attention_summary(f32(q), ek, ev)
    assert_close(f32(out), eo, what="table out")
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what="table lse")


@pytest.mark.parametrize("bits,group,dtype,lq", [(2, 32, torch.bfloat16, 1088), (4, 32, torch.bfloat16, 1088),
                                                 (2, 64, torch.float16, 257), (4, 128, torch.bfloat16, 257)])
def test_segment_table_editing_layout(device, bits, group, dtype, lq):
    # config 2's editing layout through uc_kivi_attn_mq_segments: 1088 (or 257) queries
    # over the source-VAE cache (packed prefix + residual), a second packed
    # prefix whose last tile is half full, the 256 instruction tokens
    # ([T, Hkv, D]) and 1024 ViT tokens held as [Hkv, T, D] (read through their
    # strides), against the fp32 oracle softmax over all of them
    from unicache_amd.storage.kivi_cuda import packed_segments_summary

    caches, segs = [], []
    for j, (n, resid) in enumerate(((1024, 128), (group * 11 + 40, 40))):
        ck, cv = kv_pair(n, seed=120 + j, dtype=dtype)
        caches.append(PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(n),
                                                 token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                                 residual_length=resid, backend="cuda"))
        segs.append(K.from_dense(f32(ck), f32(cv), k_bits=bits, v_bits=bits, group_size=group,
                                 residual_length=resid, in_dtype="fp16" if dtype == torch.float16 else "bf16"))
    assert caches[1].quantized_tokens % 64 == 32 or group != 32
    ik, iv = kv_pair(256, seed=130, dtype=dtype)
    tk, tv = kv_pair(1024, seed=131, dtype=dtype)
    tk_hmajor = tk.transpose(0, 1).contiguous().to(device)  # [Hkv, T, D], like an H2O segment
    tv_hmajor = tv.transpose(0, 1).contiguous().to(device)
    q = queries(lq, seed=132, dtype=dtype)
    dense = [(ik.to(device), iv.to(device)), (tk_hmajor.transpose(0, 1), tv_hmajor.transpose(0, 1))]
    out, lse = packed_segments_summary(caches, q.to(device), dense)
    assert out.shape == (lq, 28, 128) and out.dtype == dtype
    ks, vs = [f32(ik), f32(tk)], [f32(iv), f32(tv)]
    for seg in segs:
        k, v = K.dequantize(seg, "fp32")
        ks.append(k)
        vs.append(v)
    eo, el = A.attention_summary(f32(q), np.concatenate(ks), np.concatenate(vs))
    assert_close(f32(out), eo, what=f"table {bits}-bit G{group}")
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what=f"table lse {bits}-bit G{group}")


@pytest.mark.parametrize("heads_q,dtype", [(4, torch.bfloat16), (28, torch.float16)])
def test_segment_table_group_and_fp16(device, heads_q, dtype):
    # one query head per KV head (group 1: 150 query rows per KV head), and an
    # all-fp16 table (queries, packed stats and dense parts), against the oracle
    from unicache_amd.storage.kivi_cuda import packed_segments_summary

    ck, cv = kv_pair(900, seed=150, dtype=dtype)
    cache = PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(900),
                                       token_type_id=3, k_bits=4, v_bits=4, group_size=64, residual_length=100,
                                       backend="cuda")
    seg = K.from_dense(f32(ck), f32(cv), k_bits=4, v_bits=4, group_size=64, residual_length=100,
                       in_dtype="fp16" if dtype == torch.float16 else "bf16")
    dk, dv = kv_pair(333, seed=151, dtype=dtype)
    q = queries(150, heads=heads_q, seed=152, dtype=dtype)
    out, lse = packed_segments_summary([cache], q.to(device), [(dk.to(device), dv.to(device))])
    assert out.dtype == dtype and out.shape == (150, heads_q, 128)
    k, v = K.dequantize(seg, "fp32")
    eo, el = A.attention_summary(f32(q), np.concatenate([k, f32(dk)]), np.concatenate([v, f32(dv)]))
    assert_close(f32(out), eo, what=f"table Hq={heads_q} {dtype}")
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what="table lse")


def test_segment_table_rejects_bad_parts_before_launch(device):
    # a CPU dense part, mismatched dense shapes, decode-length queries and a
    # cache without a prefix raise before anything is launched
    from unicache_amd.storage.kivi_cuda import packed_segments_summary

    ck, cv = kv_pair(500, seed=140)
    cache = PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(500),
                                       token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=128,
                                       backend="cuda")
    q = queries(64, seed=141).to(device)
    dk, dv = kv_pair(40, seed=142)
    with pytest.raises(RuntimeError, match="GPU"):
        packed_segments_summary([cache], q, [(dk, dv)])
    with pytest.raises(ValueError, match="matching"):
        packed_segments_summary([cache], q, [(dk.to(device), dv[:30].to(device))])
    with pytest.raises(ValueError, match="Segment-table attention needs"):
        packed_segments_summary([cache], queries(2, seed=143).to(device), [])
    empty = PackedKIVICache.from_dense(ck[:50].to(device), cv[:50].to(device), logical_token_ids=torch.arange(50),
                                       token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=128,
                                       backend="cuda")
    with pytest.raises(ValueError, match="Segment-table attention needs"):
        packed_segments_summary([cache, empty], q, [])


def test_batched_launch_rejects_bad_items_before_launch(device):
    # every table pointer is checked on the host: a CPU dense part, mixed
    # bits, a mixed query dtype, a bad LSE shape and decode-length queries
    # raise before anything is launched
    from unicache_amd.storage.kivi_cuda import packed_batch_with_dense

    def cache(bits, group, seed):
        ck, cv = kv_pair(500, seed=seed)
        return PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(500),
                                          token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                          residual_length=128, backend="cuda")

    c2, c4 = cache(2, 32, 90), cache(4, 32, 91)
    q = queries(64, seed=92).to(device)
    out = torch.empty_like(q)
    dk, dv = kv_pair(40, seed=93)
    lse = torch.empty((28, 64), dtype=torch.float32, device=device)
    with pytest.raises(RuntimeError, match="GPU"):
        packed_batch_with_dense([(c2, q, [dk], [dv], out, lse)])
    with pytest.raises(RuntimeError, match="GPU"):
        packed_batch_with_dense([(c2, q, [], [], out, lse), (c2, q, [dk.to(device)], [dv], out, lse)])
    with pytest.raises(ValueError, match="equal bits"):
        packed_batch_with_dense([(c2, q, [], [], out, lse), (c4, q, [], [], out, lse)])
    with pytest.raises(ValueError, match="one query dtype"):
        packed_batch_with_dense([(c2, q, [], [], out, lse), (c2, q.half(), [], [], out.half(), lse)])
    with pytest.raises(ValueError, match="lse"):
        packed_batch_with_dense([(c2, q, [], [], out, lse[:, :10])])
    short = queries(2, seed=94).to(device)
    with pytest.raises(ValueError, match="multi-query"):
        packed_batch_with_dense([(c2, short, [], [], torch.empty_like(short))])


def test_decode_batch_checks_pointers_and_staleness(device):
    from unicache_amd.storage.decode import KiviDecodeBatch

    ck, cv = kv_pair(1200, seed=95)
    cache = PackedKIVICache.from_dense(ck.to(device), cv.to(device), logical_token_ids=torch.arange(1200),
                                       token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=128,
                                       backend="cuda")
    q = queries(1, seed=96).to(device)
    flat = torch.empty(28 * 128 + 1, dtype=torch.bfloat16, device=device)
    misaligned = flat[1:].view(1, 28, 128)
    with pytest.raises(ValueError, match="16-byte aligned"):
        KiviDecodeBatch([cache], [misaligned])
    with pytest.raises(RuntimeError, match="GPU"):
        KiviDecodeBatch([cache], [q.cpu()])
    batch = KiviDecodeBatch([cache], [q])
    batch.run()
    seg = K.from_dense(f32(ck), f32(cv), k_bits=2, v_bits=2, group_size=32, residual_length=128)
    eo, _ = A.packed_summary(seg, f32(q), kv_dtype="fp32")
    assert_close(f32(batch.outputs[0]), eo, what="batch decode")
    # a flush replaces the packed tensors: run() refuses until refresh()
    nk, nv = kv_pair(130, seed=97)
    for t in range(130):
        cache.append(nk[t:t + 1].to(device), nv[t:t + 1].to(device), logical_token_ids=torch.tensor([1200 + t]),
                     flush_at=256)
    with pytest.raises(RuntimeError, match="refresh"):
        batch.run()
    batch.refresh()
    batch.run()
    seg = K.from_dense(np.concatenate([f32(ck), f32(nk)]), np.concatenate([f32(cv), f32(nv)]), k_bits=2, v_bits=2,
                       group_size=32, residual_length=1330 - cache.quantized_tokens)
    assert seg.quantized_tokens == cache.quantized_tokens
    eo, _ = A.packed_summary(seg, f32(q), kv_dtype="fp32")
    assert_close(f32(batch.outputs[0]), eo, what="batch decode after flush")


def _stream_layer(device, layer, tokens):
    key, value = kv_pair(tokens, seed=300 + layer, dtype=torch.float16)
    cache = PackedKIVICache.from_dense(key.to(device), value.to(device),
                                       logical_token_ids=torch.arange(tokens, device=device), token_type_id=3,
                                       k_bits=2, v_bits=2, group_size=32, residual_length=128, backend="cuda")
    dk, dv = kv_pair(150 + 50 * layer, seed=320 + layer, dtype=torch.float16)
    return key, value, cache, (dk.to(device), dv.to(device))


def test_streaming_decode_appends_on_device(device):
    # three layers of decode steps with one token appended per layer and step
    # through MixedDecodeBatch.append (one launch, device-side lengths, a
    # flush of 128 tokens whenever a window holds 160), against caches
    # appended one by one with a table rebuilt every step: outputs bit for
    # bit, the caches' tensors and ids equal, and the oracle at the end
    from unicache_amd.storage.decode import MixedDecodeBatch

    lengths = (1500, 2100, 900)
    steps = 200
    streamed, shadow, dense, raw = [], [], [], []
    for layer, tokens in enumerate(lengths):
        key, value, c, d = _stream_layer(device, layer, tokens)
        streamed.append(c)
        dense.append(d)
        raw.append((key, value))
        shadow.append(_stream_layer(device, layer, tokens)[2])
    qs = [queries(1, seed=340 + i).to(device) for i in range(3)]
    batch = MixedDecodeBatch([[c, d] for c, d in zip(streamed, dense)], qs)
    batch.reserve(steps)
    g = torch.Generator().manual_seed(7)
    new_k = torch.randn(steps, 3, 1, 4, 128, generator=g).half().to(device)
    new_v = torch.randn(steps, 3, 1, 4, 128, generator=g).half().to(device)
    new_ids = (torch.arange(steps).view(steps, 1, 1) + torch.tensor(lengths).view(1, 3, 1) + 10000).to(device)
    for t in range(steps):
        batch.append(new_k[t], new_v[t], new_ids[t], flush_at=160, keep=32)
        for i, c in enumerate(shadow):
            c.append(new_k[t, i], new_v[t, i], logical_token_ids=new_ids[t, i])
            if c.residual_tokens >= 160:
                c.flush_residual(keep=32)
        if t in (0, 31, 32, 33, 120, steps - 1):
            ref = MixedDecodeBatch([[c, d] for c, d in zip(shadow, dense)], qs)
            batch.run()
            ref.run()
            for i in range(3):
                assert torch.equal(batch.outputs[i], ref.outputs[i]), (t, i)
                assert torch.equal(batch.lses[i], ref.lses[i]), (t, i)
    for c, s in zip(streamed, shadow):
        assert (c.quantized_tokens, c.residual_tokens) == (s.quantized_tokens, s.residual_tokens)
        for name in ("key_code", "key_scale", "key_minimum", "value_code", "value_scale", "value_minimum",
                     "residual_key", "residual_value", "logical_token_ids"):
            assert torch.equal(getattr(c, name), getattr(s, name)), name
    # the oracle over all the tokens of layer 2
    key = np.concatenate([f32(raw[2][0]), f32(new_k[:, 2, 0])])
    value = np.concatenate([f32(raw[2][1]), f32(new_v[:, 2, 0])])
    seg = K.from_dense(key, value, k_bits=2, v_bits=2, group_size=32,
                       residual_length=key.shape[0] - streamed[2].quantized_tokens, in_dtype="fp16")
    assert seg.quantized_tokens == streamed[2].quantized_tokens
    pk, pv = K.dequantize(seg, "fp32")
    eo, el = A.attention_summary(f32(qs[2]), np.concatenate([pk, f32(dense[2][0])]),
                                 np.concatenate([pv, f32(dense[2][1])]))
    assert_close(f32(batch.outputs[2]), eo, what="streamed layer 2 out")
    assert_close(f32(batch.lses[2]), el, max_abs=1e-2, mean_abs=1e-3, what="streamed layer 2 lse")


def test_streaming_decode_guards(device):
    # a cache changed behind the batch's back stops it until refresh(); a
    # second batch streaming into the same cache makes the first one stale;
    # the reserve grows by itself when used up
    from unicache_amd.storage.decode import MixedDecodeBatch

    _, _, cache, dense = _stream_layer(device, 0, 700)
    q = queries(1, seed=350).to(device)
    batch = MixedDecodeBatch([[cache, dense]], [q])
    tr0 = cache.residual_tokens  # 156: 544 of the 700 tokens are packed
    kv = torch.zeros(1, 1, 4, 128, dtype=torch.float16, device=device)
    ids = torch.tensor([[5000]], device=device)
    batch.append(kv, kv, ids)  # reserves on first use
    assert cache.residual_tokens == tr0 + 1 and cache.token_count == 701
    cache.append(kv[0], kv[0], logical_token_ids=ids[0])
    with pytest.raises(RuntimeError, match="refresh"):
        batch.append(kv, kv, ids)
    batch.refresh()
    batch.append(kv, kv, ids)
    assert cache.residual_tokens == tr0 + 3
    other = MixedDecodeBatch([[cache, dense]], [q])
    other.reserve(8)
    with pytest.raises(RuntimeError, match="refresh"):
        batch.run()
    room = other._room
    for _ in range(room + 3):
        other.append(kv, kv, ids)
    assert cache.residual_tokens == tr0 + 3 + room + 3
    with pytest.raises(ValueError):
        other.append(kv[:, :, :2], kv[:, :, :2], ids)
    with pytest.raises(ValueError):
        other.append(kv.float(), kv.float(), ids)
