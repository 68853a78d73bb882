"""Pins oracle.attention and oracle.h2o.

Known answers come from UniCache's tests (test_physical.py:181-202 LSE merge,
1195-1215 H2O per-head selection, 1217-1270 budget counts); the rest are
closed forms (LSE of the logits, GQA == repeated-KV attention computed by
torch, packed logits and P.V over a segment built word by word) and a
brute-force selection by Python's sort.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import h2o as H
from oracle import kivi as K


def test_lse_merge_equals_global_softmax():
    # test_physical.py:181-202
    rng = np.random.default_rng(11)
    sa, sb = rng.standard_normal((4, 3, 7)), rng.standard_normal((4, 3, 5))
    va, vb = rng.standard_normal((4, 7, 8)), rng.standard_normal((4, 5, 8))
    summaries = [
        ((A.softmax(sa) @ va).transpose(1, 0, 2), A.logsumexp(sa)),
        ((A.softmax(sb) @ vb).transpose(1, 0, 2), A.logsumexp(sb)),
    ]
    out, lse = A.merge_summaries(summaries)
    allv = np.concatenate([va, vb], axis=1)
    alls = np.concatenate([sa, sb], axis=-1)
    expected = (A.softmax(alls) @ allv).transpose(1, 0, 2)
    assert np.allclose(out, expected, atol=1e-5)
    assert np.allclose(lse, A.logsumexp(alls), atol=1e-6)


def test_gqa_matches_repeated_kv_torch():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((5, 28, 16)).astype(np.float32)
    k = rng.standard_normal((9, 4, 16)).astype(np.float32)
    v = rng.standard_normal((9, 4, 16)).astype(np.float32)
    logits = A.gqa_logits(q, k)
    kt = torch.from_numpy(k).double().repeat_interleave(7, dim=1)
    ref = torch.matmul(torch.from_numpy(q).double().transpose(0, 1), kt.transpose(0, 1).transpose(-1, -2))
    assert np.allclose(logits, ref.numpy(), atol=1e-10)
    p = A.softmax(logits)
    pv = A.gqa_pv(p, v)
    vt = torch.from_numpy(v).double().repeat_interleave(7, dim=1)
    ref_pv = torch.matmul(torch.from_numpy(p), vt.transpose(0, 1))
    assert np.allclose(pv, ref_pv.numpy(), atol=1e-10)


def test_attention_summary_closed_forms():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((3, 14, 32))
    k = rng.standard_normal((50, 2, 32))
    v = rng.standard_normal((50, 2, 32))
    out, lse = A.attention_summary(q, k, v)
    logits = A.gqa_logits(q, k) / math.sqrt(32)
    ref_lse = np.log(np.exp(logits).sum(-1))
    assert np.allclose(lse, ref_lse, atol=1e-10)
    # constant values -> the output is that constant whatever the weights
    out_c, _ = A.attention_summary(q, k, np.full_like(v, 2.5))
    assert np.allclose(out_c, 2.5)
    assert out.shape == (3, 14, 32)


# ---------------------------------------------- packed attention parts --
def _segment_parts():
    """A 2-bit, kernel-native segment built word by word: 2 KV heads, D = 16
    (so 1/sqrt(D) = 1/4 exactly), 32 packed tokens at G = 16 and 2 residual
    tokens, with keys and values that differ.  Returns the segment and the
    dequantized key / value as Python functions of (head, token, channel),
    written from the construction (not from the oracle's unpacking).

    Word 0xE4E4E4E4 holds the codes 0, 1, 2, 3 repeated (LSB first), word
    0x1B1B1B1B the codes 3, 2, 1, 0.  Every value below is exact in fp16 and
    bf16.
    """

    e4 = np.uint32(0xE4E4E4E4).view(np.int32)
    w1b = np.uint32(0x1B1B1B1B).view(np.int32)
    kc = np.empty((2, 16, 2), np.int32)                       # [Hkv, D, Tq/16]
    kc[0], kc[1] = e4, w1b
    ks = np.tile(np.array([0.5, 2.0], np.float32), (2, 16, 1))  # [Hkv, D, Tq/G]
    km = np.array([-1.0, 3.0], np.float32)[None, None, :] + (np.arange(16, dtype=np.float32) / 8)[None, :, None]
    km = np.ascontiguousarray(np.broadcast_to(km, (2, 16, 2)))
    vc = np.empty((2, 32, 1), np.int32)                       # [Hkv, Tq, D/16]
    vc[0], vc[1] = w1b, e4
    vs = np.full((2, 32, 1), 0.25, np.float32)                # [Hkv, Tq, D/G]
    vm = np.stack([np.arange(32), -np.arange(32)]).astype(np.float32)[:, :, None]

    def key_code(h, t):
        return t % 4 if h == 0 else 3 - t % 4

    def value_code(h, c):
        return 3 - c % 4 if h == 0 else c % 4

    def khat(h, t, d):
        if t < 32:
            g = t // 16
            return key_code(h, t) * (0.5, 2.0)[g] + (-1.0, 3.0)[g] + d / 8
        return (d - 8) * 0.25 * (t - 31) * (h + 1)

    def vhat(h, t, c):
        if t < 32:
            return value_code(h, c) * 0.25 + (t if h == 0 else -t)
        return 10.0 * (t - 31) + c / 4 + h

    rk = np.array([[[khat(h, t, d) for d in range(16)] for h in range(2)] for t in (32, 33)], np.float32)
    rv = np.array([[[vhat(h, t, c) for c in range(16)] for h in range(2)] for t in (32, 33)], np.float32)
    seg = K.PackedSegment(kc, ks, km, vc, vs, vm, rk, rv, k_bits=2, v_bits=2, group_size=16,
                          quantized_tokens=32, native=True)
    return seg, khat, vhat


def _hand_query():
    # [Lq = 2, Hq = 4, D = 16], small halves: query head h reads KV head h // 2
    return np.array([[[((l + 2 * h + d) % 5 - 2) * 0.5 for d in range(16)] for h in range(4)] for l in range(2)],
                    np.float32)


def test_packed_logits_closed_form():
    # kivi_cuda.py:283-287 / physical.py:469-470: logits over [packed | residual]
    # tokens, q . k_hat scaled by 1/sqrt(D)
    seg, khat, _ = _segment_parts()
    q = _hand_query()
    got = A.packed_logits(seg, q)
    assert got.shape == (4, 2, 34)
    expected = np.array([[[sum(float(q[l, h, d]) * khat(h // 2, t, d) for d in range(16)) / 4 for t in range(34)]
                          for l in range(2)] for h in range(4)])
    assert np.allclose(got, expected, rtol=0, atol=1e-12)
    # the residual tokens come last: token 32's logit is q . (d - 8) / 4 * (h // 2 + 1) / 4
    assert got[2, 1, 32] == sum(float(q[1, 2, d]) * (d - 8) * 0.5 for d in range(16)) / 4


def test_packed_pv_closed_form():
    # physical.py:472-473: the apply_value closure multiplies P by the
    # dequantized values (not the keys) over [packed | residual]
    seg, khat, vhat = _segment_parts()
    rng = np.random.default_rng(31)
    p = rng.random((4, 2, 34))
    p /= p.sum(-1, keepdims=True)
    got = A.packed_pv(seg, p)
    assert got.shape == (4, 2, 16)
    expected = np.array([[[sum(p[h, l, t] * vhat(h // 2, t, c) for t in range(34)) for c in range(16)]
                          for l in range(2)] for h in range(4)])
    assert np.allclose(got, expected, rtol=0, atol=1e-12)
    # a one-hot row picks one value row: the packed token 5 of KV head 1, and residual token 33 of head 0
    one = np.zeros((4, 2, 34))
    one[3, 0, 5] = 1.0
    one[0, 1, 33] = 1.0
    picked = A.packed_pv(seg, one)
    assert picked[3, 0].tolist() == [vhat(1, 5, c) for c in range(16)]
    assert picked[0, 1].tolist() == [vhat(0, 33, c) for c in range(16)]
    assert picked[3, 0].tolist() != [khat(1, 5, c) for c in range(16)]


def test_packed_summary_equals_softmax_of_packed_logits():
    # the fused summary of the whole segment is softmax(packed_logits) . V_hat
    # with the natural-log LSE of those logits
    seg, _, _ = _segment_parts()
    q = _hand_query()
    out, lse = A.packed_summary(seg, q)
    logits = A.packed_logits(seg, q)
    assert np.allclose(lse, np.log(np.exp(logits).sum(-1)), atol=1e-12)
    assert np.allclose(out.transpose(1, 0, 2), A.packed_pv(seg, A.softmax(logits)), atol=1e-12)


# --------------------------------------------------------------------- H2O --
def test_h2o_known_answer_per_kv_head():
    # test_physical.py:1195-1215
    key = np.arange(8 * 2 * 4, dtype=np.float32).reshape(8, 2, 4)
    scores = np.array([[9, 8, 5, 4, 3, 2, 0, 0], [0, 8, 1, 1, 1, 9, 0, 0]], dtype=np.float32)
    ok, ov, ids, sc, heavy, recent = H.from_dense(key, key + 1000, np.arange(8), scores, 4, 2)
    assert ids[0].tolist() == [0, 1, 6, 7]
    assert ids[1].tolist() == [1, 5, 6, 7]
    assert (heavy, recent) == (2, 2)
    assert np.array_equal(ok[1, 1], key[5, 1]) and np.array_equal(ov[0, 2], key[6, 0] + 1000)
    assert sc[1].tolist() == [8.0, 9.0, 0.0, 0.0]


@pytest.mark.parametrize(
    "n,ratio,target,recent",
    [
        (256, 0.2, 51, 13),    # config 3 instruction
        (3840, 0.2, 768, 192),  # config 3 ViT
        (4096, 0.2, 819, 205),  # config 4 instruction
        (8192, 0.2, 1638, 410),  # config 4 ViT: round(409.5) == 410 (half to even)
        (12, 0.5, 6, 2),        # test_physical.py:1217-1270 (round(1.5) == 2)
        (10, 0.25, 2, 0),       # round(2.5) == 2, round(0.5) == 0
    ],
)
def test_h2o_budget_round_half_even(n, ratio, target, recent):
    assert H.budget(n, {"target_budget_ratio": ratio, "recent_budget_fraction": 0.25}) == (target, recent)


def test_h2o_budget_clamps():
    # physical.py:511-515
    assert H.clamp_budget(10, 50, 3) == (7, 3, 7)
    assert H.clamp_budget(10, 0, 0) == (1, 0, 1)
    assert H.clamp_budget(10, 4, 9) == (0, 4, 0)


def test_select_brute_force_with_ties():
    rng = np.random.default_rng(9)
    for trial in range(50):
        t = int(rng.integers(1, 60))
        recent = int(rng.integers(0, t))
        k = int(rng.integers(0, t - recent + 1))
        s = rng.integers(0, 5, size=(3, t)).astype(np.float32)  # many ties
        got = H.select(s, k, recent)
        for h in range(3):
            order = sorted(range(t - recent), key=lambda i: (-float(s[h, i]), i))
            assert got[h, :k].tolist() == sorted(order[:k])
            assert got[h, k:].tolist() == list(range(t - recent, t))


def test_select_nan_ranks_highest():
    s = np.array([[1.0, np.nan, 5.0, np.inf, 2.0]], dtype=np.float32)
    assert H.select(s, 2, 0)[0].tolist() == [1, 3]
    assert H.select(s, 1, 0)[0].tolist() == [1]


def test_scores_from_probs_order_of_sums():
    # operators/physical.py:62-65: query sum per head, then group sum
    rng = np.random.default_rng(5)
    p = rng.random((28, 3, 11)).astype(np.float32)
    s = H.scores_from_probs(p, 4)
    ref = np.array([[p[h * 7 + g, :, t].sum() for t in range(11)] for h in range(4) for g in range(7)])
    ref = ref.reshape(4, 7, 11).sum(1)
    assert np.allclose(s, ref, rtol=1e-6)


def test_scores_from_qk_rows_sum_to_query_count():
    # every softmax row sums to 1, so sum_t scores[h, t] ~= group * Lq (bf16 rounding aside)
    rng = np.random.default_rng(8)
    q = rng.standard_normal((6, 28, 32)).astype(np.float32)
    k = rng.standard_normal((40, 4, 32)).astype(np.float32)
    s = H.scores_from_qk(q, k)
    assert s.shape == (4, 40)
    assert np.allclose(s.sum(1), 7 * 6, rtol=2e-2)


def test_trim_reselects_within_retained():
    key = np.arange(2 * 6 * 3, dtype=np.float32).reshape(2, 6, 3)
    ids = np.array([[10, 11, 12, 13, 14, 15], [20, 21, 22, 23, 24, 25]])
    sc = np.array([[5, 1, 4, 0, 0, 0], [0, 9, 9, 1, 0, 0]], dtype=np.float32)
    k2, _, i2, s2 = H.trim(key, key, ids, sc, 3, 1)
    assert i2.tolist() == [[10, 12, 15], [21, 22, 25]]
    assert s2.tolist() == [[5, 4, 0], [9, 9, 0]]


def test_compact_brute_force_and_known_answer():
    # rows 0..9 in two samples of 4 and 6: keep rows 1, 3 of the first and
    # 0, 4, 5 of the second -> source rows 1, 3, 4, 8, 9 in order
    key = np.arange(10 * 2 * 3, dtype=np.float32).reshape(10, 2, 3)
    ids = np.arange(100, 110, dtype=np.int64)
    masks = [np.array([0, 1, 0, 1], bool), np.array([1, 0, 0, 0, 1, 1], bool)]
    ok, ov, oi, lens = H.compact(key, -key, ids, [4, 6], masks)
    assert np.array_equal(ok, key[[1, 3, 4, 8, 9]]) and np.array_equal(ov, -key[[1, 3, 4, 8, 9]])
    assert np.array_equal(oi, [101, 103, 104, 108, 109]) and lens == [2, 3]
    # brute force: explicit row loop over random ragged samples
    rng = np.random.default_rng(3)
    lens_in = [0, 7, 1, 13]
    full = rng.random((sum(lens_in), 2, 3)).astype(np.float32)
    masks = [rng.random(n) < 0.4 for n in lens_in]
    ok, _, _, lens = H.compact(full, full, None, lens_in, masks)
    rows, off = [], 0
    for n, m in zip(lens_in, masks):
        for i in range(n):
            if m[i]:
                rows.append(full[off + i])
        off += n
    assert np.array_equal(ok, np.stack(rows)) and lens == [int(m.sum()) for m in masks]
