"""GPU parity of H2O: selection and gather bit-exact (ties to the lowest
index), scores within fp32 summation tolerance, indices exact where the
selection margin exceeds that tolerance."""

import numpy as np
import pytest
import torch

from oracle import h2o as H
from oracle.kivi import round_bf16
from tests.helpers import f32, kv_pair, queries
from unicache_amd.operators import per_kv_head_scores_from_probs, per_kv_head_scores_from_qk
from unicache_amd.storage import GQAH2OCache
from unicache_amd.storage.physical import h2o_select_indices
from unicache_amd.storage.tensor_backend import h2o_budget

pytestmark = pytest.mark.gpu


def test_known_answer_per_kv_head(device):
    # test_physical.py:1195-1215
    key = torch.arange(8 * 2 * 4, dtype=torch.float32).reshape(8, 2, 4)
    scores = torch.tensor([[9.0, 8.0, 5.0, 4.0, 3.0, 2.0, 0.0, 0.0], [0.0, 8.0, 1.0, 1.0, 1.0, 9.0, 0.0, 0.0]])
    cache = GQAH2OCache.from_dense(key.to(device), (key + 1000).to(device), logical_token_ids=torch.arange(8),
                                   token_type_id=1, per_kv_head_scores=scores.to(device), target_tokens=4,
                                   recent_tokens=2)
    assert cache.logical_token_ids[0].tolist() == [0, 1, 6, 7]
    assert cache.logical_token_ids[1].tolist() == [1, 5, 6, 7]
    assert torch.equal(cache.key[1, 1].cpu(), key[5, 1])
    assert torch.equal(cache.value[0, 2].cpu(), key[6, 0] + 1000)
    assert cache.resident_bytes < cache.full_precision_bytes


@pytest.mark.parametrize("tokens,k,recent", [(3840, 576, 192), (256, 38, 13), (100000, 20000, 5000), (33, 0, 33),
                                             (50, 50, 0)])
def test_select_bit_exact_with_ties(device, tokens, k, recent):
    rng = np.random.default_rng(tokens)
    scores = rng.integers(0, 50, size=(4, tokens)).astype(np.float32)  # heavy ties
    scores[1] = rng.standard_normal(tokens).astype(np.float32)
    scores[2, ::7] = np.nan
    got = h2o_select_indices(torch.from_numpy(scores).to(device), heavy_k=k, recent=recent)
    exp = H.select(scores, k, recent)
    assert np.array_equal(got.cpu().numpy(), exp)


def test_select_strided_scores(device):
    rng = np.random.default_rng(3)
    base = rng.integers(0, 9, size=(8, 500)).astype(np.float32)
    view = torch.from_numpy(base).to(device)[::2]  # head stride 1000
    got = h2o_select_indices(view, heavy_k=60, recent=10)
    assert np.array_equal(got.cpu().numpy(), H.select(base[::2], 60, 10))


def test_config3_from_dense(device):
    # 256 instruction + 3840 ViT tokens at 20% with a 25% recent window
    key, value = kv_pair(4096, seed=3)
    rng = np.random.default_rng(33)
    scores = rng.random((4, 4096)).astype(np.float32)
    ids = torch.arange(4096)
    parts = []
    for lo, hi in ((0, 256), (256, 4096)):
        target, recent = h2o_budget(hi - lo, {"target_budget_ratio": 0.2, "recent_budget_fraction": 0.25})
        c = GQAH2OCache.from_dense(key[lo:hi].to(device), value[lo:hi].to(device), logical_token_ids=ids[lo:hi],
                                   token_type_id=1, per_kv_head_scores=torch.from_numpy(scores[:, lo:hi]).to(device),
                                   target_tokens=target, recent_tokens=recent, selection_frozen=True)
        ok, ov, oid, osc, heavy, rec = H.from_dense(f32(key[lo:hi]), f32(value[lo:hi]), np.arange(lo, hi),
                                                    scores[:, lo:hi], target, recent)
        assert np.array_equal(f32(c.key), ok) and np.array_equal(f32(c.value), ov)
        assert np.array_equal(c.logical_token_ids.cpu().numpy(), oid)
        assert np.array_equal(c.cumulative_scores.cpu().numpy(), osc)
        assert (c.heavy_tokens, c.recent_tokens) == (heavy, rec)
        parts.append(c)
    assert parts[0].retained_tokens + parts[1].retained_tokens == 819


# (tokens, target, recent, score kind): ties, NaN, the 8192-token limit of the
# one-launch kernel, a recent-only budget, and a 9000-token segment that the
# entry point hands to the per-segment kernels within the same call
SEGMENTS = [(256, 51, 12, "ties"), (3840, 768, 192, "nan"), (8192, 1638, 409, "normal"), (40, 40, 40, "ties"),
            (9000, 900, 100, "normal"), (1000, 300, 0, "ties")]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_select_gather_segments_one_call(device, dtype):
    rng = np.random.default_rng(7)
    specs, expected = [], []
    for n, (tokens, target, recent, kind) in enumerate(SEGMENTS):
        key, value = kv_pair(tokens, seed=40 + n, dtype=dtype)
        if kind == "ties":
            scores = rng.integers(0, 20, size=(4, tokens)).astype(np.float32)
        else:
            scores = rng.standard_normal((4, tokens)).astype(np.float32)
        if kind == "nan":
            scores[2, ::7] = np.nan
        ids = np.arange(1000 * n, 1000 * n + tokens)
        kd, vd = key.to(device), value.to(device)
        if n == 5:  # a strided view of a larger buffer: token stride 2 * Hkv * D
            kd = torch.repeat_interleave(kd, 2, dim=0)[::2]
            vd = torch.repeat_interleave(vd, 2, dim=0)[::2]
        specs.append(dict(key=kd, value=vd, logical_token_ids=torch.from_numpy(ids).to(device), token_type_id=n,
                          per_kv_head_scores=torch.from_numpy(scores).to(device), target_tokens=target,
                          recent_tokens=recent))
        expected.append(H.from_dense(f32(key), f32(value), ids, scores, target, recent))
    caches = GQAH2OCache.from_dense_segments(specs)
    for n, (c, (ok, ov, oid, osc, heavy, rec)) in enumerate(zip(caches, expected)):
        print(f"segment {n}: {SEGMENTS[n]}", flush=True)
        assert np.array_equal(f32(c.key), ok) and np.array_equal(f32(c.value), ov)
        assert np.array_equal(c.logical_token_ids.cpu().numpy(), oid)
        assert np.array_equal(c.cumulative_scores.cpu().numpy(), osc, equal_nan=True)
        assert (c.heavy_tokens, c.recent_tokens, c.token_type_id) == (heavy, rec, n)
    # one segment per call gives the same caches
    for spec, c in zip(specs, caches):
        one = GQAH2OCache.from_dense(**spec)
        assert torch.equal(one.key, c.key) and torch.equal(one.logical_token_ids, c.logical_token_ids)


def test_select_gather_segments_mixed_shapes(device):
    # segments of different head_dim run as separate groups of the same call
    rng = np.random.default_rng(8)
    specs, expected = [], []
    for n, (tokens, d) in enumerate(((500, 64), (700, 128), (300, 64))):
        key, value = kv_pair(tokens, head_dim=d, seed=60 + n)
        scores = rng.random((4, tokens)).astype(np.float32)
        ids = np.arange(tokens)
        specs.append(dict(key=key.to(device), value=value.to(device), logical_token_ids=torch.from_numpy(ids).to(device),
                          token_type_id=1, per_kv_head_scores=torch.from_numpy(scores).to(device),
                          target_tokens=tokens // 5, recent_tokens=tokens // 20))
        expected.append(H.from_dense(f32(key), f32(value), ids, scores, tokens // 5, tokens // 20))
    for c, (ok, ov, oid, osc, _, _) in zip(GQAH2OCache.from_dense_segments(specs), expected):
        assert np.array_equal(f32(c.key), ok) and np.array_equal(f32(c.value), ov)
        assert np.array_equal(c.logical_token_ids.cpu().numpy(), oid)


def test_scores_from_probs(device):
    rng = np.random.default_rng(4)
    probs = torch.from_numpy(rng.random((28, 16, 300)).astype(np.float32)).to(torch.bfloat16)
    got = per_kv_head_scores_from_probs(probs.to(device), 4)
    assert np.allclose(got.cpu().numpy(), H.scores_from_probs(f32(probs), 4), rtol=1e-5, atol=1e-5)


def test_fused_scores_near_ties_only(device):
    # Q [128, 28, 128], K [4096, 4, 128]: a seed whose selection margin is
    # below the score error; the selections may then differ only in near-ties
    # (config 3 itself is asserted bit-exact in test_gpu_full_size.py)
    key, _ = kv_pair(4096, seed=5, outliers=0)
    q = queries(128, seed=6)
    got = per_kv_head_scores_from_qk(q.to(device), key.to(device)).cpu().numpy()
    exp = H.scores_from_qk(f32(q), f32(key))
    err = np.abs(got - exp)
    assert err.max() <= 1e-3 * max(1.0, float(np.abs(exp).max())), err.max()
    heavy_k, recent = 576, 192
    tol = float(err.max())
    got_idx = h2o_select_indices(torch.from_numpy(got).to(device), heavy_k=heavy_k, recent=recent).cpu().numpy()
    exp_idx = H.select(exp, heavy_k, recent)
    for h in range(4):
        diff = set(got_idx[h]) ^ set(exp_idx[h])
        kth = np.sort(exp[h, : 4096 - recent])[::-1][heavy_k - 1]
        assert all(abs(exp[h, i] - kth) <= 2 * tol for i in diff)


# (Lq, Hq, Hkv, T, D, dtype): ragged row blocks (group * Lq not a multiple of
# 256), several key chunks with a ragged last tile, one key, group 1, fp16,
# and head_dim 64 (the generic kernels)
SCORE_SHAPES = [
    (5, 28, 4, 300, 128, torch.bfloat16),
    (100, 8, 2, 1000, 128, torch.float16),
    (1, 28, 4, 4097, 128, torch.bfloat16),
    (37, 4, 4, 64, 128, torch.bfloat16),
    (300, 28, 4, 1, 128, torch.bfloat16),
    (9, 6, 2, 200, 64, torch.bfloat16),
]


@pytest.mark.parametrize("lq,hq,hkv,tokens,d,dtype", SCORE_SHAPES)
def test_fused_scores_shapes(device, lq, hq, hkv, tokens, d, dtype):
    key, _ = kv_pair(tokens, heads=hkv, head_dim=d, seed=11, dtype=dtype)
    q = queries(lq, heads=hq, head_dim=d, seed=12, dtype=dtype)
    got = per_kv_head_scores_from_qk(q.to(device), key.to(device)).cpu().numpy()
    exp = H.scores_from_qk(f32(q), f32(key))
    # a probability p whose bf16 rounding flips moves its key's score by at most
    # p * 2^-8 (one bf16 ulp); flips come from fp32 rounding of the logits and
    # of the exponential, so the bound is a few ulps of the largest score
    tol = 2e-3 * max(1.0, float(np.abs(exp).max()))
    assert np.abs(got - exp).max() <= tol, np.abs(got - exp).max()
    # mass conservation: every valid row's probabilities sum to 1 up to bf16 rounding
    assert abs(float(got.sum()) - hq * lq) <= 4e-3 * hq * lq + 1e-3


def test_fused_scores_accumulate_strided_deterministic(device):
    key, _ = kv_pair(777, seed=13)
    big = queries(64, heads=28, head_dim=256, seed=14)
    q = big[..., 64:192]
    exp = H.scores_from_qk(f32(q), f32(key))
    qd, kd = big.to(device)[..., 64:192], key.to(device)  # head and row strides 256, 7168
    assert qd.stride() == (28 * 256, 256, 1)
    first = per_kv_head_scores_from_qk(qd, kd)
    again = per_kv_head_scores_from_qk(qd, kd)
    assert torch.equal(first, again)
    base = torch.full_like(first, 0.25)
    acc = per_kv_head_scores_from_qk(qd, kd, out=base.clone())
    assert torch.equal(acc, base + first)
    assert np.abs(first.cpu().numpy() - exp).max() <= 2e-3 * max(1.0, float(np.abs(exp).max()))


@pytest.mark.parametrize("d,lq,tokens", [(128, 20, 500), (64, 9, 200)])
def test_fused_scores_with_given_lse(device, d, lq, tokens):
    # probabilities against a caller LSE (the global LSE of a mixed-segment
    # call): bf16(exp(logit - lse)); here the LSE of a larger key set, so rows
    # do not sum to one
    import math

    from oracle import attention as A

    key, _ = kv_pair(tokens, head_dim=d, seed=14)
    extra, _ = kv_pair(300, head_dim=d, seed=15)
    q = queries(lq, head_dim=d, seed=16)
    lse = A.logsumexp(A.gqa_logits(f32(q), np.concatenate([f32(key), f32(extra)])) / math.sqrt(d))
    got = per_kv_head_scores_from_qk(q.to(device), key.to(device), lse=torch.from_numpy(lse).to(device))
    probs = round_bf16(np.exp(A.gqa_logits(f32(q), f32(key)) / math.sqrt(d) - lse[:, :, None]).astype(np.float32))
    exp = H.scores_from_probs(probs, 4)
    assert np.abs(got.cpu().numpy() - exp).max() <= 2e-3 * max(1.0, float(np.abs(exp).max()))


def test_trim_update_and_budget(device):
    key, value = kv_pair(64, heads=2, head_dim=16, seed=7)
    rng = np.random.default_rng(7)
    scores = rng.random((2, 64)).astype(np.float32)
    cache = GQAH2OCache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(64),
                                   token_type_id=1, per_kv_head_scores=torch.from_numpy(scores).to(device),
                                   target_tokens=16, recent_tokens=4)
    probs = torch.from_numpy(rng.random((14, 3, 16)).astype(np.float32)).to(device)
    before = cache.cumulative_scores.cpu().numpy()
    cache.update_scores(probs)
    upd = before + H.scores_from_probs(probs.cpu().numpy(), 2)
    assert np.allclose(cache.cumulative_scores.cpu().numpy(), upd, rtol=1e-6)
    k_hrd, v_hrd = f32(cache.key), f32(cache.value)
    ids, sc = cache.logical_token_ids.cpu().numpy(), cache.cumulative_scores.cpu().numpy()
    # test_physical.py:1099-1132
    assert cache.request_budget(8, 2) == 8 and cache.retained_tokens == 8
    ek, ev, eid, esc = H.trim(k_hrd, v_hrd, ids, sc, 8, 2)
    assert np.array_equal(f32(cache.key), ek) and np.array_equal(cache.logical_token_ids.cpu().numpy(), eid)
    assert cache.request_budget(16, 4) == 8 and cache.budget_shortfall_tokens == 8


def test_update_scores_row_and_element_kernels_agree(device):
    # contiguous probabilities (a workgroup per 64 keys, one wave per query head)
    # and a key-strided view (one thread per key) make the same additions
    rng = np.random.default_rng(9)
    key, value = kv_pair(200, heads=4, head_dim=32, seed=9)
    probs = torch.from_numpy(rng.random((28, 37, 200)).astype(np.float32)).to(torch.bfloat16)
    wide = torch.zeros(28, 37, 400, dtype=torch.bfloat16)
    wide[:, :, ::2] = probs
    init = torch.from_numpy(rng.random((4, 200)).astype(np.float32)).to(device)

    def cache():
        return GQAH2OCache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(200),
                                      token_type_id=1, per_kv_head_scores=init.clone(), target_tokens=200,
                                      recent_tokens=0)

    a, b = cache(), cache()
    before = a.cumulative_scores.cpu().numpy()
    a.update_scores(probs.to(device))
    b.update_scores(wide.to(device)[:, :, ::2])
    assert torch.equal(a.cumulative_scores, b.cumulative_scores)
    exp = before + H.scores_from_probs(f32(probs), 4)
    assert np.allclose(a.cumulative_scores.cpu().numpy(), exp, rtol=1e-5)


def test_h2o_attention_parts(device):
    import math

    from oracle import attention as A
    from tests.helpers import assert_close

    key, value = kv_pair(300, seed=8)
    scores = torch.rand(4, 300)
    cache = GQAH2OCache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(300),
                                   token_type_id=1, per_kv_head_scores=scores.to(device), target_tokens=60,
                                   recent_tokens=15)
    q = queries(3, seed=9)
    logits, apply_value = cache.attention_parts(q.to(device))
    k_td = np.transpose(f32(cache.key), (1, 0, 2))
    v_td = np.transpose(f32(cache.value), (1, 0, 2))
    assert_close(f32(logits), A.gqa_logits(f32(q), k_td) / math.sqrt(128), max_abs=1e-3, mean_abs=1e-4,
                 what="h2o logits")
    p = torch.softmax(logits, -1).to(torch.bfloat16)
    assert_close(f32(apply_value(p)), A.gqa_pv(f32(p), v_td), what="h2o av")
