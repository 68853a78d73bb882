"""Oracle checks at the full sizes of the benchmark configurations (the
shapes bench.py times), complementing the reduced-size parity tests:

- config 1: the 224-item (28 layers x batch 8, 8192 tokens) decode table in
  one uc_kivi_attn_decode_batch launch, sampled items against the oracle;
- config 2: the whole editing pass, 1088 queries over 2304 keys, 2- and 4-bit;
- config 3: H2O scores of 512 queries over 4096 keys, then the per-segment
  selection -- indices asserted bit-exact at a seed whose selection margin
  exceeds twice the score tolerance;
- config 4: the mixed decode segment table (20352-token VAE cache + 2585
  dense tokens) before and after a residual flush.

Inputs follow bench.py's recipe (seeded N(0,1), 8 key channels x10 per head)."""

import numpy as np
import pytest
import torch

from bench import make_kv
from oracle import attention as A
from oracle import h2o as H
from oracle import kivi as K
from tests.helpers import assert_close, f32, kv_pair, queries
from unicache_amd.adapters.bagel import run_fused_mixed_attention
from unicache_amd.operators import per_kv_head_scores_from_qk
from unicache_amd.storage import GQAH2OCache, PackedKIVICache
from unicache_amd.storage.decode import KiviDecodeBatch, MixedDecodeBatch
from unicache_amd.storage.physical import h2o_select_indices
from unicache_amd.storage.tensor_backend import h2o_budget

pytestmark = pytest.mark.gpu


def _packed(key, value, *, bits=2, group=32, residual=128):
    return PackedKIVICache.from_dense(key, value, logical_token_ids=torch.arange(key.shape[0], device=key.device),
                                      token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                      residual_length=residual, backend="cuda")


def _query(lq, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(lq, 28, 128, generator=g, device=device).to(torch.bfloat16)


def test_config1_full_table_sampled_items(device):
    caches, qs = [], []
    for layer in range(28):
        for b in range(8):
            key, value = make_kv(8192, seed=1000 * layer + b, device=device)
            caches.append(_packed(key, value))
            qs.append(_query(1, 7 + 1000 * layer + b, device))
    assert (caches[0].quantized_tokens, caches[0].residual_tokens) == (8064, 128)
    batch = KiviDecodeBatch(caches, qs)
    batch.run()
    torch.cuda.synchronize()
    for layer, b in ((0, 0), (13, 5), (27, 7)):
        i = 8 * layer + b
        print(f"config 1 item layer={layer} seq={b}", flush=True)
        key, value = make_kv(8192, seed=1000 * layer + b, device=device)
        seg = K.from_dense(f32(key), f32(value), k_bits=2, v_bits=2, group_size=32, residual_length=128)
        eo, el = A.packed_summary(seg, f32(qs[i]), kv_dtype="fp32")
        assert_close(f32(batch.outputs[i]), eo, what=f"config 1 item {i} out")
        assert_close(f32(batch.lses[i]), el, max_abs=1e-2, mean_abs=1e-3, what=f"config 1 item {i} lse")


@pytest.mark.parametrize("bits", [2, 4])
def test_config2_full_editing_pass(device, bits):
    # 1088 queries x 28 heads over [instruction 256 | ViT 1024 | VAE residual 128]
    # bf16 + 896 packed VAE tokens = 2304 keys, one fused call
    vk, vv = make_kv(1024, seed=5000, device=device)
    cache = _packed(vk, vv, bits=bits)
    ik, iv = make_kv(256, seed=5100, device=device)
    tk, tv = make_kv(1024, seed=5200, device=device)
    q = _query(1088, 9000, device)
    out, lse = run_fused_mixed_attention(q, torch.cat([ik, tk]), torch.cat([iv, tv]), [cache], return_lse=True)
    seg = K.from_dense(f32(vk), f32(vv), k_bits=bits, v_bits=bits, group_size=32, residual_length=128)
    pk, pv = K.dequantize(seg, "fp32")
    keys = np.concatenate([f32(ik), f32(tk), pk])
    values = np.concatenate([f32(iv), f32(tv), pv])
    assert keys.shape[0] == 2304
    eo, el = A.attention_summary(f32(q), keys, values)
    assert_close(f32(out), eo, what=f"config 2 {bits}-bit out")
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what=f"config 2 {bits}-bit lse")


# Config 3 at seed 1 of a CPU scan of seeds 0..59 (keys kv_pair(4096,
# seed=101, no outliers), queries queries(512, seed=201)): the oracle's scores
# leave a gap of 1.09e-3 between the 38th and 39th instruction-history scores
# and 8.3e-5 between the 576th and 577th ViT-history scores (smallest over the
# 4 KV heads), the largest margins of the scan.  The score tolerance covers
# one bf16 rounding flip of a probability in [2^-8, 2^-7) (2^-15 = 3.05e-5, the
# error measured on the GPU at this seed) and stays below half of both margins.
C3_SEED = 1
C3_SCORE_TOL = 4e-5


def test_config3_full_scores_and_bit_exact_selection(device):
    key, value = kv_pair(4096, seed=100 + C3_SEED, outliers=0)
    q = queries(512, seed=200 + C3_SEED)
    got = per_kv_head_scores_from_qk(q.to(device), key.to(device)).cpu().numpy()
    exp = H.scores_from_qk(f32(q), f32(key))
    err = float(np.abs(got.astype(np.float64) - exp).max())
    print(f"config 3 score error {err:.3g} (tolerance {C3_SCORE_TOL})", flush=True)
    assert err <= C3_SCORE_TOL
    ids = torch.arange(4096)
    retained = 0
    for lo, hi in ((0, 256), (256, 4096)):
        target, recent = h2o_budget(hi - lo, {"target_budget_ratio": 0.2, "recent_budget_fraction": 0.25})
        heavy_k, recent, _ = H.clamp_budget(hi - lo, target, recent)
        # index equality does not depend on summation order when every gap at
        # the selection boundary exceeds twice the score tolerance
        assert H.min_selection_margin(exp[:, lo:hi], heavy_k, recent) > 2 * C3_SCORE_TOL
        got_idx = h2o_select_indices(torch.from_numpy(got[:, lo:hi]).to(device), heavy_k=heavy_k, recent=recent)
        assert np.array_equal(got_idx.cpu().numpy(), H.select(exp[:, lo:hi], heavy_k, recent))
        cache = GQAH2OCache.from_dense(key[lo:hi].to(device), value[lo:hi].to(device), logical_token_ids=ids[lo:hi],
                                       token_type_id=1, per_kv_head_scores=torch.from_numpy(got[:, lo:hi]).to(device),
                                       target_tokens=target, recent_tokens=recent, selection_frozen=True)
        ok, ov, oid, _, _, _ = H.from_dense(f32(key[lo:hi]), f32(value[lo:hi]), np.arange(lo, hi), exp[:, lo:hi],
                                            target, recent)
        assert np.array_equal(cache.logical_token_ids.cpu().numpy(), oid)
        assert np.array_equal(f32(cache.key), ok) and np.array_equal(f32(cache.value), ov)
        retained += cache.retained_tokens
    assert retained == 819


def test_config4_segment_table_and_flush(device):
    # one layer of config 4: VAE 20352 fp16 tokens (20224 packed + 128 residual)
    # and 2585 dense tokens (128 protected + 819 + 1638 H2O-retained), Lq=1;
    # then 128 decode steps appended with a flush at 256 residual tokens
    vk, vv = make_kv(20352, seed=11000, device=device)
    cache = _packed(vk.half(), vv.half())
    assert (cache.quantized_tokens, cache.residual_tokens) == (20224, 128)
    dk, dv = make_kv(2585, seed=12000, device=device)
    dense = (dk.half().contiguous(), dv.half().contiguous())
    q = _query(1, 13000, device)
    batch = MixedDecodeBatch([[cache, dense]], [q])

    def check(all_k, all_v, what):
        batch.run()
        seg = K.from_dense(f32(all_k), f32(all_v), k_bits=2, v_bits=2, group_size=32,
                           residual_length=all_k.shape[0] - cache.quantized_tokens, in_dtype="fp16")
        assert seg.quantized_tokens == cache.quantized_tokens
        pk, pv = K.dequantize(seg, "fp32")
        eo, el = A.attention_summary(f32(q), np.concatenate([pk, f32(dense[0])]), np.concatenate([pv, f32(dense[1])]))
        assert_close(f32(batch.outputs[0]), eo, what=f"{what} out")
        assert_close(f32(batch.lses[0]), el, max_abs=1e-2, mean_abs=1e-3, what=f"{what} lse")

    check(vk.half(), vv.half(), "config 4")
    # decode steps append through the batch: one launch per step extends the
    # window and the device item table, no refresh and no host copy of the table
    nk, nv = make_kv(128, seed=14000, device=device)
    nk, nv = nk.half(), nv.half()
    packed_before = cache.quantized_tokens
    batch.reserve(128)
    ids = torch.arange(20352, 20352 + 128, device=device).view(128, 1, 1)
    for t in range(128):
        batch.append(nk[t:t + 1][None], nv[t:t + 1][None], ids[t], flush_at=256)
        if t == 63:
            assert cache.residual_tokens == 192 and cache.quantized_tokens == packed_before
            check(torch.cat([vk.half(), nk[:64]]), torch.cat([vv.half(), nv[:64]]), "config 4 after 64 appends")
    assert cache.quantized_tokens == packed_before + 256 and cache.residual_tokens == 0
    assert torch.equal(cache.logical_token_ids.cpu(), torch.arange(20352 + 128))
    check(torch.cat([vk.half(), nk]), torch.cat([vv.half(), nv]), "config 4 after flush")
