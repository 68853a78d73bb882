"""GPU parity of the packed attention kernels against the oracle's fp32
dequant path: max abs <= 2e-2, mean abs <= 1e-3 (outputs), LSE within 1e-3."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import kivi as K
from tests.helpers import assert_close, f32, kv_pair, queries
from unicache_amd import _native as nat
from unicache_amd.adapters import merge_attention_summaries
from unicache_amd.storage import PackedKIVICache, gqa_probability_value, gqa_query_key_logits
from unicache_amd.storage.kivi_cuda import (
    packed_kivi_attention_summary,
    packed_kivi_quantized_attention_summary,
)

pytestmark = pytest.mark.gpu


def check_summary(out, lse, seg, q, *, include_residual=True, what="summary"):
    """Outputs within 2e-2 max / 1e-3 mean of the fp32 dequant path (the
    contract) and of the bf16-dequant runtime path of UniCache; the natural
    LSE within 1e-2 max / 1e-3 mean of the fp32 path."""

    eo, el = A.packed_summary(seg, f32(q), include_residual=include_residual, kv_dtype="fp32")
    assert_close(f32(out), eo, what=f"{what} out (fp32 path)")
    # the kernels round dequantized keys to fp16 before the MFMA (UniCache's
    # runtime rounds them to bf16, 8x coarser): with x10 outlier channels a key
    # of ~40 carries up to 0.016 of rounding, ~5e-3 on the largest of ~3e4 LSEs
    assert_close(f32(lse), el, max_abs=1e-2, mean_abs=1e-3, what=f"{what} lse (fp32 path)")
    # UniCache's runtime path rounds dequantized K/V to bf16 itself; over the
    # ~4e6 outputs of config 2 it strays from the fp32 path by up to ~3e-2, so
    # against it the bounds are looser
    bo, _ = A.packed_summary(seg, f32(q), include_residual=include_residual, kv_dtype="bf16")
    assert_close(f32(out), bo, max_abs=5e-2, mean_abs=2e-3, what=f"{what} out (bf16 path)")


def _pair(tokens, seed, bits, group, residual, device, heads=4, head_dim=128):
    key, value = kv_pair(tokens, heads=heads, head_dim=head_dim, seed=seed)
    cache = PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(tokens),
                                       token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                       residual_length=residual, backend="cuda")
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=group,
                       residual_length=residual, native=bits != 8)
    return cache, seg


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("lq", [1, 37])
def test_attention_parts_qk_av(device, bits, lq):
    cache, seg = _pair(320, 5, bits, 64, 32, device)
    q = queries(lq, seed=7)
    logits, apply_value = cache.attention_parts(q.to(device))
    assert logits.dtype == torch.float32 and tuple(logits.shape) == (28, lq, 320)
    exp_logits = A.packed_logits(seg, f32(q), kv_dtype="fp32")
    assert_close(f32(logits), exp_logits, max_abs=2e-3, mean_abs=2e-4, what="logits")
    probs = torch.softmax(logits, dim=-1).to(torch.bfloat16)
    out = apply_value(probs)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (28, lq, 128)
    exp = A.packed_pv(seg, f32(probs), kv_dtype="bf16")
    assert_close(f32(out), exp, what="av")


@pytest.mark.parametrize("bits,group,tokens,residual,lq", [(2, 16, 200, 32, 1), (4, 32, 250, 20, 3),
                                                         (2, 128, 1100, 60, 2), (4, 16, 2048, 128, 1)])
def test_attention_parts_tiles_groups_and_rows(device, bits, group, tokens, residual, lq):
    # token tiles that mix packed and residual tokens (groups 16 and 32 with
    # quantized counts of 160 and 224, not multiples of 64), groups 16 to 128,
    # several query rows per head and a second chunk of 16 rows (lq = 3: 21 rows
    # per KV head)
    cache, seg = _pair(tokens, 11, bits, group, residual, device)
    q = queries(lq, seed=13)
    logits, apply_value = cache.attention_parts(q.to(device))
    exp_logits = A.packed_logits(seg, f32(q), kv_dtype="fp32")
    assert_close(f32(logits), exp_logits, max_abs=2e-3, mean_abs=2e-4, what="logits")
    probs = torch.softmax(logits, dim=-1).to(torch.bfloat16)
    out = apply_value(probs)
    assert_close(f32(out), A.packed_pv(seg, f32(probs), kv_dtype="bf16"), what="av")
    # fp32 probabilities and an fp16 query
    logits16, apply16 = cache.attention_parts(q.half().to(device))
    assert_close(f32(logits16), A.packed_logits(seg, f32(q.half()), kv_dtype="fp32"), max_abs=2e-3,
                 mean_abs=2e-4, what="fp16-query logits")
    p32 = torch.softmax(logits16, dim=-1)
    assert_close(f32(apply16(p32)), A.packed_pv(seg, f32(p32), kv_dtype="bf16"), what="fp32-probability av")


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_summary_config0(device, bits):
    # config 0: 2048 tokens (1920 packed + 128 residual), G=32, q [1, 28, 128]
    cache, seg = _pair(2048, 0, bits, 32, 128, device)
    q = queries(1, seed=1)
    out, lse = packed_kivi_attention_summary(cache, q.to(device))
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (1, 28, 128) and tuple(lse.shape) == (28, 1)
    check_summary(out, lse, seg, q, include_residual=True)
    # the packed prefix alone (kivi_cuda.py:96-120)
    po, pl = packed_kivi_quantized_attention_summary(cache, q.to(device))
    check_summary(po, pl, seg, q, include_residual=False)


def test_decode_summary_matches_parts_and_merge(device):
    cache, seg = _pair(1536, 9, 2, 32, 128, device)
    q = queries(1, seed=3).to(device)
    out, lse = packed_kivi_attention_summary(cache, q)
    logits, apply_value = cache.attention_parts(q)
    probs = torch.softmax(logits, dim=-1)
    ref = apply_value(probs.to(torch.bfloat16)).transpose(0, 1)
    assert_close(f32(out), f32(ref), what="summary vs parts")
    assert_close(f32(lse), f32(torch.logsumexp(logits, dim=-1)), max_abs=5e-3, mean_abs=1e-3, what="lse")


def test_multi_query_summary(device):
    cache, seg = _pair(1024, 4, 4, 32, 128, device)
    q = queries(37, seed=5)
    out, lse = packed_kivi_attention_summary(cache, q.to(device))
    check_summary(out, lse, seg, q, what="mq")


def test_batched_decode_items(device):
    from unicache_amd.storage.decode import KiviDecodeBatch

    caches, segs, qs = [], [], []
    for i, tokens in enumerate((1000, 2048, 700)):
        c, s = _pair(tokens, 30 + i, 2, 32, 128, device)
        caches.append(c)
        segs.append(s)
        qs.append(queries(1, seed=40 + i))
    batch = KiviDecodeBatch(caches, [q.to(device) for q in qs])
    batch.run()
    for i in range(3):
        check_summary(batch.outputs[i], batch.lses[i], segs[i], qs[i], what=f"item {i}")


@pytest.mark.parametrize("bits", [2, 4])
def test_batched_decode_many_units_ragged(device, bits):
    # 9 items x 4 KV heads = 36 units: the launch deals a unit's splits to one
    # XCD and interleaves their super-tiles (taken at >= 32 units); ragged
    # lengths leave splits with fewer super-tiles or none, one item packs a
    # single 32-token group and one has no residual
    from unicache_amd.storage.decode import KiviDecodeBatch

    lengths = (4500, 2048, 700, 3300, 1000, 6000, 513, 2600, 160)
    caches, segs, qs = [], [], []
    for i, tokens in enumerate(lengths):
        residual = 0 if i == 1 else 128
        c, s = _pair(tokens, 60 + i, bits, 32, residual, device)
        caches.append(c)
        segs.append(s)
        qs.append(queries(1, seed=70 + i))
    batch = KiviDecodeBatch(caches, [q.to(device) for q in qs])
    batch.run()
    for i in range(len(lengths)):
        check_summary(batch.outputs[i], batch.lses[i], segs[i], qs[i], what=f"item {i} ({lengths[i]} tokens)")


@pytest.mark.parametrize("residuals", [(1, 31, 32, 33, 64, 100, 127, 128), (1, 97, 128, 129, 200, 255, 256, 257)])
def test_batched_decode_residual_split_sizes(device, residuals):
    # residual splits take 32 tokens a wave when the longest residual of the
    # launch fits one split that way (<= 128 tokens) and 64 otherwise: lengths
    # around both rules, partial waves and tiles, and one item with a single
    # packed group (dense segments without packed tokens: the segment tables
    # of test_gpu_mixed.py)
    from unicache_amd.storage.decode import KiviDecodeBatch

    caches, segs, qs = [], [], []
    for i, tr in enumerate(residuals):
        packed = 32 if i == len(residuals) - 2 else 512
        c, s = _pair(packed + tr, 80 + i, 2, 32, tr, device)
        assert c.quantized_tokens == packed and c.residual_tokens == tr
        caches.append(c)
        segs.append(s)
        qs.append(queries(1, seed=90 + i))
    batch = KiviDecodeBatch(caches, [q.to(device) for q in qs])
    batch.run()
    for i, tr in enumerate(residuals):
        check_summary(batch.outputs[i], batch.lses[i], segs[i], qs[i], what=f"item {i} (residual {tr})")


@pytest.mark.parametrize("hq,hkv,lq", [(32, 4, 1), (8, 4, 2), (16, 2, 1), (28, 4, 2), (12, 4, 3)])
def test_decode_query_rows_around_the_fold(device, hq, hkv, lq):
    # 2-bit G=32 decode with at most 8 query rows per KV head (query heads per
    # KV head x query length) uses each MFMA column half for one of a wave's two
    # key groups; 9-16 rows use all 16 columns per group.  Lengths leave waves
    # whose second half has no packed token (544 and 2464 packed tokens).
    for tokens, seed in ((700, 140), (2600, 141)):
        cache, seg = _pair(tokens, seed, 2, 32, 128, device, heads=hkv)
        q = queries(lq, heads=hq, seed=seed + 10)
        out, lse = packed_kivi_attention_summary(cache, q.to(device))
        check_summary(out, lse, seg, q, what=f"Hq {hq} Hkv {hkv} Lq {lq} T {tokens}")


def test_decode_is_deterministic(device):
    cache, _ = _pair(4096, 11, 2, 32, 128, device)
    q = queries(1, seed=2).to(device)
    a = packed_kivi_attention_summary(cache, q)
    b = packed_kivi_attention_summary(cache, q)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_gqa_helpers(device):
    key, value = kv_pair(77, seed=8)
    q = queries(5, seed=9)
    logits = gqa_query_key_logits(q.to(device), key.to(device))
    assert_close(f32(logits), A.gqa_logits(f32(q), f32(key)), max_abs=1e-3, mean_abs=1e-4, what="qk")
    p = torch.softmax(logits / math.sqrt(128), dim=-1)
    pv = gqa_probability_value(p, value.to(device))
    assert pv.dtype == torch.bfloat16
    assert_close(f32(pv), A.gqa_pv(f32(p), f32(value)), what="pv")


@pytest.mark.parametrize("lq,tokens,dtype", [(100, 300, torch.bfloat16), (70, 1000, torch.float16),
                                             (90, 301, torch.bfloat16)])
def test_gqa_logits_mfma_tiles(device, lq, tokens, dtype):
    # >= 64 query rows per KV head take the MFMA logits kernel: ragged row
    # blocks and key chunks; fp32 accumulation of up to ~100-sized products.
    # 301 keys: rows that do not start on 16 bytes take the 4-byte stores
    key, _ = kv_pair(tokens, seed=31, dtype=dtype)
    q = queries(lq, seed=32, dtype=dtype)
    got = gqa_query_key_logits(q.to(device), key.to(device))
    assert_close(f32(got), A.gqa_logits(f32(q), f32(key)), max_abs=2e-3, mean_abs=1e-4, what="qk mfma")
    # head-major storage read through strides (the H2O segment layout): same tiles, same bits
    kh = key.transpose(0, 1).contiguous().to(device).transpose(0, 1)
    assert torch.equal(gqa_query_key_logits(q.to(device), kh), got)


@pytest.mark.parametrize("pdtype,vdtype", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                           (torch.float32, torch.float16)])
def test_gqa_pv_mfma_tiles(device, pdtype, vdtype):
    # >= 64 query rows per KV head take the MFMA P.V kernel, P cast to the value
    # dtype first (physical.py:59); 301 keys end inside a 64-key tile and inside an
    # 8-key run, and the row padding past them holds NaN that must not leak in
    lq, t = 100, 301
    _, value = kv_pair(t, seed=33, dtype=vdtype)
    g = torch.Generator().manual_seed(34)
    probs = torch.softmax(torch.randn(28, lq, t, generator=g) * 3, -1)
    wide = torch.full((28, lq, 304), float("nan"))
    wide[..., :t] = probs
    got = gqa_probability_value(wide.to(pdtype).to(device)[..., :t], value.to(device))
    assert got.dtype == vdtype
    exp = A.gqa_pv(f32(probs.to(pdtype).to(vdtype)), f32(value))
    assert_close(f32(got), exp, max_abs=1e-2, mean_abs=1e-3, what="pv mfma")


def test_gqa_generic_and_mfma_routes_agree(device):
    # the same products through the MFMA tiles (contiguous inputs, >= 64 rows per
    # KV head) and through the generic kernels (fp32 query; key-strided P): both
    # within tolerance of the oracle and of each other
    key, value = kv_pair(200, seed=35)
    q = queries(80, seed=36)
    mfma = gqa_query_key_logits(q.to(device), key.to(device))
    generic = gqa_query_key_logits(q.float().to(device), key.float().to(device))
    exp = A.gqa_logits(f32(q), f32(key))
    assert_close(f32(mfma), exp, max_abs=2e-3, mean_abs=1e-4, what="qk mfma")
    assert_close(f32(generic), exp, max_abs=2e-3, mean_abs=1e-4, what="qk generic")
    p = torch.softmax(mfma / math.sqrt(128), -1).to(torch.bfloat16)
    pv_mfma = gqa_probability_value(p, value.to(device))
    pt = p.transpose(1, 2).contiguous().transpose(1, 2)  # same values, key stride != 1
    pv_generic = gqa_probability_value(pt, value.to(device))
    assert_close(f32(pv_mfma), f32(pv_generic), max_abs=1e-2, mean_abs=1e-3, what="pv routes")
    assert_close(f32(pv_mfma), A.gqa_pv(f32(p), f32(value)), what="pv oracle")


def test_lse_merge(device):
    # test_physical.py:181-202 on the GPU kernel
    torch.manual_seed(11)
    sa, sb = torch.randn(4, 3, 7), torch.randn(4, 3, 5)
    va, vb = torch.randn(4, 7, 8), torch.randn(4, 5, 8)
    summaries = [
        (torch.matmul(torch.softmax(sa, -1), va).transpose(0, 1).to(device), torch.logsumexp(sa, -1).to(device)),
        (torch.matmul(torch.softmax(sb, -1), vb).transpose(0, 1).to(device), torch.logsumexp(sb, -1).to(device)),
    ]
    out, lse = merge_attention_summaries(summaries)
    allsc = torch.cat([sa, sb], -1)
    expected = torch.matmul(torch.softmax(allsc, -1), torch.cat([va, vb], 1)).transpose(0, 1)
    assert torch.allclose(out.cpu(), expected, atol=1e-5, rtol=1e-5)
    assert torch.allclose(lse.cpu(), torch.logsumexp(allsc, -1), atol=1e-6)
    eo, el = A.merge_summaries([(f32(o), f32(l)) for o, l in summaries])
    assert np.allclose(f32(out), eo, atol=1e-6) and np.allclose(f32(lse), el, atol=1e-6)


def test_lse_merge_vector_and_row_kernels_agree(device):
    # 16-byte aligned summaries take the vector kernel, 2-byte offset ones the
    # per-row kernel: the same arithmetic, so equal bits; both match the oracle
    torch.manual_seed(12)
    lq, hq, d = 37, 28, 128
    outs = [torch.randn(lq, hq, d).to(torch.bfloat16) for _ in range(3)]
    lses = [torch.randn(hq, lq) * 4 for _ in range(3)]
    lses[1][0, :5] = -math.inf  # rows where one segment is empty
    a, la = merge_attention_summaries([(o.to(device), l.to(device)) for o, l in zip(outs, lses)])
    shifted = []
    for o in outs:
        buf = torch.empty(o.numel() + 1, dtype=torch.bfloat16, device=device)
        view = buf[1:].view(lq, hq, d)
        view.copy_(o.to(device))
        shifted.append(view)
    b, lb = merge_attention_summaries([(o, l.to(device)) for o, l in zip(shifted, lses)])
    assert torch.equal(a, b) and torch.equal(la, lb)
    eo, el = A.merge_summaries([(f32(o), f32(l)) for o, l in zip(outs, lses)])
    assert_close(f32(a), eo, what="merge")
    assert np.allclose(f32(la), el, atol=1e-5)


def test_summaries_merge_to_full_attention(device):
    # packed+residual summary merged with a dense bf16 segment equals attention over all keys
    cache, seg = _pair(1024, 12, 2, 32, 128, device)
    dk, dv = kv_pair(256, seed=13)
    q = queries(1, seed=14)
    s1 = packed_kivi_attention_summary(cache, q.to(device))
    logits = gqa_query_key_logits(q.to(device), dk.to(device)) / math.sqrt(128)
    p = torch.softmax(logits, -1)
    s2 = (gqa_probability_value(p, dv.to(device)).transpose(0, 1), torch.logsumexp(logits, -1))
    out, _ = merge_attention_summaries([s1, s2])
    key, value = K.dequantize(seg, "bf16")
    eo, _ = A.attention_summary(f32(q), np.concatenate([key, f32(dk)]), np.concatenate([value, f32(dv)]))
    assert_close(f32(out), eo, what="merged")


@pytest.mark.parametrize("bits,group,tokens,residual", [(2, 64, 3000, 300), (4, 128, 2500, 40), (2, 128, 640, 0),
                                                        (4, 32, 5000, 600)])
def test_decode_summary_groups_and_long_residual(device, bits, group, tokens, residual):
    cache, seg = _pair(tokens, 50 + bits, bits, group, residual, device)
    for lq in (1, 2):
        q = queries(lq, seed=60 + lq)
        out, lse = packed_kivi_attention_summary(cache, q.to(device))
        check_summary(out, lse, seg, q, what=f"G{group} Lq{lq}")


@pytest.mark.parametrize("bits", [2, 4])
def test_mq_config2_editing(device, bits):
    # config 2's packed segment: 1024 source-VAE tokens (896 packed + 128 residual),
    # 1088 queries x 28 heads (7616 query rows per KV head) through uc_kivi_attn_mq
    cache, seg = _pair(1024, 70 + bits, bits, 32, 128, device)
    assert (cache.quantized_tokens, cache.residual_tokens) == (896, 128)
    q = queries(1088, seed=71)
    out, lse = packed_kivi_attention_summary(cache, q.to(device))
    assert tuple(out.shape) == (1088, 28, 128) and tuple(lse.shape) == (28, 1088)
    check_summary(out, lse, seg, q, what=f"mq c2 {bits}-bit")
    po, pl = packed_kivi_quantized_attention_summary(cache, q.to(device))
    check_summary(po, pl, seg, q, include_residual=False, what=f"mq c2 packed-only {bits}-bit")


@pytest.mark.parametrize("bits,group,tokens,residual,lq", [(2, 32, 500, 20, 20), (4, 128, 700, 50, 3),
                                                           (2, 64, 1300, 130, 130), (4, 32, 96, 64, 300)])
def test_mq_ragged_tiles_and_rows(device, bits, group, tokens, residual, lq):
    # packed and residual lengths that end inside a 64-key tile, query rows that
    # end inside a 128-row workgroup
    cache, seg = _pair(tokens, 80 + lq, bits, group, residual, device)
    q = queries(lq, seed=81)
    out, lse = packed_kivi_attention_summary(cache, q.to(device))
    check_summary(out, lse, seg, q, what=f"mq G{group} T{tokens} Lq{lq}")


def test_mq_fp16_inputs(device):
    key, value = kv_pair(800, seed=90, dtype=torch.float16)
    cache = PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(800),
                                       token_type_id=3, k_bits=2, v_bits=2, group_size=32,
                                       residual_length=128, backend="cuda")
    seg = K.from_dense(f32(key), f32(value), k_bits=2, v_bits=2, group_size=32, residual_length=128,
                       in_dtype="fp16")
    q = queries(64, seed=91, dtype=torch.float16)
    out, lse = packed_kivi_attention_summary(cache, q.to(device))
    assert out.dtype == torch.float16
    eo, el = A.packed_summary(seg, f32(q), include_residual=True, kv_dtype="fp32")
    assert_close(f32(out), eo, what="mq fp16")
    assert_close(f32(lse), el, max_abs=5e-3, mean_abs=1e-3, what="mq fp16 lse")


def test_mq_is_deterministic(device):
    cache, _ = _pair(1024, 95, 2, 32, 128, device)
    q = queries(200, seed=96).to(device)
    a, la = packed_kivi_attention_summary(cache, q)
    b, lb = packed_kivi_attention_summary(cache, q)
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_batched_decode_doubled_split(device):
    # 100 items x 4 KV heads of 4096 packed + 128 residual tokens: 3 splits per
    # unit (1200 workgroups) exceed one round of slots, 2 splits (800) fit, so the
    # batch runs 16 super-tiles per split; each item alone runs 8
    from unicache_amd.storage.decode import KiviDecodeBatch

    g = torch.Generator(device=device).manual_seed(61)
    caches, qs = [], []
    for i in range(100):
        k = torch.randn(4224, 4, 128, generator=g, device=device).to(torch.bfloat16)
        v = torch.randn(4224, 4, 128, generator=g, device=device).to(torch.bfloat16)
        caches.append(PackedKIVICache.from_dense(k, v, logical_token_ids=torch.arange(4224, device=device),
                                                 token_type_id=3, k_bits=2, v_bits=2, group_size=32,
                                                 residual_length=128, backend="cuda"))
        qs.append(torch.randn(1, 28, 128, generator=g, device=device).to(torch.bfloat16))
    assert caches[0].quantized_tokens == 4096
    batch = KiviDecodeBatch(caches, qs)
    batch.run()
    for i in (0, 37, 99):
        out, lse = packed_kivi_attention_summary(caches[i], qs[i])
        assert_close(f32(batch.outputs[i]), f32(out), max_abs=5e-3, mean_abs=2e-4, what=f"item {i}")
        assert_close(f32(batch.lses[i]), f32(lse), max_abs=1e-4, mean_abs=1e-5, what=f"lse {i}")
