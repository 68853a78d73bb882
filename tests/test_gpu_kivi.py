"""GPU parity of KIVI pack / dequantize / fake quant: bit-exact with the oracle."""

import numpy as np
import pytest
import torch

from oracle import kivi as K
from tests.helpers import f32, kv_pair, queries
from unicache_amd.operators import asymmetric_fake_quant, kivi_fake_quant_key, kivi_fake_quant_value
from unicache_amd.storage import PackedKIVICache
from unicache_amd.storage.kivi_cuda import dequantize_kivi_chunk, quantize_kivi_native

pytestmark = pytest.mark.gpu


def _cache(key, value, device, **kw):
    t = key.shape[0]
    return PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(t),
                                      token_type_id=3, backend="cuda", **kw)


def _assert_cache_equal(cache, seg):
    assert cache.quantized_tokens == seg.quantized_tokens
    assert cache.kernel_native_layout == seg.native
    for name in ("key_code", "value_code"):
        got = getattr(cache, name).cpu().numpy()
        exp = getattr(seg, name)
        assert got.shape == exp.shape, name
        assert np.array_equal(got.view(exp.dtype) if got.dtype != exp.dtype else got, exp), name
    for name in ("key_scale", "key_minimum", "value_scale", "value_minimum"):
        assert np.array_equal(f32(getattr(cache, name)), getattr(seg, name)), name
    assert np.array_equal(f32(cache.residual_key), seg.residual_key)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_native_pack_bit_exact(device, bits, group):
    # the shapes and seed of test_physical.py:984-1015
    torch.manual_seed(19)
    key = torch.randn(256, 4, 128, dtype=torch.bfloat16)
    value = torch.randn(256, 4, 128, dtype=torch.bfloat16)
    cache = _cache(key, value, device, k_bits=bits, v_bits=bits, group_size=group, residual_length=0)
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=group, residual_length=0)
    _assert_cache_equal(cache, seg)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_codes_at_exact_half_steps(device, bits):
    # integer-valued groups whose range is an even multiple of the code count:
    # (x - min) / scale lands exactly on halves, where the code is decided by
    # round-half-even of the correctly rounded quotient (the kernels' exact
    # fallback, not their reciprocal fast path), for keys and values alike
    top = (1 << bits) - 1
    t = torch.arange(256, dtype=torch.float32)
    ramp = (t % (2 * top + 1))[:, None, None] + torch.arange(128, dtype=torch.float32)[None, None, :] % 3
    key = (ramp.expand(256, 4, 128) + torch.arange(4, dtype=torch.float32)[None, :, None]).to(torch.bfloat16)
    value = key.flip(0).contiguous()
    cache = _cache(key, value, device, k_bits=bits, v_bits=bits, group_size=32, residual_length=0)
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=32, residual_length=0,
                       native=True, in_dtype="bf16")
    _assert_cache_equal(cache, seg)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("group", [16, 32, 64])
@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16")])
def test_pack_groups_dtypes_half_steps_and_non_finite(device, bits, group, dtype, name):
    # random rows, integer ramps whose quotients land exactly on half steps in
    # some lanes (the exact recomputation inside an otherwise reciprocal-rounded
    # group), one NaN and one inf per tensor: keys and values, every group size
    # and 16-bit input the 2/4-bit kernel-native pack takes
    tokens = 4 * group + 2 * 64
    g = torch.Generator().manual_seed(100 * bits + group)
    key = torch.randn(tokens, 4, 128, generator=g)
    value = torch.randn(tokens, 4, 128, generator=g)
    top = (1 << bits) - 1
    ramp = torch.arange(group, dtype=torch.float32) % (2 * top + 1)
    key[group:2 * group, 1, 10:20] = ramp[:, None]          # key groups along tokens
    value[5, 2, :group] = ramp                              # one value group along channels
    key[3 * group + 1, 3, 77] = float("nan")
    value[7, 0, 100] = float("inf")
    key, value = key.to(dtype), value.to(dtype)
    cache = _cache(key, value, device, k_bits=bits, v_bits=bits, group_size=group, residual_length=0)
    with np.errstate(invalid="ignore"):
        seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=group, residual_length=0,
                           native=True, in_dtype=name)
    assert cache.kernel_native_layout
    for attr in ("key_code", "value_code"):
        assert np.array_equal(getattr(cache, attr).cpu().numpy(), getattr(seg, attr)), attr
    for attr in ("key_scale", "key_minimum", "value_scale", "value_minimum"):
        assert np.array_equal(f32(getattr(cache, attr)), getattr(seg, attr), equal_nan=True), attr


def test_config0_pack_with_outliers_and_residual(device):
    key, value = kv_pair(2048, seed=0)
    cache = _cache(key, value, device, k_bits=2, v_bits=2, group_size=32, residual_length=128)
    seg = K.from_dense(f32(key), f32(value), k_bits=2, v_bits=2, group_size=32, residual_length=128)
    assert (cache.quantized_tokens, cache.residual_tokens) == (1920, 128)
    assert tuple(cache.key_code.shape) == (4, 128, 120) and tuple(cache.value_code.shape) == (4, 1920, 8)
    _assert_cache_equal(cache, seg)
    # residual is a compact clone (test_physical.py:1070-1097)
    assert cache.residual_key.untyped_storage().nbytes() == cache.residual_key.numel() * 2


@pytest.mark.parametrize("kb,vb", [(4, 2), (2, 4), (8, 8), (8, 2)])
def test_mixed_and_8bit_layouts(device, kb, vb):
    key, value = kv_pair(192, heads=2, head_dim=64, seed=3)
    cache = _cache(key, value, device, k_bits=kb, v_bits=vb, group_size=32, residual_length=40)
    seg = K.from_dense(f32(key), f32(value), k_bits=kb, v_bits=vb, group_size=32, residual_length=40,
                       native=True, in_dtype="bf16")
    _assert_cache_equal(cache, seg)
    rk, rv = cache.dequantize(torch.bfloat16)
    ok, ov = K.dequantize(seg, "bf16")
    assert np.array_equal(f32(rk), ok) and np.array_equal(f32(rv), ov)


@pytest.mark.parametrize("bits,group,head_dim,tokens", [(4, 8, 16, 72), (2, 12, 64, 100), (2, 48, 128, 200),
                                                       (8, 96, 128, 200), (4, 5, 16, 61), (2, 128, 64, 300)])
def test_reference_backend_any_group(device, bits, group, head_dim, tokens):
    # backend="reference" takes any positive group (physical.py:247-248): key
    # groups along tokens, value groups along channels ending in a partial group
    # when head_dim % group != 0, code words shared by groups and zero-padded;
    # codes, stats (in the input dtype) and the dequantized tensors bit-exact
    key, value = kv_pair(tokens, heads=2, head_dim=head_dim, seed=200 + group, outliers=2)
    cache = PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(tokens),
                                       token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                       residual_length=20, backend="reference")
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=group, residual_length=20,
                       native=False, in_dtype="bf16")
    assert not cache.kernel_native_layout and cache.quantized_tokens == seg.quantized_tokens > 0
    _assert_cache_equal(cache, seg)
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float32, "fp32")):
        rk, rv = cache.dequantize(dtype)
        ok, ov = K.dequantize(seg, name)
        assert np.array_equal(f32(rk), ok) and np.array_equal(f32(rv), ov), name
    # the reference backend attends by dequantizing (physical.py:452-475)
    q = queries(2, heads=4, head_dim=head_dim, seed=5)
    logits, apply_value = cache.attention_parts(q.to(device))
    from oracle import attention as A

    exp = A.packed_logits(seg, f32(q), kv_dtype="bf16")
    assert np.allclose(f32(logits), exp, atol=2e-2 * max(1.0, float(np.abs(exp).max())) / 50)


def test_native_layout_keeps_its_group_sizes(device):
    key, value = kv_pair(64, heads=2, head_dim=16, seed=3)
    with pytest.raises(ValueError):
        PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(64),
                                   token_type_id=3, k_bits=4, v_bits=4, group_size=8, residual_length=8,
                                   backend="cuda")
    with pytest.raises(ValueError):
        PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(64),
                                   token_type_id=3, k_bits=4, v_bits=4, group_size=0, residual_length=8,
                                   backend="reference")


def test_fp16_and_strided_inputs(device):
    key, value = kv_pair(128, seed=4, dtype=torch.float16)
    seg = K.from_dense(f32(key), f32(value), k_bits=4, v_bits=4, group_size=64, residual_length=0)
    _assert_cache_equal(_cache(key, value, device, k_bits=4, v_bits=4, group_size=64, residual_length=0), seg)
    # channel stride 2 (scalar path) and a head-major view (token stride != H*D)
    wide = torch.randn(128, 4, 256, dtype=torch.bfloat16)
    k2 = wide[:, :, ::2]
    v2 = torch.randn(4, 128, 128, dtype=torch.bfloat16).transpose(0, 1)
    seg2 = K.from_dense(f32(k2), f32(v2), k_bits=2, v_bits=2, group_size=32, residual_length=0)
    wide_d = wide.to(device)
    v2_d = v2.to(device)  # preserve_format keeps the head-major strides
    assert v2_d.stride() == v2.stride()
    c2 = PackedKIVICache.from_dense(wide_d[:, :, ::2], v2_d, logical_token_ids=torch.arange(128), token_type_id=3,
                                    k_bits=2, v_bits=2, group_size=32, residual_length=0, backend="cuda")
    _assert_cache_equal(c2, seg2)


def test_quantize_kivi_native_signature(device):
    key, value = kv_pair(64, heads=2, head_dim=64, seed=6)
    out = quantize_kivi_native(key.to(device), value.to(device), k_bits=2, v_bits=2, group_size=64)
    shapes = [tuple(t.shape) for t in out]
    # test_physical.py:1047-1053 (T=64 here: half the words)
    assert shapes == [(2, 64, 4), (2, 64, 1), (2, 64, 1), (2, 64, 4), (2, 64, 1), (2, 64, 1)]
    assert all(t.dtype == torch.float16 for t in out[1:3] + out[4:])


@pytest.mark.parametrize("bits", [2, 4])
def test_dequantize_bit_exact(device, bits):
    key, value = kv_pair(384, seed=13)
    cache = _cache(key, value, device, k_bits=bits, v_bits=bits, group_size=32, residual_length=100)
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=32, residual_length=100)
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")):
        rk, rv = cache.dequantize(dtype)
        ok, ov = K.dequantize(seg, name)
        assert np.array_equal(f32(rk), ok) and np.array_equal(f32(rv), ov), name


@pytest.mark.parametrize("bits", [2, 4])
def test_chunk_dequant_into_workspace(device, bits):
    # test_physical.py:650-688
    torch.manual_seed(13)
    key = torch.randn(384, 4, 128, dtype=torch.bfloat16)
    value = torch.randn_like(key)
    cache = _cache(key, value, device, k_bits=bits, v_bits=bits, group_size=128, residual_length=0)
    ek, ev = cache.dequantize(dtype=torch.bfloat16)
    ak, av = dequantize_kivi_chunk(cache, start=128, stop=384, dtype=torch.bfloat16)
    assert torch.equal(ak, ek[128:384]) and torch.equal(av, ev[128:384])
    wk = torch.full((300, 4, 128), -7.0, device=device, dtype=torch.bfloat16)
    wv = torch.full_like(wk, -9.0)
    dk, dv = dequantize_kivi_chunk(cache, start=128, stop=384, dtype=torch.bfloat16, output_key=wk,
                                   output_value=wv, output_offset=16)
    assert torch.equal(dk, ek[128:384]) and torch.equal(dv, ev[128:384])
    assert torch.all(wk[:16] == -7.0) and torch.all(wv[:16] == -9.0)
    assert torch.all(wk[272:] == -7.0)
    # unaligned start inside a word and a group
    uk, uv = dequantize_kivi_chunk(cache, start=37, stop=301, dtype=torch.bfloat16)
    assert torch.equal(uk, ek[37:301]) and torch.equal(uv, ev[37:301])
    with pytest.raises(ValueError):
        dequantize_kivi_chunk(cache, start=0, stop=384, dtype=torch.bfloat16, output_key=wk, output_value=wv)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_fake_quant_bit_exact(device, bits):
    key, value = kv_pair(200, seed=21)  # 200 tokens: a partial last key group
    for fn, dim in ((kivi_fake_quant_key, 0), (kivi_fake_quant_value, 2)):
        got = fn(key.to(device) if dim == 0 else value.to(device), bits=bits, group_size=32)
        src = key if dim == 0 else value
        exp = K.fake_quant(f32(src), bits=bits, dim=dim, group_size=32, out_dtype="bf16")
        assert got.dtype == torch.bfloat16
        assert np.array_equal(f32(got), exp), (bits, dim)
    assert asymmetric_fake_quant(key.to(device), bits=16, dim=0, group_size=32) is not None


def _group_ends(x, dim, group, lo, hi):
    # the first element of every group along `dim` is lo and the second hi, so
    # each group's minimum and maximum are known
    idx = torch.arange(x.shape[dim]) % group
    shape = [1, 1, 1]
    shape[dim] = -1
    idx = idx.view(shape).expand_as(x)
    return torch.where(idx == 0, torch.full_like(x, lo), torch.where(idx == 1, torch.full_like(x, hi), x))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float32, "fp32")])
def test_fake_quant_at_exact_half_steps(device, bits, dtype, name):
    # integer groups with minimum 0 and maximum 2(2^b - 1): the scale is exactly
    # 2, so every odd element's (x - min) / scale is a half, decided by
    # round-half-even of the correctly rounded quotient (the kernels' exact
    # fallback).  Keys along tokens (200 tokens: a partial last group), values
    # along channels; integers up to 256 (and 510) are exact in bf16.
    top = (1 << bits) - 1
    hi = 2 * top
    g = torch.Generator().manual_seed(40 + bits)
    base = torch.randint(0, min(hi, 256) + 1, (200, 4, 128), generator=g).to(torch.float32)
    for fn, dim in ((kivi_fake_quant_key, 0), (kivi_fake_quant_value, 2)):
        src = _group_ends(base, dim, 32, 0.0, float(hi)).to(dtype)
        got = fn(src.to(device), bits=bits, group_size=32)
        exp = K.fake_quant(f32(src), bits=bits, dim=dim, group_size=32, out_dtype=name)
        assert np.array_equal(f32(got), exp), (bits, dim)


@pytest.mark.parametrize("bits,exponent", [(2, -24), (3, -25), (4, -26), (8, -27)])
def test_fake_quant_range_below_eps_times_codes(device, bits, exponent):
    # groups whose range r satisfies eps <= r < eps * (2^b - 1) (and some below
    # eps): operators/builtin.py:50 clamps the range, then divides, so the scale
    # is below eps; a scale clamped after the division would be eps.  The
    # elements are k * 2^e * 2^j with k <= 2^b - 1 and j in 0..3 (keys), exact
    # in bf16, and every group holds k = 0 and k = 2^b - 1, so its scale is
    # exactly 2^(e + j) and every code is k.
    top = (1 << bits) - 1
    g = torch.Generator().manual_seed(60 + bits)
    k = torch.randint(0, top + 1, (200, 4, 128), generator=g).to(torch.float32)
    col = (torch.arange(128) % 4).to(torch.float32).view(1, 1, -1)
    for fn, dim in ((kivi_fake_quant_key, 0), (kivi_fake_quant_value, 2)):
        steps = _group_ends(k, dim, 32, 0.0, float(top)) * (2.0 ** exponent)
        src = (steps * torch.exp2(col if dim == 0 else torch.zeros_like(col))).to(torch.bfloat16)
        got = fn(src.to(device), bits=bits, group_size=32)
        exp = K.fake_quant(f32(src), bits=bits, dim=dim, group_size=32, out_dtype="bf16")
        assert np.array_equal(f32(got), exp), (bits, dim)
        assert torch.equal(got.cpu(), src)  # every scale is the exact step: the output is the input


@pytest.mark.parametrize("group,dtype,name", [(16, torch.float16, "fp16"), (64, torch.bfloat16, "bf16"),
                                              (128, torch.bfloat16, "bf16"), (32, torch.float32, "fp32")])
def test_fake_quant_groups_and_dtypes(device, group, dtype, name):
    # token groups held in registers (16, 64), channel groups over 2 and 8 lanes,
    # and the element-wise kernel (group 128, fp32 data); 300 tokens leave a
    # partial last key group
    key, value = kv_pair(300, seed=22, dtype=dtype)
    for fn, dim in ((kivi_fake_quant_key, 0), (kivi_fake_quant_value, 2)):
        src = key if dim == 0 else value
        got = fn(src.to(device), bits=4, group_size=group)
        exp = K.fake_quant(f32(src), bits=4, dim=dim, group_size=group, out_dtype=name)
        assert got.dtype == dtype
        assert np.array_equal(f32(got), exp), (group, dim)


@pytest.mark.parametrize("bits", [2, 4])
def test_dequantize_long_chunks_and_fp16_stats(device, bits):
    # whole-run and partial-run key words (start/stop inside words and runs),
    # fp16 input with fp16 stats, output into a wider workspace
    key, value = kv_pair(1024, seed=23, dtype=torch.float16)
    cache = _cache(key, value, device, k_bits=bits, v_bits=bits, group_size=16, residual_length=0)
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=16, residual_length=0,
                       in_dtype="fp16")
    ek, ev = K.dequantize(seg, "fp16")
    assert cache.quantized_tokens == 1024
    for start, stop in ((0, 1024), (5, 1023), (64, 128), (17, 18), (300, 701)):
        wk = torch.zeros((stop - start + 9, 4, 128), device=device, dtype=torch.float16)
        wv = torch.zeros_like(wk)
        dk, dv = dequantize_kivi_chunk(cache, start=start, stop=stop, dtype=torch.float16, output_key=wk,
                                       output_value=wv, output_offset=9)
        assert np.array_equal(f32(dk), ek[start:stop]) and np.array_equal(f32(dv), ev[start:stop]), (start, stop)
        assert torch.all(wk[:9] == 0) and torch.all(wv[:9] == 0)


def test_pack_is_deterministic(device):
    key, value = kv_pair(512, seed=2)
    a = _cache(key, value, device, k_bits=2, v_bits=2, group_size=32, residual_length=128)
    b = _cache(key, value, device, k_bits=2, v_bits=2, group_size=32, residual_length=128)
    assert torch.equal(a.key_code, b.key_code) and torch.equal(a.value_minimum, b.value_minimum)


def test_repack_monotonic(device):
    # test_physical.py:1099-1132
    key, value = kv_pair(256, heads=2, head_dim=64, seed=1)
    cache = _cache(key, value, device, k_bits=4, v_bits=4, group_size=32, residual_length=32)
    assert cache.repack_monotonic(bits=2, group_size=64)
    assert cache.k_bits == 2 and cache.group_size == 64
    assert not cache.repack_monotonic(bits=4, group_size=64)
    assert cache.budget_shortfall_events == 1
    assert cache.resident_bytes < cache.full_precision_bytes


def test_repack_after_streaming_frees_the_streamed_storage(device):
    # a flush grows the packed storage (owned by the cache) and appends keep a
    # residual window buffer; repack_monotonic replaces both, so the memory
    # they held is released, and streaming continues on the new packing
    import gc

    key, value = kv_pair(1600, seed=150)
    kd, vd = key.to(device), value.to(device)
    ids = torch.arange(1600)
    cache = PackedKIVICache.from_dense(kd[:1000], vd[:1000], logical_token_ids=ids[:1000], token_type_id=3,
                                       k_bits=4, v_bits=4, group_size=32, residual_length=128, backend="cuda")
    for t in range(1000, 1300):
        cache.append(kd[t:t + 1], vd[t:t + 1], logical_token_ids=ids[t:t + 1], flush_at=128)
    owner, store = cache._store
    assert owner == id(cache) and cache.packed_capacity >= cache.quantized_tokens
    streamed = store[0].untyped_storage().nbytes() + cache._residual_capacity.untyped_storage().nbytes()
    dk, dv = cache.dequantize(torch.bfloat16)  # what the repack re-packs
    del owner, store
    gc.collect()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(device)
    assert cache.repack_monotonic(bits=2, group_size=64)
    gc.collect()
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated(device)
    assert "_store" not in cache.__dict__ and "_residual_capacity" not in cache.__dict__
    new = cache.key_code.untyped_storage().nbytes() + 2 * cache.residual_key.untyped_storage().nbytes()
    assert after <= before - streamed + new + (1 << 16), (before, after, streamed, new)
    # appends and flushes after the repack equal packing the same tokens at once
    tail = torch.cat([dk, kd[1300:]]), torch.cat([dv, vd[1300:]])
    for t in range(1300, 1600):
        cache.append(kd[t:t + 1], vd[t:t + 1], logical_token_ids=ids[t:t + 1], flush_at=128)
    ref = PackedKIVICache.from_dense(tail[0], tail[1], logical_token_ids=ids, token_type_id=3, k_bits=2, v_bits=2,
                                     group_size=64, residual_length=1600 - cache.quantized_tokens, backend="cuda")
    assert ref.quantized_tokens == cache.quantized_tokens
    for name in ("key_code", "key_scale", "key_minimum", "value_code", "value_scale", "value_minimum",
                 "residual_key", "residual_value"):
        assert torch.equal(getattr(cache, name), getattr(ref, name)), name
    assert torch.equal(cache.logical_token_ids.cpu(), ids)


@pytest.mark.parametrize("bits,group,tokens,appended", [(2, 32, 1000, 300), (4, 64, 640, 200), (2, 128, 300, 170)])
def test_streaming_append_flush_equals_from_dense(device, bits, group, tokens, appended):
    # decode appends one token per step and flushes the residual at 128 tokens;
    # the result must be bit-identical to packing the same tokens in one go
    key, value = kv_pair(tokens + appended, seed=120 + bits)
    kd, vd = key.to(device), value.to(device)
    ids = torch.arange(tokens + appended)
    cache = PackedKIVICache.from_dense(kd[:tokens], vd[:tokens], logical_token_ids=ids[:tokens], token_type_id=3,
                                       k_bits=bits, v_bits=bits, group_size=group, residual_length=128,
                                       backend="cuda")
    tq0, tr0 = cache.quantized_tokens, cache.residual_tokens
    flushed = in_place = 0
    for t in range(tokens, tokens + appended):
        before = (cache.key_code.data_ptr(), cache.packed_capacity)
        n = cache.append(kd[t:t + 1], vd[t:t + 1], logical_token_ids=ids[t:t + 1], flush_at=128)
        flushed += n
        assert cache.quantized_tokens <= cache.packed_capacity and cache.packed_capacity % group == 0
        # a flush appends rows in place while the storage has room, else grows it by half
        if n and before[1] >= cache.quantized_tokens:
            assert (cache.key_code.data_ptr(), cache.packed_capacity) == before
            in_place += 1
        elif n:
            assert cache.packed_capacity >= before[1] + before[1] // 2
    assert flushed == 0 or in_place or cache.packed_capacity == cache.quantized_tokens
    expect_packed = tq0 + K.streamed_split(tr0, appended, flush_at=128, group_size=group)
    assert cache.quantized_tokens == expect_packed == tq0 + flushed
    total = tokens + appended
    ref = PackedKIVICache.from_dense(kd, vd, logical_token_ids=ids, token_type_id=3, k_bits=bits, v_bits=bits,
                                     group_size=group, residual_length=total - expect_packed, backend="cuda")
    assert ref.quantized_tokens == expect_packed
    for name in ("key_code", "key_scale", "key_minimum", "value_code", "value_scale", "value_minimum",
                 "residual_key", "residual_value"):
        assert torch.equal(getattr(cache, name), getattr(ref, name)), name
    assert torch.equal(cache.logical_token_ids.cpu(), ids)
    # and the oracle's packing of the flushed prefix
    seg = K.from_dense(f32(key), f32(value), k_bits=bits, v_bits=bits, group_size=group,
                       residual_length=total - expect_packed)
    assert np.array_equal(cache.key_code.cpu().numpy().view(np.uint32), seg.key_code.view(np.uint32))
    assert np.array_equal(cache.value_code.cpu().numpy().view(np.uint32), seg.value_code.view(np.uint32))


def test_streaming_decode_matches_fresh_cache(device):
    key, value = kv_pair(1500, seed=131)
    kd, vd = key.to(device), value.to(device)
    ids = torch.arange(1500)
    cache = PackedKIVICache.from_dense(kd[:1200], vd[:1200], logical_token_ids=ids[:1200], token_type_id=3,
                                       k_bits=2, v_bits=2, group_size=32, residual_length=128, backend="cuda")
    for t in range(1200, 1500):
        cache.append(kd[t:t + 1], vd[t:t + 1], logical_token_ids=ids[t:t + 1], flush_at=128)
    fresh = PackedKIVICache.from_dense(kd, vd, logical_token_ids=ids, token_type_id=3, k_bits=2, v_bits=2,
                                       group_size=32, residual_length=1500 - cache.quantized_tokens, backend="cuda")
    from unicache_amd.storage.kivi_cuda import packed_kivi_attention_summary

    q = queries(1, seed=132).to(device)
    a, la = packed_kivi_attention_summary(cache, q)
    b, lb = packed_kivi_attention_summary(fresh, q)
    assert torch.equal(a, b) and torch.equal(la, lb)


@pytest.mark.parametrize("native", [True, False])
def test_non_finite_inputs_match_oracle(device, native):
    # NaN and +/-inf inside some key and value groups: torch.amin / amax
    # propagate NaN (NaN stats, codes 0), inf gives inf / NaN stats; codes must
    # match bit for bit and stats as values (NaN where the oracle has NaN)
    key, value = kv_pair(256, seed=17)
    key[5, 1, 7] = float("nan")        # key group 0 of (head 1, channel 7)
    key[70, 2, 100] = float("inf")     # key group 2 of (head 2, channel 100)
    key[200, 0, 3] = float("-inf")
    value[9, 3, 40] = float("nan")     # value group 1 of (token 9, head 3)
    value[100, 0, 127] = float("inf")
    cache = PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(256),
                                       token_type_id=3, k_bits=2, v_bits=2, group_size=32, residual_length=0,
                                       backend="cuda" if native else "reference")
    with np.errstate(invalid="ignore"):
        seg = K.from_dense(f32(key), f32(value), k_bits=2, v_bits=2, group_size=32, residual_length=0,
                           native=native)
    assert cache.kernel_native_layout == seg.native
    for name in ("key_code", "value_code"):
        assert np.array_equal(getattr(cache, name).cpu().numpy(), getattr(seg, name)), name
    for name in ("key_scale", "key_minimum", "value_scale", "value_minimum"):
        assert np.array_equal(f32(getattr(cache, name)), getattr(seg, name), equal_nan=True), name
    assert np.isnan(f32(cache.key_scale)).sum() == 1 and np.isnan(f32(cache.value_minimum)).sum() == 1
    # fake quant of the same tensors
    from unicache_amd.operators import kivi_fake_quant_key, kivi_fake_quant_value

    with np.errstate(invalid="ignore"):
        fk = K.fake_quant(f32(key), bits=2, dim=0, group_size=32)
        fv = K.fake_quant(f32(value), bits=2, dim=-1, group_size=32)
    assert np.array_equal(f32(kivi_fake_quant_key(key.to(device), bits=2, group_size=32)), fk, equal_nan=True)
    assert np.array_equal(f32(kivi_fake_quant_value(value.to(device), bits=2, group_size=32)), fv, equal_nan=True)
