"""Pins oracle.kivi (the CPU restatement of UniCache's KIVI arithmetic).

Each check is a closed form, a hand-computed known answer, a shape/golden
value from UniCache's own tests, or an invariant linking two independently
written reference functions; none re-types the oracle's formula.
"""

import numpy as np
import pytest

from oracle import kivi as K


# ------------------------------------------------------------ bit layout --
def test_pack_layout_closed_form_2bit():
    # codes 0..3 repeated: word = sum_j code_j << 2j, LSB first (physical.py:81-84)
    codes = np.array([[0, 1, 2, 3] * 4], dtype=np.uint8)  # one word of 16 codes
    word = K.pack_codes(codes, 2, dim=1)
    expected = sum(c << (2 * j) for j, c in enumerate([0, 1, 2, 3] * 4))
    assert word.shape == (1, 1)
    assert int(word.view(np.uint32)[0, 0]) == expected == 0xE4E4E4E4


def test_pack_sign_wrap_top_slot():
    # a 3 in slot 15 sets bit 31: the int32 word is negative (physical.py:81-84)
    codes = np.zeros((16,), dtype=np.uint8)
    codes[15] = 3
    word = K.pack_codes(codes, 2, dim=0)
    assert word.dtype == np.int32 and int(word[0]) == -(1 << 30)
    assert int(word.view(np.uint32)[0]) == 0xC0000000


def test_pack_4bit_and_padding():
    codes = np.array([15, 0, 7, 1, 2], dtype=np.uint8)  # 5 codes -> padded to 8
    word = K.pack_codes(codes, 4, dim=0)
    assert word.shape == (1,)
    assert int(word.view(np.uint32)[0]) == 0xF | (0 << 4) | (7 << 8) | (1 << 12) | (2 << 16)
    back = K.unpack_codes(word, 4, dim=0, length=5)
    assert back.tolist() == [15, 0, 7, 1, 2]


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_round_trip_brute_force(bits):
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 1 << bits, size=(3, 37, 5), dtype=np.uint8)
    for dim in range(3):
        packed = K.pack_codes(codes, bits, dim)
        assert np.array_equal(K.unpack_codes(packed, bits, dim, codes.shape[dim]), codes)
        # every code sits at bit (index % per_word) * bits of word index // per_word
        per = 32 // bits
        flat = np.moveaxis(codes, dim, -1)
        words = np.moveaxis(packed.view(np.uint32), dim, -1)
        for idx in [(0, 0, 0), (2, 36, 4), (1, 17, 3)]:
            pos = idx[dim]
            other = tuple(i for d, i in enumerate(idx) if d != dim)
            w = int(words[other + (pos // per,)])
            assert (w >> ((pos % per) * bits)) & ((1 << bits) - 1) == int(flat[other + (pos,)])


# ----------------------------------------------------------- known answers --
def q(values, bits):
    codes, scale, mn = K.quantize_codes(np.array(values, dtype=np.float32)[:, None], bits=bits, group_dim=0,
                                        group_size=len(values))
    return codes[:, 0].tolist(), float(scale[0, 0]), float(mn[0, 0])


def test_quantize_ramp_is_identity():
    assert q([0.0, 1.0, 2.0, 3.0], 2) == ([0, 1, 2, 3], 1.0, 0.0)
    codes, scale, mn = q([float(i) for i in range(16)], 4)
    assert codes == list(range(16)) and scale == 1.0 and mn == 0.0


def test_quantize_constant_group():
    codes, scale, mn = q([1.5] * 8, 2)
    assert codes == [0] * 8 and scale == float(np.finfo(np.float32).eps) and mn == 1.5


def test_quantize_round_half_even():
    # scale 1: (x - mn) = 0.5 -> 0 and 1.5 -> 2 under round-half-even (torch.round)
    codes, scale, _ = q([0.0, 0.5, 1.5, 2.5, 3.0], 2)
    assert scale == 1.0 and codes == [0, 0, 2, 2, 3]


def test_quantize_single_max_hits_top_code():
    codes, _, _ = q([-2.0, -2.0, -2.0, 7.25], 4)
    assert codes == [0, 0, 0, 15]


def test_quantize_partial_last_group():
    data = np.arange(10, dtype=np.float32)[:, None]
    codes, scale, mn = K.quantize_codes(data, bits=2, group_dim=0, group_size=4)
    # groups [0..3], [4..7], [8, 9]
    assert scale.shape == (3, 1) and mn[:, 0].tolist() == [0.0, 4.0, 8.0]
    assert float(scale[2, 0]) == np.float32(1.0) / np.float32(3.0)
    assert codes[:, 0].tolist() == [0, 1, 2, 3, 0, 1, 2, 3, 0, 3]


# --------------------------------------------------------------- invariants --
def test_dequant_error_within_half_step():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 4, 32)).astype(np.float32)
    for bits in (2, 4, 8):
        codes, scale, mn = K.quantize_codes(x, bits=bits, group_dim=0, group_size=32)
        s = np.repeat(scale, 32, axis=0)
        m = np.repeat(mn, 32, axis=0)
        recon = codes.astype(np.float32) * s + m
        assert np.all(np.abs(recon - x) <= s * 0.5 * (1 + 1e-5))


def test_fake_quant_agrees_with_packed_codes():
    # operators/builtin.py:31-53 computes scale as max(mx-mn, eps)/max; physical.py:129
    # as max((mx-mn)/max, eps).  For non-degenerate groups both give the same codes,
    # so fake quant equals code*scale+min of the packing quantizer.
    rng = np.random.default_rng(11)
    x = K.round_bf16(rng.standard_normal((96, 2, 64)).astype(np.float32) * 3)
    for bits in (2, 4):
        for dim, gs in ((0, 32), (2, 16)):
            fq = K.fake_quant(x, bits=bits, dim=dim, group_size=gs, out_dtype="fp32")
            codes, scale, mn = K.quantize_codes(x, bits=bits, group_dim=dim, group_size=gs)
            s = np.repeat(scale, gs, axis=dim)
            m = np.repeat(mn, gs, axis=dim)
            assert np.array_equal(fq, (codes.astype(np.float32) * s).astype(np.float32) + m)


@pytest.mark.parametrize("bits,exponent", [(2, -24), (3, -25), (4, -26), (8, -27)])
def test_fake_quant_clamps_the_range_before_dividing(bits, exponent):
    # operators/builtin.py:50: scale = max(mx - mn, eps) / (2^b - 1).  For the
    # ramp k * 2^e (k = 0 .. 2^b - 1) the range r = (2^b - 1) * 2^e lies in
    # [eps, eps * (2^b - 1)), so the scale is exactly 2^e, every code is k and
    # the ramp comes back unchanged.  The packing quantizer's
    # max(r / (2^b - 1), eps) (physical.py:129) would clamp the scale to eps and
    # round the ramp to multiples of eps instead.
    top = (1 << bits) - 1
    step = np.float32(2.0 ** exponent)
    assert K.EPS <= top * step < K.EPS * top
    ramp = np.arange(top + 1, dtype=np.float32) * step
    for out_dtype in ("fp32", "bf16"):  # every ramp value has <= 8 significant bits
        assert K.fake_quant(ramp, bits=bits, dim=0, group_size=top + 1, out_dtype=out_dtype).tolist() == ramp.tolist()
    clamped_after = np.clip(np.rint(ramp / K.EPS), 0, top) * K.EPS
    assert not np.array_equal(clamped_after, ramp)  # the two formulas really differ here
    # groups along the last dim (values), two groups with their own minima
    rows = np.stack([ramp, ramp[::-1] + np.float32(0.5)])[None]  # [1, 2, top + 1]
    out = K.fake_quant(rows, bits=bits, dim=-1, group_size=top + 1, out_dtype="fp32")
    assert out.tolist() == rows.tolist()


def test_fake_quant_range_below_eps():
    # r = 3 * 2^-26 < eps at 2 bits: the scale is fl(eps / 3) and the codes of
    # 0, 2^-26, 2^-25, 3 * 2^-26 are rint(3k/8) = 0, 0, 1, 1 (scaled by 1 + O(2^-24)),
    # so the output is [0, 0, s, s]; a scale clamped after dividing (eps) would
    # give all zeros
    s = np.float32(K.EPS / np.float32(3))
    x = np.array([0, 1, 2, 3], np.float32) * np.float32(2.0 ** -26)
    assert K.fake_quant(x, bits=2, dim=0, group_size=4, out_dtype="fp32").tolist() == [0.0, 0.0, s, s]


def test_bf16_rounding_known_values():
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -0.0, np.inf, 3.0e38], dtype=np.float32)
    out = K.round_bf16(vals)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 1.5*2^-8 rounds up to 1 + 2^-7
    assert out[:4].tolist() == [1.0, 1.0, 1.0078125, 1.0078125]
    assert out[4] == 0.0 and np.signbit(out[4]) and out[5] == np.inf
    assert out[6] == np.float32(3.0040553e38)  # 0x7F61B1E6 -> 0x7F62 (low half > 0x8000)
    assert np.isnan(K.round_bf16(np.array([np.nan], dtype=np.float32)))[0]


# ------------------------------------------------------- layouts and split --
def test_residual_split_reference_cases():
    # test_physical.py:1070-1097: 320 tokens, G=128, R=32 -> 256 packed + 64 residual
    assert K.split_tokens(320, 128, 32) == (256, 64)
    assert K.split_tokens(96, 32, 16) == (64, 32)          # test_physical.py:959-982
    assert K.split_tokens(2048, 32, 128) == (1920, 128)    # config 0
    assert K.split_tokens(8192, 32, 128) == (8064, 128)    # config 1
    assert K.split_tokens(1024, 32, 128) == (896, 128)     # config 2
    assert K.split_tokens(1024, 128, 32) == (896, 128)     # engine preset on config 2
    assert K.split_tokens(20352, 32, 128) == (20224, 128)  # config 4
    assert K.split_tokens(10, 32, 4) == (0, 10)


def test_native_layout_shapes_from_reference_test():
    # test_physical.py:1047-1053: T=128, Hkv=2, D=64, G=64, 2-bit
    rng = np.random.default_rng(6)
    key = K.round_bf16(rng.standard_normal((128, 2, 64)).astype(np.float32))
    seg = K.from_dense(key, key, k_bits=2, v_bits=2, group_size=64, residual_length=0)
    assert seg.native
    assert seg.key_code.shape == (2, 64, 8)
    assert seg.key_scale.shape == (2, 64, 2)
    assert seg.value_code.shape == (2, 128, 4)
    assert seg.value_scale.shape == (2, 128, 1)
    assert np.array_equal(seg.key_scale, K.round_f16(seg.key_scale))


def test_native_and_reference_layouts_hold_the_same_codes():
    rng = np.random.default_rng(5)
    key = K.round_bf16(rng.standard_normal((96, 4, 64)).astype(np.float32))
    value = K.round_bf16(rng.standard_normal((96, 4, 64)).astype(np.float32))
    nat = K.from_dense(key, value, k_bits=4, v_bits=2, group_size=32, residual_length=0, native=True)
    ref = K.from_dense(key, value, k_bits=4, v_bits=2, group_size=32, residual_length=0, native=False)
    assert np.array_equal(np.transpose(nat.key_code, (2, 0, 1)), ref.key_code)
    assert np.array_equal(np.transpose(nat.value_code, (1, 0, 2)), ref.value_code)
    k1, v1 = K.dequantize(nat, "fp32")
    k2, v2 = K.dequantize(ref, "fp32")
    # stats differ only by their storage rounding (fp16 vs bf16)
    assert np.allclose(k1, k2, atol=0.05) and np.allclose(v1, v2, atol=0.05)


def test_round_trip_keeps_residual_exact():
    # test_physical.py:959-982
    rng = np.random.default_rng(0)
    key = K.round_bf16(rng.standard_normal((96, 4, 128)).astype(np.float32))
    value = K.round_bf16(rng.standard_normal((96, 4, 128)).astype(np.float32))
    for bits in (2, 4, 8):
        seg = K.from_dense(key, value, k_bits=bits, v_bits=bits, group_size=32, residual_length=16,
                           native=bits != 8)
        rk, rv = K.dequantize(seg, "bf16")
        assert rk.shape == key.shape
        assert np.array_equal(rk[-32:], key[-32:]) and np.array_equal(rv[-32:], value[-32:])
        assert seg.quantized_tokens % 32 == 0
        assert float(np.abs(rk - key).mean()) > 0


def test_rounding_matches_torch_casts():
    # independent implementation: torch's Float->BFloat16 / Float->Half casts
    import torch

    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-30, 30, 100000))).astype(np.float32)
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    tb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    th = torch.from_numpy(x).to(torch.float16).float().numpy()
    assert np.array_equal(K.round_bf16(x), tb)
    assert np.array_equal(K.round_f16(x), th)


@pytest.mark.parametrize("initial,appended,flush_at,group", [(128, 64, 128, 32), (100, 300, 128, 32),
                                                           (0, 1000, 128, 32), (130, 7, 160, 64), (31, 1, 32, 32)])
def test_streamed_split_matches_closed_form(initial, appended, flush_at, group):
    # flush_at is a multiple of group here, so each flush empties the window:
    # the packed count is the number of completed windows
    packed = K.streamed_split(initial, appended, flush_at=flush_at, group_size=group)
    if initial < flush_at:
        assert packed == flush_at * ((initial + appended) // flush_at)
    assert packed % group == 0 and 0 <= initial + appended - packed < flush_at + group


# ------------------------------------------------------ dequantize pinned --
def _hand_segment(native: bool) -> K.PackedSegment:
    """One KV head, 16 channels, 32 tokens, G=16, 2-bit, built word by word.

    Every key channel d holds the codes [0,1,2,3]*4 in both of its words
    (0xE4E4E4E4); group 0 has scale 0.5 / minimum -1, group 1 scale 2 /
    minimum 3.  Every value token t holds the codes [3,2,1,0]*4
    (0x1B1B1B1B) with scale 0.25 and minimum t.  All stats are exact in fp16
    and bf16, so the expected values below are exact.
    """

    word_k = np.uint32(0xE4E4E4E4).view(np.int32)
    word_v = np.uint32(0x1B1B1B1B).view(np.int32)
    kc = np.full((1, 16, 2), word_k, dtype=np.int32)               # [Hkv, D, T/16]
    ks = np.tile(np.array([0.5, 2.0], np.float32), (1, 16, 1))     # [Hkv, D, T/G]
    km = np.tile(np.array([-1.0, 3.0], np.float32), (1, 16, 1))
    vc = np.full((1, 32, 1), word_v, dtype=np.int32)               # [Hkv, T, D/16]
    vs = np.full((1, 32, 1), 0.25, np.float32)                     # [Hkv, T, D/G]
    vm = np.arange(32, dtype=np.float32).reshape(1, 32, 1)
    if not native:  # UniCache's reference layout: K [T/16, Hkv, D], V [T, Hkv, D/16]
        kc, ks, km = (np.ascontiguousarray(np.transpose(a, (2, 0, 1))) for a in (kc, ks, km))
        vc, vs, vm = (np.ascontiguousarray(np.transpose(a, (1, 0, 2))) for a in (vc, vs, vm))
    empty = np.zeros((0, 1, 16), np.float32)
    return K.PackedSegment(kc, ks, km, vc, vs, vm, empty, empty, k_bits=2, v_bits=2, group_size=16,
                           quantized_tokens=32, native=native)


@pytest.mark.parametrize("native", [True, False])
def test_dequantize_hand_built_words(native):
    key, value = K.dequantize(_hand_segment(native), "fp32")
    assert key.shape == (32, 1, 16) and value.shape == (32, 1, 16)
    # keys: token t of channel d has code t % 4; group 0 -> code*0.5 - 1, group 1 -> code*2 + 3
    assert key[:16, 0, 0].tolist() == [-1.0, -0.5, 0.0, 0.5] * 4
    assert key[16:, 0, 0].tolist() == [3.0, 5.0, 7.0, 9.0] * 4
    assert np.array_equal(key, np.broadcast_to(key[:, :, :1], key.shape))  # same in every channel
    # values: channel c of token t has code 3 - c % 4, scale 0.25, minimum t
    assert value[0, 0].tolist() == [0.75, 0.5, 0.25, 0.0] * 4
    assert value[5, 0].tolist() == [5.75, 5.5, 5.25, 5.0] * 4
    assert value[31, 0, :4].tolist() == [31.75, 31.5, 31.25, 31.0]


def test_dequantize_hand_built_bf16_cast():
    # with minimum 3 + 2^-6: 3 + 2^-6 is a bf16 value, 9 + 2^-6 is not and the
    # output cast rounds it to 9 (a quarter ulp away)
    seg = _hand_segment(True)
    seg.key_minimum = seg.key_minimum + np.float32(2.0 ** -6)
    key, _ = K.dequantize(seg, "bf16")
    assert key[16, 0, 0] == 3.015625 and key[19, 0, 0] == 9.0 and key[0, 0, 0] == -0.984375


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_round_trip_error_bound_per_element(bits):
    # |dequant(quant(x)) - x| <= s/2 from the rounding of the code, plus what
    # storing s and m in fp16 (native) or bf16 (reference layout) and the final
    # bf16 cast add: code*|s'-s| + |m'-m| + half an output ulp.
    rng = np.random.default_rng(21 + bits)
    key = rng.standard_normal((160, 2, 64)).astype(np.float32)
    key[:, :, 5] *= 10.0
    key = K.round_bf16(key)
    value = K.round_bf16(rng.standard_normal((160, 2, 64)).astype(np.float32))
    native = bits != 8
    seg = K.from_dense(key, value, k_bits=bits, v_bits=bits, group_size=32, residual_length=0, native=native)
    rk, rv = K.dequantize(seg, "bf16")
    storage_ulp = 2.0 ** -10 if native else 2.0 ** -7  # relative half-ulp of fp16 / bf16 stats
    top = (1 << bits) - 1
    for x, r, gdim in ((key, rk, 0), (value, rv, 2)):
        _, scale, mn = K.quantize_codes(x, bits=bits, group_dim=gdim, group_size=32)
        s = np.repeat(scale, 32, axis=gdim).astype(np.float64)
        m = np.repeat(mn, 32, axis=gdim).astype(np.float64)
        bound = s / 2 * (1 + 1e-5) + top * s * storage_ulp + np.abs(m) * storage_ulp \
            + np.abs(r.astype(np.float64)) * 2.0 ** -8
        err = np.abs(r.astype(np.float64) - x)
        assert np.all(err <= bound), float((err - bound).max())
        # and the bound is tight enough to mean something: most errors use < s/2
        assert float(np.mean(err <= s / 2 + 1e-6)) > 0.5


def test_native_mean_error_not_worse_than_reference_layout():
    # test_physical.py:1056-1068: the kernel-native cache's mean reconstruction
    # error is at most 1.1x the reference layout's plus 1e-3
    rng = np.random.default_rng(6)
    key = K.round_bf16(rng.standard_normal((128, 2, 64)).astype(np.float32))
    value = K.round_bf16(rng.standard_normal((128, 2, 64)).astype(np.float32))
    nat = K.from_dense(key, value, k_bits=2, v_bits=2, group_size=64, residual_length=0, native=True)
    ref = K.from_dense(key, value, k_bits=2, v_bits=2, group_size=64, residual_length=0, native=False)
    for original, native_out, ref_out in zip((key, value), K.dequantize(nat, "bf16"), K.dequantize(ref, "bf16")):
        assert np.isfinite(native_out).all()
        native_error = np.abs(native_out - original).mean()
        ref_error = np.abs(ref_out - original).mean()
        assert native_error <= ref_error * 1.10 + 1e-3
        # 2-bit codes over G=64 leave a mean error well under one scale step
        assert 0.05 < native_error < 0.5


def test_non_finite_groups_follow_torch():
    # torch.amin / amax propagate NaN and clamp_min keeps it: a group with a NaN
    # gets NaN scale and minimum, codes 0, and dequantizes to NaN; a +inf
    # element gives an inf scale (every other code 0)
    with np.errstate(invalid="ignore"):
        codes, scale, mn = K.quantize_codes(np.array([[1.0], [np.nan], [3.0], [2.0]], np.float32), bits=2,
                                            group_dim=0, group_size=4)
        assert codes[:, 0].tolist() == [0, 0, 0, 0] and np.isnan(scale[0, 0]) and np.isnan(mn[0, 0])
        codes, scale, mn = K.quantize_codes(np.array([[1.0], [np.inf], [3.0], [2.0]], np.float32), bits=2,
                                            group_dim=0, group_size=4)
        assert codes[:, 0].tolist() == [0, 0, 0, 0] and scale[0, 0] == np.inf and mn[0, 0] == 1.0
        fq = K.fake_quant(np.array([0.0, np.nan, 2.0, 3.0], np.float32), bits=2, dim=0, group_size=4,
                          out_dtype="fp32")
        assert np.isnan(fq).all()
        fq = K.fake_quant(np.array([0.0, 1.0, 2.0, 3.0], np.float32), bits=2, dim=0, group_size=4,
                          out_dtype="fp32")
        assert fq.tolist() == [0.0, 1.0, 2.0, 3.0]
