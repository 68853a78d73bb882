"""numpy restatement of UniCache's KIVI quantize / pack / dequantize.

Values are carried as float32 arrays; "bf16" / "fp16" data are float32 arrays
whose values are exactly representable in that format (see round_bf16 /
round_f16).  Every arithmetic step is a float32 numpy ufunc, i.e. one IEEE
rounding per operation, in the order of the torch code cited.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

F32 = np.float32
EPS = np.float32(np.finfo(np.float32).eps)  # torch.finfo(torch.float32).eps


# ------------------------------------------------------------- rounding --
def round_bf16(x) -> np.ndarray:
    """float32 -> nearest-even bfloat16 value (as float32), NaN -> 0x7fc0
    (torch's Float->BFloat16 cast)."""

    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, 0x7FC00000, r).astype(np.uint32)
    return r.view(np.float32).reshape(a.shape)


def round_f16(x) -> np.ndarray:
    """float32 -> nearest-even float16 value (as float32)."""

    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return round_f16(x)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


# ---------------------------------------------------------------- packing --
def pack_codes(codes: np.ndarray, bits: int, dim: int) -> np.ndarray:
    """physical.py:66-85.  2/4-bit codes -> int32 words, code j of a word at
    bit j*bits (LSB first) along `dim`, zero-padded to a multiple of 32/bits.
    8-bit codes stay uint8."""

    if bits == 8:
        return codes.astype(np.uint8)
    if bits not in (2, 4):
        raise ValueError(bits)
    dim = dim % codes.ndim
    factor = 32 // bits
    moved = np.moveaxis(codes.astype(np.uint32), dim, -1)
    length = moved.shape[-1]
    padded = -(-length // factor) * factor
    if padded != length:
        pad = np.zeros(moved.shape[:-1] + (padded - length,), dtype=np.uint32)
        moved = np.concatenate([moved, pad], axis=-1)
    moved = moved.reshape(moved.shape[:-1] + (padded // factor, factor))
    shifts = (np.arange(factor, dtype=np.uint32) * bits).astype(np.uint32)
    words = np.bitwise_or.reduce(moved << shifts, axis=-1).astype(np.uint32)
    return np.ascontiguousarray(np.moveaxis(words.view(np.int32), -1, dim))


def unpack_codes(packed: np.ndarray, bits: int, dim: int, length: int) -> np.ndarray:
    """physical.py:88-104."""

    dim = dim % packed.ndim
    if bits == 8:
        index = [slice(None)] * packed.ndim
        index[dim] = slice(0, length)
        return packed[tuple(index)].astype(np.uint8)
    factor = 32 // bits
    moved = np.moveaxis(packed.view(np.uint32), dim, -1)
    shifts = (np.arange(factor, dtype=np.uint32) * bits).astype(np.uint32)
    mask = np.uint32((1 << bits) - 1)
    codes = ((moved[..., None] >> shifts) & mask).reshape(moved.shape[:-1] + (-1,))
    codes = codes[..., :length]
    return np.ascontiguousarray(np.moveaxis(codes.astype(np.uint8), -1, dim))


# ----------------------------------------------------------- quantization --
def quantize_codes(data: np.ndarray, *, bits: int, group_dim: int, group_size: int):
    """physical.py:107-136 (loop form; the vectorised form 139-175 is
    equal for full groups).  Returns (codes uint8, scale f32, minimum f32)
    with stats stacked along group_dim and NOT yet rounded to a storage dtype.

      mn = amin, mx = amax over the group        (exact)
      scale = max((mx - mn) / (2^b - 1), eps)    (two fp32 roundings)
      code  = clamp(rint((x - mn) / scale), 0, 2^b - 1)

    NaN follows torch: amin / amax of a group holding a NaN are NaN, and
    clamp_min keeps the NaN scale.  Such a group's codes are NaN in fp32;
    torch's NaN -> uint8 cast (physical.py:166) is unspecified by C++ and
    gives 0 on x86, which is the value written here (explicitly, rather than
    through numpy's equally unspecified cast).
    """

    data = np.asarray(data, dtype=np.float32)
    gd = group_dim % data.ndim
    length = data.shape[gd]
    max_code = F32((1 << bits) - 1)
    codes, scales, minima = [], [], []
    for start in range(0, length, group_size):
        stop = min(length, start + group_size)
        chunk = np.take(data, np.arange(start, stop), axis=gd)
        mn = chunk.min(axis=gd, keepdims=True)
        mx = chunk.max(axis=gd, keepdims=True)
        scale = np.maximum((mx - mn) / max_code, EPS).astype(F32)
        q = np.clip(np.rint((chunk - mn) / scale), F32(0), max_code)
        codes.append(np.where(np.isnan(q), F32(0), q).astype(np.uint8))
        scales.append(np.squeeze(scale, axis=gd))
        minima.append(np.squeeze(mn, axis=gd))
    return (
        np.concatenate(codes, axis=gd),
        np.stack(scales, axis=gd).astype(F32),
        np.stack(minima, axis=gd).astype(F32),
    )


def quantize_grouped(data, *, bits, group_dim, group_size, pack_dim, stats_dtype="bf16"):
    """physical.py:107-175: (packed codes, scale, minimum, length), with the
    stats rounded to `stats_dtype` (the input dtype in UniCache's reference
    layout, fp16 in the kernel-native layout)."""

    codes, scale, minimum = quantize_codes(data, bits=bits, group_dim=group_dim, group_size=group_size)
    length = np.asarray(data).shape[group_dim % np.asarray(data).ndim]
    return (
        pack_codes(codes, bits, pack_dim),
        round_to(scale, stats_dtype),
        round_to(minimum, stats_dtype),
        length,
    )


def dequantize_grouped(packed, scale, minimum, *, bits, group_dim, group_size, pack_dim, length, out_dtype):
    """physical.py:178-201: code*scale then +min in fp32 (two roundings),
    then a cast to the output dtype."""

    codes = unpack_codes(packed, bits, pack_dim, length).astype(F32)
    gd = group_dim % codes.ndim
    chunks = []
    for gi, start in enumerate(range(0, length, group_size)):
        stop = min(length, start + group_size)
        chunk = np.take(codes, np.arange(start, stop), axis=gd)
        s = np.expand_dims(np.take(scale, gi, axis=gd), gd).astype(F32)
        m = np.expand_dims(np.take(minimum, gi, axis=gd), gd).astype(F32)
        chunks.append((chunk * s).astype(F32) + m)
    return round_to(np.concatenate(chunks, axis=gd).astype(F32), out_dtype)


# ---------------------------------------------------- kernel-native layout --
@dataclass
class PackedSegment:
    """The tensors of a PackedKIVICache (physical.py:204-226), as numpy."""

    key_code: np.ndarray | None
    key_scale: np.ndarray | None
    key_minimum: np.ndarray | None
    value_code: np.ndarray | None
    value_scale: np.ndarray | None
    value_minimum: np.ndarray | None
    residual_key: np.ndarray
    residual_value: np.ndarray
    k_bits: int
    v_bits: int
    group_size: int
    quantized_tokens: int
    native: bool


def quantize_native(key, value, *, k_bits, v_bits, group_size):
    """kivi_cuda.py:157-190 with physical.py's arithmetic: keys as
    [Hkv, D, T] grouped and packed along tokens, values as [Hkv, T, D]
    grouped and packed along channels; stats rounded to fp16."""

    key_native = np.ascontiguousarray(np.transpose(key, (1, 2, 0)))
    value_native = np.ascontiguousarray(np.transpose(value, (1, 0, 2)))
    kc, ks, km, _ = quantize_grouped(key_native, bits=k_bits, group_dim=2, group_size=group_size, pack_dim=2,
                                     stats_dtype="fp16")
    vc, vs, vm, _ = quantize_grouped(value_native, bits=v_bits, group_dim=2, group_size=group_size, pack_dim=2,
                                     stats_dtype="fp16")
    return kc, ks, km, vc, vs, vm


def split_tokens(tokens: int, group_size: int, residual_length: int) -> tuple[int, int]:
    """physical.py:258-263: (quantized, residual) with the residual in
    [R, R + G) unless the segment is shorter."""

    requested = min(tokens, max(0, int(residual_length)))
    quantized = ((tokens - requested) // group_size) * group_size
    return quantized, tokens - quantized


def from_dense(key, value, *, k_bits, v_bits, group_size, residual_length, native=True, in_dtype="bf16"):
    """PackedKIVICache.from_dense (physical.py:228-332).  native=True is the
    kernel layout (2/4-bit K and V); otherwise UniCache's reference layout
    with stats in the input dtype."""

    key = np.asarray(key, dtype=np.float32)
    value = np.asarray(value, dtype=np.float32)
    tokens = key.shape[0]
    quantized, _ = split_tokens(tokens, group_size, residual_length)
    native = bool(native and quantized and k_bits in (2, 4) and v_bits in (2, 4))
    parts = (None,) * 6
    if quantized:
        qk, qv = key[:quantized], value[:quantized]
        if native:
            parts = quantize_native(qk, qv, k_bits=k_bits, v_bits=v_bits, group_size=group_size)
        else:
            kc, ks, km, _ = quantize_grouped(qk, bits=k_bits, group_dim=0, group_size=group_size, pack_dim=0,
                                             stats_dtype=in_dtype)
            vc, vs, vm, _ = quantize_grouped(qv, bits=v_bits, group_dim=2, group_size=group_size, pack_dim=2,
                                             stats_dtype=in_dtype)
            parts = (kc, ks, km, vc, vs, vm)
    return PackedSegment(*parts, residual_key=key[quantized:].copy(), residual_value=value[quantized:].copy(),
                         k_bits=k_bits, v_bits=v_bits, group_size=group_size, quantized_tokens=quantized,
                         native=native)


def dequantize(seg: PackedSegment, out_dtype: str = "bf16"):
    """PackedKIVICache.dequantize (physical.py:379-423): [T, Hkv, D] K and V."""

    if not seg.quantized_tokens:
        return round_to(seg.residual_key, out_dtype), round_to(seg.residual_value, out_dtype)
    if seg.native:
        kc = np.transpose(seg.key_code, (2, 0, 1))
        ks = np.transpose(seg.key_scale, (2, 0, 1))
        km = np.transpose(seg.key_minimum, (2, 0, 1))
        vc = np.transpose(seg.value_code, (1, 0, 2))
        vs = np.transpose(seg.value_scale, (1, 0, 2))
        vm = np.transpose(seg.value_minimum, (1, 0, 2))
    else:
        kc, ks, km, vc, vs, vm = (seg.key_code, seg.key_scale, seg.key_minimum, seg.value_code,
                                  seg.value_scale, seg.value_minimum)
    head_dim = seg.residual_key.shape[-1]
    qk = dequantize_grouped(kc, ks, km, bits=seg.k_bits, group_dim=0, group_size=seg.group_size, pack_dim=0,
                            length=seg.quantized_tokens, out_dtype=out_dtype)
    qv = dequantize_grouped(vc, vs, vm, bits=seg.v_bits, group_dim=2, group_size=seg.group_size, pack_dim=2,
                            length=head_dim, out_dtype=out_dtype)
    key = np.concatenate([qk, round_to(seg.residual_key, out_dtype)], axis=0)
    value = np.concatenate([qv, round_to(seg.residual_value, out_dtype)], axis=0)
    return key, value


# -------------------------------------------------------------- fake quant --
def fake_quant(data, *, bits: int, dim: int, group_size: int, out_dtype: str = "bf16"):
    """asymmetric_fake_quant (operators/builtin.py:31-53): groups of
    min(group_size, length) along `dim`;
      scale = max(mx - mn, eps) / (2^b - 1)
      out   = rint((x - mn) / scale).clamp(0, 2^b - 1) * scale + mn
    then cast to the input dtype."""

    data = np.asarray(data, dtype=np.float32)
    if data.size == 0 or bits >= 16:
        return data
    dim = dim % data.ndim
    length = data.shape[dim]
    group = max(1, min(int(group_size), int(length)))
    max_int = F32((1 << bits) - 1)
    chunks = []
    for start in range(0, length, group):
        stop = min(length, start + group)
        chunk = np.take(data, np.arange(start, stop), axis=dim)
        mn = chunk.min(axis=dim, keepdims=True)
        mx = chunk.max(axis=dim, keepdims=True)
        scale = (np.maximum(mx - mn, EPS) / max_int).astype(F32)
        code = np.clip(np.rint((chunk - mn) / scale), F32(0), max_int).astype(F32)
        chunks.append((code * scale).astype(F32) + mn)
    return round_to(np.concatenate(chunks, axis=dim).astype(F32), out_dtype)


def streamed_split(initial_residual: int, appended: int, *, flush_at: int, group_size: int) -> int:
    """Tokens moved from the residual into the packed prefix when `appended`
    tokens arrive one at a time and the residual (starting at
    `initial_residual` tokens) is flushed -- its whole group-aligned head
    quantized -- whenever it reaches `flush_at` tokens.

    Streaming has no reference counterpart (UniCache packs once,
    unicache/storage/physical.py:228-332).  What pins it is the invariant the
    GPU tests check: after the flushes the packed state equals from_dense of
    the flushed prefix with residual_length=0, because K groups run along
    tokens and never straddle the prefix boundary, and V is grouped per token.
    """

    residual, packed = int(initial_residual), 0
    for _ in range(int(appended)):
        residual += 1
        if residual >= flush_at:
            moved = (residual // group_size) * group_size
            packed += moved
            residual -= moved
    return packed
