"""Physical KV-cache layouts of UniCache's engine, backed by MI355X kernels.

Drop-in for ``unicache/storage/physical.py``: the same classes, constructor
arguments, attributes, return layouts and exceptions.  Every tensor operation
on the cache contents (pack, dequantize, QK/AV, H2O selection and gather) runs
in libunicache_hip.so; torch only allocates memory and orders streams.

Backends, both on the HIP kernels: ``backend="cuda"`` stores 2/4-bit caches
in KIVI's kernel-native layout (fp16 stats) that the fused attention kernels
read; ``backend="reference"`` (UniCache's default) stores UniCache's own
layout -- codes packed along tokens (keys) / channels (values), stats in the
input dtype -- and attends by dequantizing, as UniCache's reference backend
does (physical.py:452-475).  UniCache runs its reference backend on CPU
tensors as well; here every backend needs GPU tensors and raises
RuntimeError otherwise (there is no CPU path).
"""

from __future__ import annotations

import ctypes

import math
import weakref
from dataclasses import dataclass
from typing import Callable

import torch

from .. import _native as nat


def tensor_bytes(tensor: torch.Tensor | None) -> int:
    return 0 if tensor is None else int(tensor.numel() * tensor.element_size())


def _check_backend(backend: str) -> None:
    if backend not in ("cuda", "reference"):
        raise ValueError(f"Unknown KIVI physical backend: {backend}")


def _dense_strides(t: torch.Tensor) -> tuple[int, int, int]:
    st, sh, sd = t.stride()
    return int(st), int(sh), int(sd)


def gqa_query_key_logits(query: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """QK for native GQA tensors without repeating KV heads (physical.py:20-39).

    query [Lq, Hq, D], key [T, Hkv, D] -> fp32 [Hq, Lq, T] (unscaled).
    """

    if query.dim() != 3 or key.dim() != 3:
        raise ValueError("GQA QK expects [tokens, heads, head_dim] tensors")
    if int(query.shape[-1]) != int(key.shape[-1]):
        raise ValueError("GQA QK query/key head dimensions must match")
    query_heads, kv_heads = int(query.shape[1]), int(key.shape[1])
    if query_heads % kv_heads != 0:
        raise ValueError("GQA query heads must be divisible by KV heads")
    return _dense_qk(query, key, scale=1.0)


def gqa_probability_value(probabilities: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """AV for native GQA tensors (physical.py:42-63): [Hq, Lq, T] x [T, Hkv, D]."""

    if probabilities.dim() != 3 or value.dim() != 3:
        raise ValueError(
            "GQA AV expects probabilities [heads, queries, keys] and values [keys, heads, dim]"
        )
    query_heads, kv_heads = int(probabilities.shape[0]), int(value.shape[1])
    if query_heads % kv_heads != 0:
        raise ValueError("GQA probability heads must be divisible by KV heads")
    if int(probabilities.shape[-1]) != int(value.shape[0]):
        raise ValueError("GQA AV probability key width must match value tokens")
    return _dense_av(probabilities, value)


def _dense_qk(query: torch.Tensor, key: torch.Tensor, *, scale: float) -> torch.Tensor:
    """scale * q.k over a dense key view [T, Hkv, D] (any token/head strides,
    unit channel stride) through uc_kivi_qk with no packed part."""

    device = nat.require_device(query, key, what="GQA QK")
    q = query.contiguous()
    lq, hq, d = map(int, q.shape)
    if key.stride(-1) != 1:
        key = key.contiguous()
    tokens, hkv = int(key.shape[0]), int(key.shape[1])
    logits = torch.empty((hq, lq, tokens), dtype=torch.float32, device=device)
    nat.call(
        "uc_kivi_qk", q.data_ptr(), nat.dtype_code(q.dtype), lq, hq,
        None, None, None, nat.UC_FP16, 0, 0, 2, 32,
        key.data_ptr(), nat.dtype_code(key.dtype), tokens, int(key.stride(0)), int(key.stride(1)),
        hkv, d, float(scale), logits.data_ptr(), nat.stream(device),
    )
    return logits


def _dense_av(probabilities: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """probs [Hq, Lq, T] x dense value view [T, Hkv, D] -> [Hq, Lq, D] of
    value.dtype, through uc_kivi_av with no packed part."""

    device = nat.require_device(probabilities, value, what="GQA AV")
    hq, lq, tokens = map(int, probabilities.shape)
    if value.stride(-1) != 1:
        value = value.contiguous()
    hkv, d = int(value.shape[1]), int(value.shape[2])
    out = torch.empty((hq, lq, d), dtype=value.dtype, device=device)
    ws = nat.workspace(device, nat.workspace_bytes(nat.UC_OP_KIVI_AV, 1, hq, lq, d, tokens))
    nat.call(
        "uc_kivi_av", probabilities.data_ptr(), nat.dtype_code(probabilities.dtype),
        *map(int, probabilities.stride()), lq, hq,
        None, None, None, nat.UC_FP16, 0, 0, 2, 32,
        value.data_ptr(), nat.dtype_code(value.dtype), tokens, int(value.stride(0)), int(value.stride(1)),
        hkv, d, out.data_ptr(), nat.dtype_code(value.dtype), ws.data_ptr(), nat.stream(device),
    )
    return out


# --------------------------------------------------------------- layouts --
def native_pack_layout(tokens: int, heads: int, head_dim: int, k_bits: int, v_bits: int, group_size: int):
    """Shapes and dtypes of the kernel-native packed tensors (kivi_cuda.py:177-190)."""

    return {
        "key_code": ((heads, head_dim, tokens * k_bits // 32), torch.int32),
        "key_stats": ((heads, head_dim, tokens // group_size), torch.float16),
        "value_code": ((heads, tokens, head_dim * v_bits // 32), torch.int32),
        "value_stats": ((heads, tokens, head_dim // group_size), torch.float16),
    }


# The kernel-native tensors keep the shapes above but live in token-major
# storage with room for `capacity` tokens per head:
#     key code   int32 [Hkv, C*kb/32, D]   key scale / minimum fp16 [Hkv, C/G, D]
#     value code int32 [Hkv, C, D*vb/32]   value scale / minimum fp16 [Hkv, C, D/G]
# The cache exposes views of the first T tokens, permuted back to the shapes
# of native_pack_layout, so one head's token range is one contiguous run of
# every tensor (the decode kernels stream it with 16-byte loads) and a flush
# appends rows in place.  The attention entry points of the library take this
# layout and the capacity C (uc_kivi_item.packed_capacity).
_CARVE_ALIGN = 256


def _carve(specs, device) -> list[torch.Tensor]:
    """Tensors of the given (shape, dtype) carved from one allocation, each
    starting on a 256-byte boundary: one allocator call per cache instead of
    one per tensor."""

    offsets, total = [], 0
    for shape, dtype in specs:
        offsets.append(total)
        total += -(-math.prod(shape) * dtype.itemsize // _CARVE_ALIGN) * _CARVE_ALIGN
    buf = torch.empty(max(total, _CARVE_ALIGN), dtype=torch.uint8, device=device)
    typed = {}  # one view per dtype, then one strided view per tensor
    out = []
    for (shape, dtype), off in zip(specs, offsets):
        base = typed.get(dtype)
        if base is None:
            base = typed[dtype] = buf.view(dtype)
        stride, acc = [], 1
        for n in reversed(shape):
            stride.append(acc)
            acc *= n
        out.append(base.as_strided(shape, tuple(reversed(stride)), off // dtype.itemsize))
    return out


def _native_specs(capacity: int, heads: int, head_dim: int, k_bits: int, v_bits: int, group_size: int):
    """(shape, dtype) of the token-major storage of the six packed tensors."""

    stats = ((heads, capacity // group_size, head_dim), torch.float16)
    vstats = ((heads, capacity, head_dim // group_size), torch.float16)
    return [((heads, capacity * k_bits // 32, head_dim), torch.int32), stats, stats,
            ((heads, capacity, head_dim * v_bits // 32), torch.int32), vstats, vstats]


def _native_storage(capacity: int, heads: int, head_dim: int, k_bits: int, v_bits: int, group_size: int,
                    device) -> tuple[torch.Tensor, ...]:
    return tuple(_carve(_native_specs(capacity, heads, head_dim, k_bits, v_bits, group_size), device))


def _native_views(storage, tokens: int, k_bits: int, group_size: int) -> tuple[torch.Tensor, ...]:
    """The first `tokens` tokens of token-major storage in the native shapes."""

    kc, ks, km, vc, vs, vm = storage
    heads, d = int(kc.shape[0]), int(kc.shape[2])
    nw, ng = tokens * k_bits // 32, tokens // group_size
    kcs, kss = int(kc.stride(0)), int(ks.stride(0))
    vw, vg = int(vc.shape[2]), int(vs.shape[2])
    vcs, vss = int(vc.stride(0)), int(vs.stride(0))
    return (kc.as_strided((heads, d, nw), (kcs, 1, d)), ks.as_strided((heads, d, ng), (kss, 1, d)),
            km.as_strided((heads, d, ng), (kss, 1, d)), vc.as_strided((heads, tokens, vw), (vcs, vw, 1)),
            vs.as_strided((heads, tokens, vg), (vss, vg, 1)), vm.as_strided((heads, tokens, vg), (vss, vg, 1)))


def _native_storage_of(views, capacity: int, k_bits: int, group_size: int) -> tuple[torch.Tensor, ...]:
    """Token-major storage tensors behind native views of capacity C."""

    kc, ks, km, vc, vs, vm = views
    heads, head_dim = int(kc.shape[0]), int(kc.shape[1])
    cw, cg = capacity * k_bits // 32, capacity // group_size
    vw, vg = int(vc.shape[2]), int(vs.shape[2])
    return (kc.as_strided((heads, cw, head_dim), (cw * head_dim, head_dim, 1)),
            ks.as_strided((heads, cg, head_dim), (cg * head_dim, head_dim, 1)),
            km.as_strided((heads, cg, head_dim), (cg * head_dim, head_dim, 1)),
            vc.as_strided((heads, capacity, vw), (capacity * vw, vw, 1)),
            vs.as_strided((heads, capacity, vg), (capacity * vg, vg, 1)),
            vm.as_strided((heads, capacity, vg), (capacity * vg, vg, 1)))


def _pack_native_into(storage, offset: int, key: torch.Tensor, value: torch.Tensor, *, k_bits: int, v_bits: int,
                      group_size: int, tokens: int | None = None, stream: int | None = None) -> None:
    """HIP quantize+pack of [n, Hkv, D] K/V into tokens offset..offset+n of
    token-major storage (offset a multiple of group_size).  `tokens` packs
    only the first rows of key / value; a caller that has checked the devices
    passes its `stream`."""

    if stream is None:
        stream = nat.stream(nat.require_device(key, value, storage[0], what="KIVI native packing"))
    kc, ks, km, vc, vs, vm = storage
    _pack_native_at((kc.data_ptr(), ks.data_ptr(), km.data_ptr(), vc.data_ptr(), vs.data_ptr(), vm.data_ptr()),
                    int(kc.shape[1]) * 32 // k_bits, offset, key, value, k_bits=k_bits, v_bits=v_bits,
                    group_size=group_size, tokens=tokens, stream=stream)


def _pack_native_at(ptrs, capacity: int, offset: int, key: torch.Tensor, value: torch.Tensor, *, k_bits: int,
                    v_bits: int, group_size: int, tokens: int | None, stream: int) -> None:
    """uc_kivi_pack into token-major storage of `capacity` tokens given by the
    addresses of its six tensors (token 0 of head 0)."""

    if key.dtype != value.dtype:
        raise ValueError("KIVI packing expects key and value of one dtype")
    heads, head_dim = int(key.shape[1]), int(key.shape[2])
    tokens = int(key.shape[0]) if tokens is None else int(tokens)
    kd, vw, vg = head_dim, head_dim * v_bits // 32, head_dim // group_size
    kw0, g0 = offset * k_bits // 32, offset // group_size
    kc, ks, km, vc, vs, vm = ptrs
    kcs, kss = capacity * k_bits // 32 * kd, capacity // group_size * kd  # head strides
    nat.call(
        "uc_kivi_pack",
        key.data_ptr(), *_dense_strides(key), value.data_ptr(), *_dense_strides(value),
        nat.dtype_code(key.dtype), tokens, heads, head_dim, k_bits, v_bits, group_size, nat.UC_FP16,
        # key code (h, d, w), key stats (h, d, g): token-major rows of D channels
        kc + 4 * kw0 * kd, kcs, 1, kd,
        ks + 2 * g0 * kd, km + 2 * g0 * kd, kss, 1, kd,
        vc + 4 * offset * vw, capacity * vw, vw, 1,
        vs + 2 * offset * vg, vm + 2 * offset * vg, capacity * vg, vg, 1,
        stream,
    )


def _native_block(capacity: int, heads: int, head_dim: int, k_bits: int, v_bits: int, group_size: int, device,
                  ids_dtype=None, ids_len: int = 0):
    """One allocation holding the token-major storage of `capacity` tokens and
    optionally an ids slot: the six native views of all `capacity` tokens (one
    view op each), the storage addresses, and the ids tensor (or None).  The
    few host operations matter: from_dense runs once per materialised segment."""

    specs = _native_specs(capacity, heads, head_dim, k_bits, v_bits, group_size)
    if ids_dtype is not None:
        specs.append(((ids_len,), ids_dtype))
    offsets, total = [], 0
    for shape, dtype in specs:
        offsets.append(total)
        total += -(-math.prod(shape) * dtype.itemsize // _CARVE_ALIGN) * _CARVE_ALIGN
    buf = torch.empty(max(total, _CARVE_ALIGN), dtype=torch.uint8, device=device)
    i32, f16 = buf.view(torch.int32), buf.view(torch.float16)
    d, nw, ng = head_dim, capacity * k_bits // 32, capacity // group_size
    vw, vg = head_dim * v_bits // 32, head_dim // group_size
    o = offsets
    views = (i32.as_strided((heads, d, nw), (nw * d, 1, d), o[0] // 4),
             f16.as_strided((heads, d, ng), (ng * d, 1, d), o[1] // 2),
             f16.as_strided((heads, d, ng), (ng * d, 1, d), o[2] // 2),
             i32.as_strided((heads, capacity, vw), (capacity * vw, vw, 1), o[3] // 4),
             f16.as_strided((heads, capacity, vg), (capacity * vg, vg, 1), o[4] // 2),
             f16.as_strided((heads, capacity, vg), (capacity * vg, vg, 1), o[5] // 2))
    base = buf.data_ptr()
    ids = None
    if ids_dtype is not None:
        ids = buf.view(ids_dtype).as_strided((ids_len,), (1,), o[6] // ids_dtype.itemsize)
    return views, tuple(base + off for off in o[:6]), ids


def _pack_native(key: torch.Tensor, value: torch.Tensor, *, k_bits: int, v_bits: int, group_size: int,
                 capacity: int | None = None):
    """HIP quantize+pack into the kernel-native layout (fp16 stats), in
    token-major storage with room for `capacity` tokens (default: exactly the
    input's)."""

    device = nat.require_device(key, value, what="KIVI native packing")
    tokens, heads, head_dim = map(int, key.shape)
    capacity = tokens if capacity is None else int(capacity)
    if capacity < tokens or capacity % group_size:
        raise ValueError("KIVI packed capacity must be a multiple of group_size covering the tokens")
    if capacity == tokens:  # the views of the whole storage: one view op per tensor
        views, ptrs, _ = _native_block(capacity, heads, head_dim, k_bits, v_bits, group_size, device)
        _pack_native_at(ptrs, capacity, 0, key, value, k_bits=k_bits, v_bits=v_bits, group_size=group_size,
                        tokens=None, stream=nat.stream(device))
        return views
    storage = _native_storage(capacity, heads, head_dim, k_bits, v_bits, group_size, device)
    _pack_native_into(storage, 0, key, value, k_bits=k_bits, v_bits=v_bits, group_size=group_size)
    return _native_views(storage, tokens, k_bits, group_size)


def _reference_layout_shapes(tokens, heads, head_dim, bits, group_size, *, is_key):
    """UniCache's non-native layout: codes along dim 0 (K) / dim 2 (V)."""

    per_word = 1 if bits == 8 else 32 // bits  # codes zero-padded to whole words (physical.py:72-85)
    if is_key:
        code = (-(-tokens // per_word), heads, head_dim)
        stats = (tokens // group_size, heads, head_dim)
    else:
        code = (tokens, heads, -(-head_dim // per_word))
        stats = (tokens, heads, -(-head_dim // group_size))  # a partial last group (physical.py:151-158)
    return code, stats, (torch.uint8 if bits == 8 else torch.int32)


def _pack_reference_layout(key, value, *, k_bits, v_bits, group_size):
    """HIP quantize+pack into UniCache's non-native layout (stats in the input
    dtype), used when a payload is 8-bit (physical.py:291-304)."""

    device = nat.require_device(key, value, what="KIVI packing")
    tokens, heads, head_dim = map(int, key.shape)
    kshape, kstat_shape, kdt = _reference_layout_shapes(tokens, heads, head_dim, k_bits, group_size, is_key=True)
    vshape, vstat_shape, vdt = _reference_layout_shapes(tokens, heads, head_dim, v_bits, group_size, is_key=False)
    kc = torch.empty(kshape, dtype=kdt, device=device)
    ks = torch.empty(kstat_shape, dtype=key.dtype, device=device)
    km = torch.empty_like(ks)
    vc = torch.empty(vshape, dtype=vdt, device=device)
    vs = torch.empty(vstat_shape, dtype=key.dtype, device=device)
    vm = torch.empty_like(vs)
    # key code element (h, d, w) -> [w, h, d]; key stats (h, d, g) -> [g, h, d]
    kc_s = (kc.stride(1), kc.stride(2), kc.stride(0))
    ks_s = (ks.stride(1), ks.stride(2), ks.stride(0))
    # value code (h, t, w) -> [t, h, w]; value stats (h, t, g) -> [t, h, g]
    vc_s = (vc.stride(1), vc.stride(0), vc.stride(2))
    vs_s = (vs.stride(1), vs.stride(0), vs.stride(2))
    nat.call(
        "uc_kivi_pack",
        key.data_ptr(), *_dense_strides(key), value.data_ptr(), *_dense_strides(value),
        nat.dtype_code(key.dtype), tokens, heads, head_dim, k_bits, v_bits, group_size,
        nat.dtype_code(key.dtype),
        kc.data_ptr(), *map(int, kc_s), ks.data_ptr(), km.data_ptr(), *map(int, ks_s),
        vc.data_ptr(), *map(int, vc_s), vs.data_ptr(), vm.data_ptr(), *map(int, vs_s),
        nat.stream(device),
    )
    return kc, ks, km, vc, vs, vm


# ------------------------------------------------------------------ KIVI --
@dataclass
class PackedKIVICache:
    """A KIVI packed KV segment with a full-precision residual suffix
    (physical.py:204-475)."""

    key_code: torch.Tensor | None
    key_scale: torch.Tensor | None
    key_minimum: torch.Tensor | None
    value_code: torch.Tensor | None
    value_scale: torch.Tensor | None
    value_minimum: torch.Tensor | None
    residual_key: torch.Tensor
    residual_value: torch.Tensor
    logical_token_ids: torch.Tensor
    token_type_id: int
    k_bits: int
    v_bits: int
    group_size: int
    quantized_tokens: int
    head_dim: int
    num_kv_heads: int
    backend: str = "reference"
    kernel_native_layout: bool = False
    budget_shortfall_events: int = 0

    @classmethod
    def from_dense(
        cls,
        key: torch.Tensor,
        value: torch.Tensor,
        *,
        logical_token_ids: torch.Tensor,
        token_type_id: int,
        k_bits: int,
        v_bits: int,
        group_size: int,
        residual_length: int,
        backend: str = "reference",
    ) -> "PackedKIVICache":
        """Split [tokens, Hkv, D] K/V into a group-aligned packed prefix and a
        residual suffix (physical.py:228-332)."""

        if key.shape != value.shape or key.dim() != 3:
            raise ValueError("KIVI physical cache expects matching [tokens, kv_heads, head_dim] tensors")
        if k_bits not in {2, 4, 8} or v_bits not in {2, 4, 8}:
            raise ValueError("KIVI physical cache supports 2, 4, or 8 bit payloads")
        tokens, heads, head_dim = map(int, key.shape)
        if group_size <= 0:
            raise ValueError("KIVI physical cache group_size must be positive")
        _check_backend(backend)
        if backend == "cuda" and (k_bits in {2, 4} or v_bits in {2, 4}):
            # the kernel-native layout (physical.py:247-256 pins 64 or 128 for it)
            if group_size not in {16, 32, 64, 128}:
                raise ValueError("The MI355X KIVI kernels support group_size 16, 32, 64 or 128")
            if head_dim % group_size != 0:
                raise ValueError("The MI355X KIVI value kernel requires head_dim divisible by group_size")
        requested_residual = min(tokens, max(0, int(residual_length)))
        # keep any incomplete prefix group in the residual (physical.py:258-263)
        quantized = ((tokens - requested_residual) // group_size) * group_size
        q_key, q_value = key[:quantized], value[:quantized]
        kernel_native_layout = bool(backend == "cuda" and quantized and k_bits in {2, 4} and v_bits in {2, 4})
        if kernel_native_layout:
            return cls._from_dense_native(key, value, quantized, logical_token_ids, token_type_id, k_bits, v_bits,
                                          group_size)
        if quantized:
            packed = _pack_reference_layout(q_key, q_value, k_bits=k_bits, v_bits=v_bits, group_size=group_size)
            key_code, key_scale, key_minimum, value_code, value_scale, value_minimum = packed
        else:
            nat.require_device(key, value, what="KIVI physical cache")
            key_code = key_scale = key_minimum = None
            value_code = value_scale = value_minimum = None
        return cls(
            key_code=key_code,
            key_scale=key_scale,
            key_minimum=key_minimum,
            value_code=value_code,
            value_scale=value_scale,
            value_minimum=value_minimum,
            # a clone, so a suffix view does not pin the whole dense segment
            residual_key=key[quantized:].clone(),
            residual_value=value[quantized:].clone(),
            logical_token_ids=logical_token_ids.detach().clone(),
            token_type_id=int(token_type_id),
            k_bits=int(k_bits),
            v_bits=int(v_bits),
            group_size=int(group_size),
            quantized_tokens=quantized,
            head_dim=head_dim,
            num_kv_heads=heads,
            backend=str(backend),
            kernel_native_layout=kernel_native_layout,
        )

    @classmethod
    def _from_dense_native(cls, key, value, quantized, logical_token_ids, token_type_id, k_bits, v_bits,
                           group_size) -> "PackedKIVICache":
        """from_dense into the kernel-native layout: the packed storage and the
        logical ids share one allocation and one HIP pass quantizes and packs;
        the residual rows are compact clones, as UniCache's are."""

        if key.device.type != "cuda":
            raise RuntimeError("KIVI native packing requires CUDA tensors")  # kivi_cuda.py:157-190
        device = nat.require_device(key, value, what="KIVI native packing")
        if key.dtype != value.dtype:
            raise ValueError("KIVI packing expects key and value of one dtype")
        heads, head_dim = int(key.shape[1]), int(key.shape[2])
        ids = logical_token_ids.detach()
        ids_here = ids.device == device and ids.dim() == 1
        views, ptrs, ids_slot = _native_block(quantized, heads, head_dim, k_bits, v_bits, group_size, device,
                                              ids.dtype if ids_here else None, int(ids.shape[0]) if ids_here else 0)
        stream = nat.stream(device)
        _pack_native_at(ptrs, quantized, 0, key, value, k_bits=k_bits, v_bits=v_bits, group_size=group_size,
                        tokens=quantized, stream=stream)
        # the residual rows as compact copies, so a suffix view does not pin
        # the whole dense segment (physical.py:316-319), and the ids: one
        # launch for the three copies
        tail_k, tail_v = key[quantized:], value[quantized:]
        res_k = torch.empty(tail_k.shape, dtype=key.dtype, device=device)
        res_v = torch.empty(tail_v.shape, dtype=value.dtype, device=device)
        if tail_k.is_contiguous() and tail_v.is_contiguous() and (not ids_here or ids.is_contiguous()):
            nbytes = tail_k.numel() * tail_k.element_size()
            spans = [tail_k.data_ptr(), res_k.data_ptr(), nbytes, tail_v.data_ptr(), res_v.data_ptr(), nbytes]
            if ids_here:
                spans += [ids.data_ptr(), ids_slot.data_ptr(), ids.numel() * ids.element_size()]
            table = (ctypes.c_int64 * len(spans))(*spans)
            nat.call("uc_copy_spans", ctypes.addressof(table), len(spans) // 3, stream)
            ids_copy = ids_slot if ids_here else ids.clone()
        else:
            res_k.copy_(tail_k)
            res_v.copy_(tail_v)
            ids_copy = ids_slot.copy_(ids) if ids_here else ids.clone()
        return cls(*views, res_k, res_v, ids_copy, int(token_type_id), int(k_bits), int(v_bits), int(group_size),
                   quantized, head_dim, heads, "cuda", True)

    def _native_store(self, device) -> tuple[torch.Tensor, ...] | None:
        """Token-major storage behind the native packed tensors (None without a
        packed prefix): the one this cache created when its tensors are still
        views of it, else rebuilt after checking the tensors' layout."""

        if not self.quantized_tokens:
            return None
        store = self._owned_store()
        if store is not None:
            return store
        views = (self.key_code, self.key_scale, self.key_minimum, self.value_code, self.value_scale,
                 self.value_minimum)
        cap = self.native_packed_pointers(device)[-1]
        return _native_storage_of(views, cap, self.k_bits, self.group_size)

    def _owned_store(self) -> tuple[torch.Tensor, ...] | None:
        """The token-major storage this cache allocated itself (a flush that
        outgrew the previous one), while the packed tensors are still views of
        it; None otherwise.  Only owned storage is written in place: storage
        reached through tensors the cache was given, or shared with a copy of
        this object, may back another cache's tokens."""

        owner, store = self.__dict__.get("_store", (None, None))
        if store is None or owner != id(self) or not self.quantized_tokens:
            return None
        views = (self.key_code, self.key_scale, self.key_minimum, self.value_code, self.value_scale,
                 self.value_minimum)
        if (all(v.data_ptr() == t.data_ptr() for v, t in zip(views, store))
                and int(self.key_code.shape[2]) == self.quantized_tokens * self.k_bits // 32
                and int(self.value_code.shape[1]) == self.quantized_tokens):
            return store
        return None

    def _residual_slot(self) -> tuple[torch.Tensor | None, int]:
        """(buffer, first row) of the residual inside this cache's [2, size,
        Hkv, D] residual buffer, or (None, 0) when the residual lives elsewhere."""

        buf = getattr(self, "_residual_capacity", None)
        if buf is None or self.residual_key.dtype != buf.dtype:
            return None, 0
        row = self.num_kv_heads * self.head_dim * buf.element_size()
        size, tr = int(buf.shape[1]), self.residual_tokens
        off, rem = divmod(self.residual_key.data_ptr() - buf.data_ptr(), row)
        if (rem or not 0 <= off <= size - tr or not self.residual_key.is_contiguous()
                or self.residual_value.data_ptr() != self.residual_key.data_ptr() + size * row):
            return None, 0
        return buf, off

    def _set_residual(self, buf: torch.Tensor, off: int, tokens: int) -> None:
        hd = self.num_kv_heads * self.head_dim
        shape, stride = (tokens, self.num_kv_heads, self.head_dim), (hd, self.head_dim, 1)
        base = buf.storage_offset() + off * hd
        self.residual_key = buf.as_strided(shape, stride, base)
        self.residual_value = buf.as_strided(shape, stride, base + int(buf.shape[1]) * hd)

    @property
    def token_count(self) -> int:
        return int(self.logical_token_ids.numel())

    @property
    def mutation_count(self) -> int:
        """How many times this cache has replaced or grown its tensors (append,
        flush_residual, repack_monotonic).  Item tables holding raw pointers
        into the cache compare it to notice that they are stale."""

        return getattr(self, "_mutations", 0)

    def _mutated(self) -> None:
        self._mutations = self.mutation_count + 1

    @property
    def residual_tokens(self) -> int:
        return int(self.residual_key.shape[0])

    @property
    def packed_capacity(self) -> int:
        """Tokens per head that the native packed storage holds (>=
        quantized_tokens; flushes append in place up to it); 0 without a
        native packed prefix."""

        if not self.kernel_native_layout or self.key_code is None:
            return 0
        return int(self.key_code.stride(0)) // self.head_dim * 32 // self.k_bits

    def native_packed_pointers(self, device: torch.device | None = None) -> tuple[int, ...]:
        """(key code, key scale, key minimum, value code, value scale, value
        minimum) device addresses and the packed capacity, after checking that
        the six tensors are the token-major native layout the attention
        kernels read by address (dtypes, shapes, strides, device, 16-byte
        alignment).  Raises ValueError / RuntimeError otherwise."""

        if not self.kernel_native_layout or self.key_code is None:
            raise RuntimeError("Packed KIVI attention requires kernel-native layout")
        views = (self.key_code, self.key_scale, self.key_minimum, self.value_code, self.value_scale,
                 self.value_minimum)
        device = device or self.key_code.device
        # the checks below hold as long as the six tensor objects, their storage
        # addresses, the token count and the capacity are the ones last checked
        # (decode and attention_parts calls check them on every call)
        memo = self.__dict__.get("_layout_memo")
        state = (self.quantized_tokens, self.packed_capacity, device)
        if memo is not None and memo[1] == state and all(r() is t for r, t in zip(memo[0], views)):
            ptrs = tuple(t.data_ptr() for t in views)
            if ptrs == memo[2][:6]:
                return memo[2]
        h, d, g, tq = self.num_kv_heads, self.head_dim, self.group_size, self.quantized_tokens
        cap = self.packed_capacity
        vw, vg = d * self.v_bits // 32, d // g
        cw, cg = cap * self.k_bits // 32, cap // g
        expected = (
            ("key_code", torch.int32, (h, d, tq * self.k_bits // 32), (cw * d, 1, d)),
            ("key_scale", torch.float16, (h, d, tq // g), (cg * d, 1, d)),
            ("key_minimum", torch.float16, (h, d, tq // g), (cg * d, 1, d)),
            ("value_code", torch.int32, (h, tq, vw), (cap * vw, vw, 1)),
            ("value_scale", torch.float16, (h, tq, vg), (cap * vg, vg, 1)),
            ("value_minimum", torch.float16, (h, tq, vg), (cap * vg, vg, 1)),
        )
        ptrs = []
        for name, dtype, shape, stride in expected:
            t = getattr(self, name)
            if t.device != device:
                raise RuntimeError(f"Packed KIVI {name} must be on {device} (got {t.device})")
            if t.dtype != dtype or tuple(t.shape) != shape or tuple(t.stride()) != stride:
                raise ValueError(
                    f"Packed KIVI {name} is not in the token-major native layout: expected {dtype} {shape} "
                    f"strides {stride}, got {t.dtype} {tuple(t.shape)} strides {tuple(t.stride())}")
            if t.data_ptr() % 16:
                raise ValueError(f"Packed KIVI {name} must be 16-byte aligned")
            ptrs.append(t.data_ptr())
        if cap < tq or cap % g:
            raise ValueError("Packed KIVI capacity must be a multiple of group_size covering the packed tokens")
        result = (*ptrs, cap)
        self.__dict__["_layout_memo"] = (tuple(weakref.ref(t) for t in views), state, result)
        return result

    def native_item(self, query_ptr: int, out_ptr: int, lse_ptr: int | None, *, residual_key_ptr: int | None = None,
                    residual_value_ptr: int | None = None, residual_tokens: int = 0) -> "nat.KiviItem":
        """Launch-table entry (uc_kivi_item) for the packed prefix plus the
        given residual rows."""

        kc, ks, km, vc, vs, vm, cap = self.native_packed_pointers()
        return nat.KiviItem(kc, ks, km, vc, vs, vm, residual_key_ptr, residual_value_ptr, query_ptr, out_ptr,
                            lse_ptr, self.quantized_tokens, int(residual_tokens), cap)

    @property
    def resident_bytes(self) -> int:
        tensors = (
            self.key_code, self.key_scale, self.key_minimum,
            self.value_code, self.value_scale, self.value_minimum,
            self.residual_key, self.residual_value, self.logical_token_ids,
        )
        return sum(tensor_bytes(item) for item in tensors)

    @property
    def byte_breakdown(self) -> dict[str, int]:
        return {
            "payload_bytes": tensor_bytes(self.key_code) + tensor_bytes(self.value_code),
            "scale_bytes": tensor_bytes(self.key_scale) + tensor_bytes(self.value_scale),
            "minimum_bytes": tensor_bytes(self.key_minimum) + tensor_bytes(self.value_minimum),
            "residual_bytes": tensor_bytes(self.residual_key) + tensor_bytes(self.residual_value),
            "indices_bytes": tensor_bytes(self.logical_token_ids),
            "score_bytes": 0,
        }

    @property
    def full_precision_bytes(self) -> int:
        element_size = int(self.residual_key.element_size())
        return self.token_count * self.num_kv_heads * self.head_dim * 2 * element_size

    def _code_strides(self):
        """(key code, key stats, value code, value stats) strides in the
        (h, d, w) / (h, d, g) / (h, t, w) / (h, t, g) order of the C ABI."""

        kc, ks, vc, vs = self.key_code, self.key_scale, self.value_code, self.value_scale
        if self.kernel_native_layout:
            return tuple(kc.stride()), tuple(ks.stride()), tuple(vc.stride()), tuple(vs.stride())
        return (
            (kc.stride(1), kc.stride(2), kc.stride(0)),
            (ks.stride(1), ks.stride(2), ks.stride(0)),
            (vc.stride(1), vc.stride(0), vc.stride(2)),
            (vs.stride(1), vs.stride(0), vs.stride(2)),
        )

    def dequantize_into(self, out_key: torch.Tensor | None, out_value: torch.Tensor | None,
                        *, start: int, stop: int, output_offset: int) -> None:
        """Restore packed tokens [start, stop) into rows output_offset.. of the
        given [n, Hkv, D] buffers (either may be None)."""

        if stop <= start:
            return
        ref = out_key if out_key is not None else out_value
        device = nat.require_device(self.key_code, ref, what="KIVI dequantization")
        kcs, kss, vcs, vss = self._code_strides()
        if out_key is not None and out_value is not None:
            if out_key.stride() != out_value.stride() or out_key.dtype != out_value.dtype:
                raise ValueError("KIVI dequantization output workspace has an invalid layout")
        nat.call(
            "uc_kivi_dequant",
            nat.ptr(self.key_code) if out_key is not None else None, *map(int, kcs),
            self.key_scale.data_ptr(), self.key_minimum.data_ptr(), *map(int, kss),
            nat.ptr(self.value_code) if out_value is not None else None, *map(int, vcs),
            self.value_scale.data_ptr(), self.value_minimum.data_ptr(), *map(int, vss),
            nat.dtype_code(self.key_scale.dtype), self.num_kv_heads, self.head_dim,
            self.k_bits, self.v_bits, self.group_size, int(start), int(stop),
            nat.ptr(out_key), nat.ptr(out_value), nat.dtype_code(ref.dtype),
            *map(int, ref.stride()), int(output_offset), nat.stream(device),
        )

    def dequantize(self, dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Restore [tokens, Hkv, D] K and V (physical.py:379-423)."""

        dtype = dtype or self.residual_key.dtype
        if not self.quantized_tokens:
            return self.residual_key.to(dtype), self.residual_value.to(dtype)
        total = self.quantized_tokens + self.residual_tokens
        shape = (total, self.num_kv_heads, self.head_dim)
        key = torch.empty(shape, dtype=dtype, device=self.key_code.device)
        value = torch.empty_like(key)
        self.dequantize_into(key, value, start=0, stop=self.quantized_tokens, output_offset=0)
        key[self.quantized_tokens:].copy_(self.residual_key)
        value[self.quantized_tokens:].copy_(self.residual_value)
        return key, value

    def repack_monotonic(self, *, bits: int, group_size: int | None = None) -> bool:
        """Lower precision, never raising it back (physical.py:425-450)."""

        target_bits = int(bits)
        target_group = int(group_size or self.group_size)
        if target_bits > self.k_bits or target_bits > self.v_bits or target_group < self.group_size:
            self.budget_shortfall_events += 1
            return False
        if target_bits == self.k_bits and target_bits == self.v_bits and target_group == self.group_size:
            return True
        key, value = self.dequantize(dtype=self.residual_key.dtype)
        replacement = PackedKIVICache.from_dense(
            key,
            value,
            logical_token_ids=self.logical_token_ids,
            token_type_id=self.token_type_id,
            k_bits=target_bits,
            v_bits=target_bits,
            group_size=target_group,
            residual_length=int(self.residual_key.shape[0]),
            backend=self.backend,
        )
        shortfalls, mutations = self.budget_shortfall_events, self.mutation_count
        # drop the streaming buffers of the old packing (grown packed storage,
        # residual window) so the repack frees them
        for name in ("_store", "_residual_capacity", "_ids_capacity", "_stream"):
            self.__dict__.pop(name, None)
        self.__dict__.update(replacement.__dict__)
        self.budget_shortfall_events = shortfalls
        self._mutations = mutations + 1
        return True

    # ------------------------------------------------------------ streaming --
    # Decode appends one token per step to the full-precision residual; once the
    # residual reaches `flush_at` tokens its group-aligned head is quantized and
    # appended to the packed prefix (keys as new token words per channel, values
    # as new rows).  Because groups never straddle the prefix boundary, the
    # packed state after a flush equals from_dense(all flushed tokens,
    # residual_length=0).  UniCache builds caches once (physical.py:228-332);
    # this is the streaming extension long-context decode needs.

    def append(self, key: torch.Tensor, value: torch.Tensor, *, logical_token_ids: torch.Tensor,
               flush_at: int | None = None) -> int:
        """Append [n, Hkv, D] tokens to the residual; flush when it reaches
        `flush_at` tokens.  Returns the number of tokens packed by the flush."""

        if key.shape != value.shape or key.dim() != 3 or tuple(key.shape[1:]) != (self.num_kv_heads, self.head_dim):
            raise ValueError("KIVI append expects [tokens, kv_heads, head_dim] K/V matching the cache")
        if key.dtype != self.residual_key.dtype or value.dtype != self.residual_value.dtype:
            raise ValueError("KIVI append expects K/V in the residual dtype")
        nat.require_device(key, value, self.residual_key, what="KIVI append")
        n = int(key.shape[0])
        if int(logical_token_ids.numel()) != n:
            raise ValueError("KIVI append needs one logical id per appended token")
        tr = self.residual_tokens
        # residual K and V rows live at one offset of a [2, size, Hkv, D]
        # buffer: appends write after them, a flush advances the offset, and
        # the rows slide back to the front only when the end is reached
        buf, off = self._residual_slot()
        if buf is None or buf.dtype != key.dtype or int(buf.shape[1]) < tr + n:
            size = max(4 * (tr + n), 256)
            new = torch.empty((2, size, self.num_kv_heads, self.head_dim), dtype=key.dtype, device=key.device)
            if tr:
                new[0, :tr].copy_(self.residual_key)
                new[1, :tr].copy_(self.residual_value)
            buf, off = new, 0
            self._residual_capacity = buf
        elif off + tr + n > int(buf.shape[1]):
            if tr:
                tail = buf[:, off:off + tr]
                buf[:, :tr].copy_(tail if off >= tr else tail.clone())
            off = 0
        buf[0, off + tr:off + tr + n].copy_(key)
        buf[1, off + tr:off + tr + n].copy_(value)
        self._set_residual(buf, off, tr + n)
        self._append_ids(logical_token_ids, n)
        self._mutated()
        if flush_at is not None and self.residual_tokens >= int(flush_at):
            return self.flush_residual()
        return 0

    def reserve(self, tokens: int) -> None:
        """Room for `tokens` more appended tokens, and for flushing all of
        them into the packed prefix, with no further allocation: packed
        storage owned by this cache with capacity for them, a residual-window
        buffer with that many free rows behind the window, and logical-id
        capacity on the cache's device.  Tensors move (and mutation_count
        rises) only where room is missing.  Streaming caches only: native equal
        2- or 4-bit K/V (backend='cuda')."""

        tokens = int(tokens)
        if tokens <= 0:
            return
        if self.k_bits != self.v_bits or self.k_bits not in (2, 4) or self.backend != "cuda" or (
                self.quantized_tokens and not self.kernel_native_layout):
            raise ValueError("KIVI reserve needs a native equal 2- or 4-bit cache (backend='cuda')")
        device = nat.require_device(self.residual_key, self.residual_value, what="KIVI reserve")
        heads, d, g, bits = self.num_kv_heads, self.head_dim, self.group_size, self.k_bits
        tq, tr = self.quantized_tokens, self.residual_tokens
        moved = False
        need = -(-(tq + tr + tokens) // g) * g
        owned = self._owned_store()
        if owned is None or int(owned[3].shape[1]) < need:
            old = self._native_store(device)
            grown = _native_storage(need, heads, d, bits, bits, g, device)
            if tq:
                for dst, src in zip(_native_views(grown, tq, bits, g), _native_views(old, tq, bits, g)):
                    dst.copy_(src)
                (self.key_code, self.key_scale, self.key_minimum,
                 self.value_code, self.value_scale, self.value_minimum) = _native_views(grown, tq, bits, g)
            self._store = (id(self), grown)
            moved = True
        buf, off = self._residual_slot()
        if buf is None or int(buf.shape[1]) - off < tr + tokens:
            new = torch.empty((2, max(tr + tokens, 256), heads, d), dtype=self.residual_key.dtype, device=device)
            if tr:
                new[0, :tr].copy_(self.residual_key)
                new[1, :tr].copy_(self.residual_value)
            self._residual_capacity = new
            self._set_residual(new, 0, tr)
            moved = True
        cur = self.logical_token_ids
        ids = self.__dict__.get("_ids_capacity")
        total = int(cur.numel())
        if (ids is None or ids.device != device or int(ids.numel()) < total + tokens or ids.dtype != cur.dtype
                or cur.device != device or cur.data_ptr() != ids.data_ptr() or not cur.is_contiguous()):
            ids = torch.empty(total + tokens, dtype=cur.dtype, device=device)
            ids[:total].copy_(cur)
            self._ids_capacity = ids
            self.logical_token_ids = ids[:total]
            moved = True
        if moved:
            self._mutated()

    def _append_ids(self, ids: torch.Tensor, n: int) -> None:
        """Append n logical ids: they go after the current ones in a capacity
        buffer that grows geometrically, so an append copies only its own ids."""

        cur = self.logical_token_ids
        total = int(cur.numel())
        buf = self.__dict__.get("_ids_capacity")
        if (buf is None or buf.dtype != cur.dtype or buf.device != cur.device or int(buf.numel()) < total + n
                or cur.data_ptr() != buf.data_ptr() or not cur.is_contiguous()):
            new = torch.empty(max(2 * (total + n), 1024), dtype=cur.dtype, device=cur.device)
            new[:total].copy_(cur)
            buf = self._ids_capacity = new
        buf[total:total + n].copy_(ids.reshape(-1))
        self.logical_token_ids = buf[:total + n]

    def flush_residual(self, keep: int = 0) -> int:
        """Quantize the residual except its last `keep` tokens (rounded so the
        packed length stays a multiple of group_size) and append it to the
        packed prefix: in place while the token-major storage has room
        (packed_capacity), else into storage 1.5x larger.  Returns the number
        of tokens packed."""

        tr = self.residual_tokens
        count = ((tr - max(0, int(keep))) // self.group_size) * self.group_size
        if count <= 0:
            return 0
        if self.k_bits != self.v_bits or self.k_bits not in (2, 4):
            raise ValueError("Streaming KIVI flush supports equal 2-bit or 4-bit K/V")
        if self.backend != "cuda" or (self.quantized_tokens and not self.kernel_native_layout):
            raise RuntimeError("Streaming KIVI flush requires the kernel-native layout (backend='cuda')")
        device = nat.require_device(self.residual_key, self.residual_value, what="KIVI flush")
        stream = nat.stream(device)
        tq, bits, g = self.quantized_tokens, self.k_bits, self.group_size
        store = self._native_store(device)
        cap = int(store[3].shape[1]) if store is not None else 0
        # in place only into storage this cache allocated (see _owned_store)
        if tq + count > cap or self._owned_store() is None:
            # grow geometrically so a run of flushes copies the prefix O(log n) times
            cap = -(-max(tq + count, cap + cap // 2) // g) * g
            grown = _native_storage(cap, self.num_kv_heads, self.head_dim, bits, bits, g, device)
            if tq:
                for dst, src in zip(_native_views(grown, tq, bits, g), _native_views(store, tq, bits, g)):
                    dst.copy_(src)
            store = grown
        _pack_native_into(store, tq, self.residual_key, self.residual_value, k_bits=bits, v_bits=bits, group_size=g,
                          tokens=count, stream=stream)
        (self.key_code, self.key_scale, self.key_minimum,
         self.value_code, self.value_scale, self.value_minimum) = _native_views(store, tq + count, bits, g)
        self._store = (id(self), store)
        self.quantized_tokens = tq + count
        self.kernel_native_layout = True
        buf, off = self._residual_slot()
        if buf is not None:  # the kept tail stays where it is
            self._set_residual(buf, off + count, tr - count)
        else:
            self.residual_key = self.residual_key[count:].clone()
            self.residual_value = self.residual_value[count:].clone()
        self._mutated()
        return count

    def attention_parts(
        self, query: torch.Tensor
    ) -> tuple[torch.Tensor, Callable[[torch.Tensor], torch.Tensor]]:
        """Scaled logits over [packed | residual] and an AV closure
        (physical.py:452-475)."""

        _check_backend(self.backend)
        if self.backend == "cuda":
            from .kivi_cuda import packed_kivi_attention_parts

            return packed_kivi_attention_parts(self, query)
        key, value = self.dequantize(dtype=query.dtype)
        logits = _dense_qk(query, key, scale=1.0 / math.sqrt(query.shape[-1]))

        def apply_value(probabilities: torch.Tensor) -> torch.Tensor:
            return gqa_probability_value(probabilities, value)

        return logits, apply_value


# A packed cache that a MixedDecodeBatch streams into (MixedDecodeBatch.append)
# has its residual window and logical ids extended on the device; the batch
# records the new lengths in the cache's _StreamState, and the cache's
# residual_key / residual_value / logical_token_ids views are rebuilt from it
# on their next read.  Every reader -- the cache's own methods and outside
# code alike -- therefore sees the appended tokens.
class _StreamState:
    __slots__ = ("buf", "ids", "off", "tr", "tq", "dirty")

    def __init__(self, buf: torch.Tensor, ids: torch.Tensor, off: int, tr: int, tq: int) -> None:
        self.buf, self.ids, self.off, self.tr, self.tq, self.dirty = buf, ids, off, tr, tq, False

    def pull(self, cache: "PackedKIVICache") -> None:
        d = cache.__dict__
        heads, hd = cache.num_kv_heads, cache.head_dim
        shape, stride = (self.tr, heads, hd), (heads * hd, hd, 1)
        base = self.buf.storage_offset() + self.off * heads * hd
        d["_residual_key"] = self.buf.as_strided(shape, stride, base)
        d["_residual_value"] = self.buf.as_strided(shape, stride, base + int(self.buf.shape[1]) * heads * hd)
        d["_logical_token_ids"] = self.ids[:self.tq + self.tr]
        self.dirty = False


def _streamed_field(name: str) -> property:
    slot = "_" + name

    def get(self):
        d = self.__dict__
        state = d.get("_stream")
        if state is not None and state.dirty:
            state.pull(self)
        return d[slot]

    def set(self, value):
        self.__dict__[slot] = value

    return property(get, set, doc=f"PackedKIVICache.{name} (current after device-side appends)")


for _name in ("residual_key", "residual_value", "logical_token_ids"):
    setattr(PackedKIVICache, _name, _streamed_field(_name))


# ------------------------------------------------------------------- H2O --
def h2o_select_indices(scores: torch.Tensor, *, heavy_k: int, recent: int) -> torch.Tensor:
    """[Hkv, heavy_k + recent] int64: per KV head the heavy_k top scores of the
    history (lowest index wins ties), ascending, then the recent window."""

    device = nat.require_device(scores, what="H2O selection")
    if scores.dtype != torch.float32:
        scores = scores.float()
    heads, tokens = map(int, scores.shape)
    out = torch.empty((heads, int(heavy_k) + int(recent)), dtype=torch.long, device=device)
    nat.call(
        "uc_h2o_select", scores.data_ptr(), *map(int, scores.stride()), heads, tokens,
        int(heavy_k), int(recent), out.data_ptr(), nat.stream(device),
    )
    return out


def _gather(key, value, key_strides, indexes, ids, ids_strides, scores, *, heads, head_dim):
    device = nat.require_device(key, value, indexes, what="GQA compaction")
    retained = int(indexes.shape[1])
    out_key = torch.empty((heads, retained, head_dim), dtype=key.dtype, device=device)
    out_value = torch.empty_like(out_key)
    ids64 = ids if ids.dtype == torch.int64 else ids.to(torch.int64)
    out_ids = torch.empty((heads, retained), dtype=torch.int64, device=device)
    scores32 = scores if scores.dtype == torch.float32 else scores.float()
    out_scores = torch.empty((heads, retained), dtype=torch.float32, device=device)
    nat.call(
        "uc_gqa_gather", key.data_ptr(), value.data_ptr(), *map(int, key_strides),
        nat.dtype_code(key.dtype), heads, head_dim, indexes.data_ptr(), retained,
        ids64.data_ptr(), int(ids_strides[0]), int(ids_strides[1]),
        scores32.data_ptr(), *map(int, scores32.stride()),
        out_key.data_ptr(), out_value.data_ptr(), out_ids.data_ptr(), out_scores.data_ptr(),
        nat.stream(device),
    )
    if ids.dtype != torch.int64:
        out_ids = out_ids.to(ids.dtype)
    return out_key, out_value, out_ids, out_scores


@dataclass
class GQAH2OCache:
    """Per-KV-head physical H2O cache with fixed-width selected storage
    (physical.py:478-654)."""

    key: torch.Tensor  # [kv_heads, retained_tokens, head_dim]
    value: torch.Tensor
    logical_token_ids: torch.Tensor  # [kv_heads, retained_tokens]
    cumulative_scores: torch.Tensor
    token_type_id: int
    original_tokens: int
    heavy_tokens: int
    recent_tokens: int
    selection_frozen: bool = False
    budget_shortfall_tokens: int = 0

    @classmethod
    def from_dense(
        cls,
        key: torch.Tensor,
        value: torch.Tensor,
        *,
        logical_token_ids: torch.Tensor,
        token_type_id: int,
        per_kv_head_scores: torch.Tensor,
        target_tokens: int,
        recent_tokens: int,
        selection_frozen: bool = False,
    ) -> "GQAH2OCache":
        """Select and gather one segment (physical.py:499-557)."""

        return cls.from_dense_segments([dict(
            key=key, value=value, logical_token_ids=logical_token_ids, token_type_id=token_type_id,
            per_kv_head_scores=per_kv_head_scores, target_tokens=target_tokens, recent_tokens=recent_tokens,
            selection_frozen=selection_frozen)])[0]

    @classmethod
    def from_dense_segments(cls, segments: list) -> list:
        """``from_dense`` for several segments -- each a dict of its keyword
        arguments plus ``key`` and ``value`` -- with one allocation and one
        uc_h2o_select_gather_segments launch for all of them (segments that
        share dtype, KV heads and head_dim; others are grouped by shape).
        Results equal one ``from_dense`` call per segment."""

        prepared = [cls._prepare(**seg) for seg in segments]
        out: list = [None] * len(prepared)
        groups: dict = {}
        for i, p in enumerate(prepared):
            groups.setdefault((p["key"].dtype, p["key"].device, p["kv_heads"], p["head_dim"]), []).append(i)
        for (dtype, device, kv_heads, head_dim), idx in groups.items():
            specs = []
            for i in idx:
                r = prepared[i]["retained"]
                specs += [((kv_heads, r), torch.int64), ((kv_heads, r, head_dim), dtype),
                          ((kv_heads, r, head_dim), dtype), ((kv_heads, r), torch.int64),
                          ((kv_heads, r), torch.float32)]
            views = _carve(specs, device)
            table = (nat.H2OSegment * len(idx))()
            for n, i in enumerate(idx):
                p = prepared[i]
                index, out_key, out_value, out_ids, out_scores = views[5 * n:5 * n + 5]
                key, scores, ids64 = p["key"], p["scores"], p["ids64"]
                table[n] = nat.H2OSegment(
                    key.data_ptr(), p["value"].data_ptr(), *map(int, key.stride()), scores.data_ptr(),
                    *map(int, scores.stride()), ids64.data_ptr(), 0, int(ids64.stride(0)), p["tokens"],
                    p["heavy_k"], p["recent"], index.data_ptr(), out_key.data_ptr(), out_value.data_ptr(),
                    out_ids.data_ptr(), out_scores.data_ptr())
                p["outputs"] = (out_key, out_value, out_ids, out_scores)
            nat.call("uc_h2o_select_gather_segments", table, len(idx), nat.dtype_code(dtype), kv_heads, head_dim,
                     nat.stream(device))
            for i in idx:
                p = prepared[i]
                out_key, out_value, out_ids, out_scores = p["outputs"]
                if p["ids_dtype"] != torch.int64:
                    out_ids = out_ids.to(p["ids_dtype"])
                out[i] = cls(
                    key=out_key,
                    value=out_value,
                    logical_token_ids=out_ids,
                    cumulative_scores=out_scores,
                    token_type_id=int(p["token_type_id"]),
                    original_tokens=p["tokens"],
                    heavy_tokens=p["heavy"],
                    recent_tokens=p["recent"],
                    selection_frozen=bool(p["selection_frozen"]),
                )
        return out

    @staticmethod
    def _prepare(*, key, value, logical_token_ids, token_type_id, per_kv_head_scores, target_tokens, recent_tokens,
                 selection_frozen=False) -> dict:
        """Checks and budget arithmetic of one segment (physical.py:499-515)."""

        if key.shape != value.shape or key.dim() != 3:
            raise ValueError("Physical H2O expects matching [tokens, kv_heads, head_dim] tensors")
        tokens, kv_heads, head_dim = map(int, key.shape)
        if tuple(per_kv_head_scores.shape) != (kv_heads, tokens):
            raise ValueError("Physical H2O scores must be [kv_heads, segment_tokens]")
        if key.stride() != value.stride():
            value = value.contiguous()
            key = key.contiguous()
        # budget arithmetic of physical.py:511-515
        target = min(tokens, max(1, int(target_tokens)))
        recent = min(target, max(0, int(recent_tokens)))
        heavy = target - recent
        history_end = tokens - recent
        heavy_k = min(heavy, history_end)
        logical = logical_token_ids.to(device=key.device)
        if logical.dim() != 1:
            raise ValueError("Physical H2O logical_token_ids must be [segment_tokens]")
        device = nat.require_device(key, value, logical, what="GQA compaction")
        scores = per_kv_head_scores.to(device=device)
        if scores.dtype != torch.float32:
            scores = scores.float()
        ids64 = logical if logical.dtype == torch.int64 else logical.to(torch.int64)
        return dict(key=key, value=value, scores=scores, ids64=ids64, ids_dtype=logical.dtype, tokens=tokens,
                    kv_heads=kv_heads, head_dim=head_dim, heavy=heavy, heavy_k=heavy_k, recent=recent,
                    retained=heavy_k + recent, token_type_id=token_type_id, selection_frozen=selection_frozen)

    @property
    def num_kv_heads(self) -> int:
        return int(self.key.shape[0])

    @property
    def retained_tokens(self) -> int:
        return int(self.key.shape[1])

    @property
    def resident_bytes(self) -> int:
        return sum(
            tensor_bytes(item)
            for item in (self.key, self.value, self.logical_token_ids, self.cumulative_scores)
        )

    @property
    def byte_breakdown(self) -> dict[str, int]:
        return {
            "payload_bytes": tensor_bytes(self.key) + tensor_bytes(self.value),
            "scale_bytes": 0,
            "minimum_bytes": 0,
            "residual_bytes": 0,
            "indices_bytes": tensor_bytes(self.logical_token_ids),
            "score_bytes": tensor_bytes(self.cumulative_scores),
        }

    @property
    def full_precision_bytes(self) -> int:
        return (
            self.original_tokens * self.num_kv_heads * int(self.key.shape[-1]) * 2 * self.key.element_size()
        )

    def attention_parts(
        self, query: torch.Tensor
    ) -> tuple[torch.Tensor, Callable[[torch.Tensor], torch.Tensor]]:
        """Scaled logits over the retained tokens and an AV closure
        (physical.py:585-596); the head-major [Hkv, R, D] storage is read in
        place through strides."""

        key = self.key.transpose(0, 1)
        value = self.value.transpose(0, 1)
        if query.dim() != 3 or int(query.shape[1]) % self.num_kv_heads:
            raise ValueError("GQA query heads must be divisible by KV heads")
        logits = _dense_qk(query, key, scale=1.0 / math.sqrt(query.shape[-1]))

        def apply_value(probabilities: torch.Tensor) -> torch.Tensor:
            return gqa_probability_value(probabilities, value)

        return logits, apply_value

    def update_scores(self, probabilities: torch.Tensor) -> None:
        """Accumulate the attention each surviving token receives per KV head
        (physical.py:598-610)."""

        if probabilities.dim() != 3:
            raise ValueError("H2O probabilities must be [query_heads, queries, tokens]")
        query_heads = int(probabilities.shape[0])
        if query_heads % self.num_kv_heads != 0:
            raise ValueError("Query heads must be divisible by KV heads for GQA H2O")
        device = nat.require_device(probabilities, self.cumulative_scores, what="H2O update")
        updated = self.cumulative_scores.float().clone()
        nat.call(
            "uc_h2o_colsum", probabilities.data_ptr(), nat.dtype_code(probabilities.dtype),
            *map(int, probabilities.stride()), query_heads, int(probabilities.shape[1]),
            self.retained_tokens, self.num_kv_heads, 1, updated.data_ptr(), nat.stream(device),
        )
        self.cumulative_scores = updated

    def update_scores_from_query(self, query: torch.Tensor, lse: torch.Tensor) -> None:
        """update_scores(exp(logits - lse).to(bf16)) for the retained keys without
        materialising the probabilities: the H2O update of a mixed-segment
        call, whose normaliser is the global LSE (adapters/bagel.py:1845-1856)."""

        from ..operators.physical import per_kv_head_scores_from_qk

        if query.dim() != 3 or int(query.shape[1]) % self.num_kv_heads:
            raise ValueError("Query heads must be divisible by KV heads for GQA H2O")
        q = query if query.dtype == self.key.dtype else query.to(self.key.dtype)
        updated = self.cumulative_scores.float().clone()
        per_kv_head_scores_from_qk(q, self.key.transpose(0, 1), out=updated, lse=lse)
        self.cumulative_scores = updated

    def enforce_budget(self) -> None:
        self.trim(self.heavy_tokens + self.recent_tokens, self.recent_tokens)

    def request_budget(self, target_tokens: int, recent_tokens: int) -> int:
        requested = max(1, int(target_tokens))
        effective = min(requested, self.retained_tokens)
        self.budget_shortfall_tokens += requested - effective
        self.recent_tokens = min(effective, max(0, int(recent_tokens)))
        self.heavy_tokens = effective - self.recent_tokens
        self.enforce_budget()
        return effective

    def trim(self, target_tokens: int, recent_tokens: int) -> None:
        """Per-head re-selection over the retained tokens (physical.py:624-654)."""

        target = min(self.retained_tokens, max(1, int(target_tokens)))
        if target >= self.retained_tokens:
            return
        recent = min(target, max(0, int(recent_tokens)))
        heavy = target - recent
        history_end = self.retained_tokens - recent
        heavy_k = min(heavy, history_end) if heavy else 0
        indexes = h2o_select_indices(self.cumulative_scores, heavy_k=heavy_k, recent=recent)
        key_strides = (self.key.stride(1), self.key.stride(0), self.key.stride(2))
        self.key, self.value, self.logical_token_ids, self.cumulative_scores = _gather(
            self.key, self.value, key_strides, indexes, self.logical_token_ids,
            (self.logical_token_ids.stride(0), self.logical_token_ids.stride(1)),
            self.cumulative_scores, heads=self.num_kv_heads, head_dim=int(self.key.shape[-1]),
        )


PhysicalSegment = PackedKIVICache | GQAH2OCache


@dataclass
class PhysicalLayerCache:
    segments: list[PhysicalSegment]

    @property
    def resident_bytes(self) -> int:
        return sum(segment.resident_bytes for segment in self.segments)

    @property
    def full_precision_bytes(self) -> int:
        return sum(segment.full_precision_bytes for segment in self.segments)

    def add(self, segment: PhysicalSegment) -> None:
        self.segments.append(segment)
