"""KIVI fake quantization (quantize-dequantize, no packing) on the MI355X
kernels: drop-in for asymmetric_fake_quant / kivi_fake_quant_key /
kivi_fake_quant_value of unicache/operators/builtin.py:31-65."""

from __future__ import annotations

import torch

from .. import _native as nat

SUPPORTED_FAKE_QUANT_BITS = frozenset({2, 3, 4, 8, 16})


def asymmetric_fake_quant(data: torch.Tensor, *, bits: int, dim: int, group_size: int) -> torch.Tensor:
    """Per-group asymmetric min-max quantize-dequantize of a [tokens, heads,
    head_dim] tensor along `dim` (0 or 2), groups of min(group_size, length)."""

    if data.numel() == 0 or bits >= 16:
        return data
    if bits not in SUPPORTED_FAKE_QUANT_BITS:
        raise ValueError(f"Unsupported fake quant bits: {bits}")
    if data.dim() != 3:
        raise ValueError("KIVI fake quantization expects [tokens, heads, head_dim] tensors")
    dim = dim if dim >= 0 else data.dim() + dim
    if dim not in (0, 2):
        raise ValueError("KIVI fake quantization groups along tokens (0) or channels (2)")
    device = nat.require_device(data, what="KIVI fake quantization")
    out = torch.empty_strided(data.shape, data.stride(), dtype=data.dtype, device=device)
    if not data.is_contiguous():
        data = data.contiguous()
        out = torch.empty_like(data)
    tokens, heads, head_dim = map(int, data.shape)
    nat.call(
        "uc_kivi_fake_quant", data.data_ptr(), *map(int, data.stride()), nat.dtype_code(data.dtype),
        tokens, heads, head_dim, int(bits), int(dim), int(group_size), out.data_ptr(), nat.stream(device),
    )
    return out


def kivi_fake_quant_key(k_segment: torch.Tensor, *, bits: int, group_size: int) -> torch.Tensor:
    # keys: groups along tokens, one scale/zero per (head, channel)
    return asymmetric_fake_quant(k_segment, bits=bits, dim=0, group_size=group_size)


def kivi_fake_quant_value(v_segment: torch.Tensor, *, bits: int, group_size: int) -> torch.Tensor:
    # values: groups along head_dim, one scale/zero per (token, head)
    return asymmetric_fake_quant(v_segment, bits=bits, dim=-1, group_size=group_size)
