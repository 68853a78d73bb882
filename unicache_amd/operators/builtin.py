"""KIVI fake quantization (quantize-dequantize, no packing) on the MI355X
kernels: drop-in for asymmetric_fake_quant / kivi_fake_quant_key /
kivi_fake_quant_value of unicache/operators/builtin.py:31-65 and the
KIVIQuantizationOperator that applies them to a cache segment
(operators/builtin.py:281-476)."""

from __future__ import annotations

import math

import torch

from .. import _native as nat
from ..core.capabilities import CapabilityDescriptor
from ..core.registry import OperatorExecutionContext, ProcessingOperator

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


class KIVIQuantizationOperator(ProcessingOperator):
    """KIVI fake quantization of one cache segment in the attention view
    (operators/builtin.py:281-476): the segment's tokens except its last
    `residual_length` and, with preserve_protected, the protected ones are
    quantized and dequantized in place of the originals -- keys in groups of
    `group_size` selected tokens per channel, values in groups of channels per
    token.  The selected rows are gathered, fake-quantized and written back by
    HIP kernels (mask scan, row copies, uc_kivi_fake_quant, uc_scatter_rows);
    the record and storage-snapshot keys are UniCache's.  The host-backed
    working set (an offload-hierarchy replica) is not part of this build."""

    family = "quantization"
    stages = {"pre_attention", "attention"}
    executable = True
    capabilities = CapabilityDescriptor(
        stages=frozenset(stages),
        layouts=frozenset({"attention_view", "dense"}),
        devices=frozenset({"cuda"}),
        requires=frozenset({"key", "value", "segment_mask", "cache_storage_view"}),
        mutation_scope="attention_view",
        physical_storage_mutation=False,
        accepts_quantized_input=False,
    )

    def __init__(self, name: str = "kivi_quantization") -> None:
        self.name = name

    def build_params(self, params: dict) -> dict:
        out = dict(params)
        bits = int(out.get("bits", 4))
        for name, value in (("bits", bits), ("k_bits", out.get("k_bits", bits)), ("v_bits", out.get("v_bits", bits))):
            if int(value) not in SUPPORTED_FAKE_QUANT_BITS:
                raise ValueError(
                    f"{self.name} {name}={value} is unsupported; expected one of {sorted(SUPPORTED_FAKE_QUANT_BITS)}"
                )
        working_set_mode = str(out.get("working_set_mode", "attention_view"))
        if working_set_mode not in {"attention_view", "host_backed"}:
            raise ValueError(f"{self.name} working_set_mode must be attention_view or host_backed")
        if working_set_mode == "host_backed":
            raise ValueError(f"{self.name} working_set_mode host_backed needs the offload hierarchy, "
                             "which this build does not include")
        out["working_set_mode"] = working_set_mode
        return out

    def execute(self, ctx: OperatorExecutionContext) -> OperatorExecutionContext:
        bits = int(ctx.params.get("bits", 4))
        k_bits = int(ctx.params.get("k_bits", bits))
        v_bits = int(ctx.params.get("v_bits", bits))
        group_size = int(ctx.params.get("group_size", 32))
        residual_length = int(ctx.params.get("residual_length", 32))
        preserve_protected = bool(ctx.params.get("preserve_protected", True))
        bypass_quantization = bool(ctx.params.get("bypass_quantization", False))
        if str(ctx.params.get("working_set_mode", "attention_view")) != "attention_view":
            raise ValueError(f"{self.name} supports the attention_view working set only")

        device = nat.require_device(ctx.k, ctx.v, what="KIVI fake quantization")
        segment = ctx.segment_mask.to(device=device, dtype=torch.bool).contiguous()
        protected = ctx.protected_mask.to(device=device, dtype=torch.bool).contiguous()
        n = int(segment.numel())
        if int(protected.numel()) != n:
            raise RuntimeError("segment_mask and protected_mask must have the same length")
        # one launch: the rows to quantize -- segment tokens but the last
        # residual_length of them and, with preserve, the protected ones; none
        # with bypass -- their compact order, and the three counts; one host read
        dst = torch.empty(max(n, 1), dtype=torch.int32, device=device)
        src = torch.empty(max(n, 1), dtype=torch.int32, device=device)
        counts = torch.empty(3, dtype=torch.int64, device=device)
        nat.call("uc_fake_quant_mask", segment.data_ptr(), protected.data_ptr(), n, residual_length,
                 int(preserve_protected), int(bypass_quantization), dst.data_ptr(), src.data_ptr(),
                 counts.data_ptr(), nat.stream(device))
        segment_tokens, quant_tokens, protected_in_segment = map(int, counts.tolist())

        full_precision_tokens = segment_tokens - quant_tokens
        elem_bytes = max(1, ctx.k.element_size())
        attention_num_heads = int(ctx.k.shape[1])
        storage_num_kv_heads = int(
            ctx.storage.layout.num_kv_heads
            if ctx.storage is not None
            else (ctx.storage_num_kv_heads or attention_num_heads)
        )
        head_dim = int(ctx.k.shape[2])
        attention_elements_per_token = attention_num_heads * head_dim
        storage_elements_per_token = storage_num_kv_heads * head_dim
        original_storage = float(segment_tokens * storage_elements_per_token * 2 * elem_bytes)
        full_precision_bytes = float(full_precision_tokens * storage_elements_per_token * 2 * elem_bytes)
        key_groups = math.ceil(quant_tokens / max(1, group_size)) if quant_tokens else 0
        value_groups = math.ceil(head_dim / max(1, group_size)) if quant_tokens else 0
        # fp32 min/scale metadata: the ideal packed estimate of the reference
        metadata_bytes = float(
            (key_groups * storage_num_kv_heads * head_dim + quant_tokens * storage_num_kv_heads * value_groups) * 2 * 4
        )
        packed_payload_bytes = float((quant_tokens * storage_elements_per_token * (k_bits + v_bits)) / 8.0)
        ideal_storage = full_precision_bytes + packed_payload_bytes + metadata_bytes

        if quant_tokens > 0:
            ctx.k, ctx.v = _fake_quant_rows_at(ctx.k, ctx.v, dst[:n], quant_tokens, k_bits=k_bits, v_bits=v_bits,
                                               group_size=group_size)
        ctx.record({
            "quantized_tokens": quant_tokens,
            "protected_tokens_preserved": protected_in_segment if preserve_protected else 0,
            "processed_input_kv_bytes": float(quant_tokens * attention_elements_per_token * 2 * elem_bytes),
            "quantized_replica_cache_hit": 0.0,
        })
        ctx.set_storage_snapshot({
            "segment_tokens": segment_tokens,
            "quantized_tokens": quant_tokens,
            "full_precision_tokens": full_precision_tokens,
            "attention_num_heads": attention_num_heads,
            "storage_num_kv_heads": storage_num_kv_heads,
            "gqa_repeat": float(attention_num_heads / max(storage_num_kv_heads, 1)),
            "original_storage_bytes": original_storage,
            "ideal_packed_payload_bytes": packed_payload_bytes,
            "ideal_metadata_bytes": metadata_bytes,
            "ideal_total_storage_bytes": ideal_storage,
            "logical_host_backed": 0.0,
        })
        return ctx


def fake_quant_rows(key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor, count: int, *, k_bits: int,
                    v_bits: int, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Copies of [T, H, D] key / value whose rows under `mask` (`count` of
    them) are replaced by kivi_fake_quant_key / _value of those rows taken in
    order -- key[mask] = fake_quant(key[mask]) of operators/builtin.py:420-430,
    on the mask scan, row copy and row scatter kernels."""

    from ..storage.tensor_backend import _aligned_mask, _scan

    device = nat.require_device(key, value, mask, what="KIVI fake quantization")
    dst, _ = _scan(_aligned_mask(mask, device))
    return _fake_quant_rows_at(key, value, dst, count, k_bits=k_bits, v_bits=v_bits, group_size=group_size)


def _fake_quant_rows_at(key: torch.Tensor, value: torch.Tensor, dst: torch.Tensor, count: int, *, k_bits: int,
                        v_bits: int, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fake_quant_rows with the compact order of the rows (dst, -1 for the
    others) already on the device: K and V rows gathered in one launch,
    fake-quantized, and scattered into copies of K and V."""

    from ..storage.tensor_backend import _copy_rows_many

    device = key.device
    stream = nat.stream(device)
    rows_k, rows_v = _copy_rows_many([key, value], dst, count)
    outs = []
    for data, rows, fq, b in ((key, rows_k, kivi_fake_quant_key, k_bits), (value, rows_v, kivi_fake_quant_value,
                                                                          v_bits)):
        rows = fq(rows, bits=b, group_size=group_size)
        out = data.clone(memory_format=torch.contiguous_format)
        row_bytes = int(rows[0].numel()) * rows.element_size()
        nat.call("uc_scatter_rows", rows.contiguous().data_ptr(), row_bytes, dst.data_ptr(), int(dst.numel()),
                 out.data_ptr(), int(out.stride(0)) * out.element_size(), stream)
        outs.append(out)
    return outs[0], outs[1]
