"""ctypes binding of libunicache_hip.so (the C ABI in include/unicache_hip.h).

The library is loaded lazily on first use, after ``torch`` so that it binds to
the HIP runtime torch already loaded.  A missing or incompatible library
raises ``RuntimeError``: the engine has no CPU or torch fallback.
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libunicache_hip.so")
ABI_VERSION = 3

UC_BF16, UC_FP16, UC_FP32 = 0, 1, 2
UC_OK, UC_EINVAL, UC_ERUNTIME = 0, -1, -2
UC_OP_KIVI_AV, UC_OP_H2O_SCORES = 2, 3

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float


class KiviItem(ctypes.Structure):
    """Mirror of ``uc_kivi_item``."""

    _fields_ = [
        ("key_code", _P),
        ("key_scale", _P),
        ("key_min", _P),
        ("value_code", _P),
        ("value_scale", _P),
        ("value_min", _P),
        ("residual_key", _P),
        ("residual_value", _P),
        ("query", _P),
        ("out", _P),
        ("lse", _P),
        ("quantized_tokens", _L),
        ("residual_tokens", _L),
        ("packed_capacity", _L),
        ("residual_token_stride", _L),
        ("residual_head_stride", _L),
    ]


class DenseSegment(ctypes.Structure):
    """Mirror of ``uc_dense_segment`` (strides in elements)."""

    _fields_ = [
        ("key", _P),
        ("value", _P),
        ("tokens", _L),
        ("token_stride", _L),
        ("head_stride", _L),
    ]


class AppendEntry(ctypes.Structure):
    """Mirror of ``uc_append_entry``."""

    _fields_ = [("item", _L), ("advance", _L), ("ids", _P)]


class H2OSegment(ctypes.Structure):
    """Mirror of ``uc_h2o_segment``."""

    _fields_ = [
        ("key", _P), ("value", _P), ("k_st", _L), ("k_sh", _L), ("k_sd", _L),
        ("scores", _P), ("s_sh", _L), ("s_st", _L),
        ("ids", _P), ("ids_sh", _L), ("ids_st", _L),
        ("tokens", _L), ("heavy_k", _L), ("recent", _L),
        ("indices", _P), ("out_key", _P), ("out_value", _P), ("out_ids", _P), ("out_scores", _P),
    ]


class RowCopy(ctypes.Structure):
    """Mirror of ``uc_row_copy``."""

    _fields_ = [("src", _P), ("src_row_stride_bytes", _L), ("row_bytes", _L), ("dst", _P)]


class MqQuery(ctypes.Structure):
    """Mirror of ``uc_mq_query``."""

    _fields_ = [
        ("query", _P),
        ("out", _P),
        ("lse", _P),
        ("query_len", _L),
        ("packed_begin", ctypes.c_int32),
        ("n_packed", ctypes.c_int32),
        ("dense_begin", ctypes.c_int32),
        ("n_dense", ctypes.c_int32),
    ]


# name -> (restype, argtypes)
_SIGNATURES = {
    "uc_abi_version": (_I, []),
    "uc_last_error": (ctypes.c_char_p, []),
    "uc_kivi_pack": (
        _I,
        [_P, _L, _L, _L, _P, _L, _L, _L, _I, _L, _L, _L, _I, _I, _I, _I,
         _P, _L, _L, _L, _P, _P, _L, _L, _L,
         _P, _L, _L, _L, _P, _P, _L, _L, _L, _P],
    ),
    "uc_kivi_dequant": (
        _I,
        [_P, _L, _L, _L, _P, _P, _L, _L, _L,
         _P, _L, _L, _L, _P, _P, _L, _L, _L,
         _I, _L, _L, _I, _I, _I, _L, _L, _P, _P, _I, _L, _L, _L, _L, _P],
    ),
    "uc_kivi_fake_quant": (_I, [_P, _L, _L, _L, _I, _L, _L, _L, _I, _I, _I, _P, _P]),
    "uc_kivi_qk": (
        _I,
        [_P, _I, _L, _L, _P, _P, _P, _I, _L, _L, _I, _I, _P, _I, _L, _L, _L, _L, _L, _F, _P, _P],
    ),
    "uc_kivi_av": (
        _I,
        [_P, _I, _L, _L, _L, _L, _L, _P, _P, _P, _I, _L, _L, _I, _I, _P, _I, _L, _L, _L, _L, _L,
         _P, _I, _P, _P],
    ),
    "uc_kivi_attn_decode": (
        _I,
        [ctypes.POINTER(KiviItem), _I, _I, _L, _L, _L, _L, _I, _I, _I, _F, _P, _L, _P],
    ),
    "uc_kivi_attn_decode_static": (
        _I,
        [ctypes.POINTER(KiviItem), _I, _I, _L, _L, _L, _L, _I, _I, _I, _F, _P],
    ),
    "uc_kivi_decode_scratch_bytes": (_L, []),
    "uc_kivi_attn_decode_batch": (
        _I,
        [_P, _L, _I, _I, _L, _L, _L, _L, _I, _I, _I, _F, _L, _L, _P, _L, _P],
    ),
    "uc_kivi_attn_decode_segments_host": (
        _I,
        [ctypes.POINTER(KiviItem), _L, _I, _I, _L, _L, _L, _L, _I, _I, _I, _F, _P, _L, _P],
    ),
    "uc_kivi_attn_decode_segments": (
        _I,
        [_P, _L, _L, _I, _I, _L, _L, _L, _L, _I, _I, _I, _F, _L, _L, _P, _L, _P],
    ),
    "uc_kivi_attn_mq": (_I, [ctypes.POINTER(KiviItem), _I, _I, _L, _L, _L, _L, _I, _I, _I, _F, _P, _L, _P]),
    "uc_kivi_mq_workspace_bytes": (_L, [_L, _L, _L, _L]),
    "uc_kivi_attn_mq_batch": (
        _I,
        [ctypes.POINTER(KiviItem), ctypes.POINTER(ctypes.c_int64), _I, _I, _I, _L, _L, _L, _I, _I, _I, _F, _P, _L,
         _P],
    ),
    "uc_kivi_attn_mq_segments": (
        _I,
        [ctypes.POINTER(KiviItem), _I, ctypes.POINTER(DenseSegment), _I, _P, _P, _P, _I, _I, _L, _L, _L, _L,
         _I, _I, _I, _F, _P],
    ),
    "uc_kivi_attn_mq_table": (
        _I,
        [ctypes.POINTER(MqQuery), _I, ctypes.POINTER(KiviItem), _I, ctypes.POINTER(DenseSegment), _I, _I, _I, _L,
         _L, _L, _I, _I, _I, _F, _P],
    ),
    "uc_lse_merge": (_I, [_P, _P, _I, _I, _L, _L, _L, _P, _P, _P]),
    "uc_h2o_scores": (
        _I,
        [_P, _L, _L, _L, _P, _L, _L, _L, _I, _L, _L, _L, _L, _L, _F, _I, _P, _P, _P],
    ),
    "uc_h2o_scores_lse": (
        _I,
        [_P, _L, _L, _L, _P, _L, _L, _L, _I, _L, _L, _L, _L, _L, _F, _P, _I, _P, _P, _P],
    ),
    "uc_h2o_colsum": (_I, [_P, _I, _L, _L, _L, _L, _L, _L, _L, _I, _P, _P]),
    "uc_h2o_select": (_I, [_P, _L, _L, _L, _L, _L, _L, _P, _P]),
    "uc_mask_scan": (_I, [_P, _L, _P, _P, _P]),
    "uc_compact_rows": (_I, [_P, _L, _L, _P, _L, _P, _P]),
    "uc_scatter_rows": (_I, [_P, _L, _P, _L, _P, _L, _P]),
    "uc_copy_spans": (_I, [_P, _I, _P]),
    "uc_kivi_residual_append": (_I, [_P, _P, _I, _P, _P, _P, _L, _L, _L, _I, _P]),
    "uc_compact_rows_multi": (_I, [ctypes.POINTER(RowCopy), _I, _P, _L, _P]),
    "uc_fake_quant_mask": (_I, [_P, _P, _L, _L, _I, _I, _P, _P, _P, _P]),
    "uc_h2o_select_gather_segments": (_I, [ctypes.POINTER(H2OSegment), _I, _I, _L, _L, _P]),
    "uc_h2o_select_gather": (
        _I,
        [_P, _P, _L, _L, _L, _I, _L, _L, _L, _P, _L, _L, _L, _L, _P, _L, _L, _P, _P, _P, _P, _P, _P],
    ),
    "uc_gqa_gather": (
        _I,
        [_P, _P, _L, _L, _L, _I, _L, _L, _P, _L, _P, _L, _L, _P, _L, _L, _P, _P, _P, _P, _P],
    ),
    "uc_workspace_bytes": (_L, [_I, _L, _L, _L, _L, _L]),
    "uc_kivi_decode_workspace_bytes": (_L, [_L, _I, _I, _L, _L, _L, _L, _L, _L]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    """Names of the C entry points this binding expects the library to export."""

    return sorted(_SIGNATURES)


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library (without touching the GPU) and declare signatures."""

    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                "libunicache_hip.so is not built; run `python -m unicache_amd.build` "
                "(the MI355X engine has no CPU fallback)"
            )
        try:
            lib = ctypes.CDLL(path)
        except OSError as exc:
            raise RuntimeError(f"Cannot load {path}: {exc}") from exc
        for name, (restype, argtypes) in _SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise RuntimeError(f"{path} does not export {name}") from exc
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.uc_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(
                f"libunicache_hip.so ABI version {version} != expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load_library()


def check(rc: int, name: str) -> None:
    """Map a C return code to the reference's exception types."""

    if rc == UC_OK:
        return
    message = (lib().uc_last_error() or b"").decode(errors="replace") or f"{name} failed"
    if rc == UC_EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


_DTYPE_CODES = {torch.bfloat16: UC_BF16, torch.float16: UC_FP16, torch.float32: UC_FP32}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise ValueError(f"Unsupported dtype for the MI355X kernels: {dtype}") from exc


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device: torch.device) -> int:
    """The current HIP stream of `device` as an address."""

    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor | None, what: str) -> torch.device:
    """All given tensors must live on one GPU; returns that device."""

    device = None
    for tensor in tensors:
        if tensor is None:
            continue
        if tensor.device.type != "cuda":
            raise RuntimeError(f"{what} requires GPU tensors (got {tensor.device})")
        if device is None:
            device = tensor.device
        elif tensor.device != device:
            raise RuntimeError(f"{what} received tensors on different devices")
    if device is None:
        raise RuntimeError(f"{what} received no GPU tensor")
    return device


@functools.lru_cache(maxsize=256)
def workspace_bytes(op: int, n_items: int, heads_q: int, query_len: int, head_dim: int, max_tokens: int) -> int:
    size = int(lib().uc_workspace_bytes(op, n_items, heads_q, query_len, head_dim, max_tokens))
    if size < 0:
        raise ValueError("uc_workspace_bytes: unknown operation")
    return size


@functools.lru_cache(maxsize=256)
def decode_workspace_bytes(n_items, bits, group_size, heads_q, heads_kv, head_dim, query_len, max_tq, max_tr) -> int:
    size = int(lib().uc_kivi_decode_workspace_bytes(n_items, bits, group_size, heads_q, heads_kv, head_dim,
                                                    query_len, max_tq, max_tr))
    if size < 0:
        raise ValueError("uc_kivi_decode_workspace_bytes: bad arguments")
    return size


def mq_workspace_bytes(heads_kv, head_dim, quantized_tokens, residual_tokens) -> int:
    size = int(lib().uc_kivi_mq_workspace_bytes(heads_kv, head_dim, quantized_tokens, residual_tokens))
    if size < 0:
        raise ValueError("uc_kivi_mq_workspace_bytes: bad arguments")
    return size


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A caller-owned uint8 workspace from torch's caching allocator."""

    return torch.empty(max(1, int(nbytes)), dtype=torch.uint8, device=device)
