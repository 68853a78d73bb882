"""All-layer decode over many packed KIVI segments in one launch.

KiviDecodeBatch fixes, once, a device table of (packed segment, residual,
query, output) items -- e.g. every (layer, sequence) of a decode step -- plus
the outputs and the split-K workspace.  run() then enqueues a single
uc_kivi_attn_decode_batch launch (and its LSE combine) and allocates nothing,
so it can sit in a tight decode loop or a captured HIP graph.  Callers update
the query tensors in place between steps.

The device tables hold raw pointers, so both classes check every pointer on
the host when they build a table (device, the token-major packed layout,
contiguity and 16-byte alignment of the vector-loaded rows), keep the tensors
behind the table alive, and refuse
to run once a packed cache has replaced its tensors (append, flush, repack)
until refresh() rebuilds the table.
"""

from __future__ import annotations

import ctypes
import math

import torch

from .. import _native as nat

_PACKED = ("key_code", "key_scale", "key_minimum", "value_code", "value_scale", "value_minimum")


def _check_rows(t: torch.Tensor, device: torch.device, what: str) -> None:
    """A tensor whose rows the decode kernels read by address: on `device`,
    contiguous, 16-byte aligned."""

    if t.device != device:
        raise RuntimeError(f"{what} must be on {device} (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if t.data_ptr() % 16:
        raise ValueError(f"{what} must be 16-byte aligned")


def _check_cache(c, device: torch.device, what: str) -> list[torch.Tensor]:
    """Validate a packed cache's tensors for a device item table (the
    token-major native layout, on `device`); returns the tensors the table
    will point into."""

    try:
        c.native_packed_pointers(device)
    except (ValueError, RuntimeError) as exc:
        raise type(exc)(f"{what}: {exc}") from None
    tensors = [getattr(c, name) for name in _PACKED]
    if c.residual_tokens:
        _check_rows(c.residual_key, device, f"{what}: residual_key")
        _check_rows(c.residual_value, device, f"{what}: residual_value")
        tensors += [c.residual_key, c.residual_value]
    return tensors


class _TableGuard:
    """The tensors behind a device item table and the mutation counts of its
    packed caches when the table was built."""

    def __init__(self, caches, tensors) -> None:
        self.tensors = list(tensors)
        self.caches = list(caches)
        self.counts = [c.mutation_count for c in self.caches]

    def check(self, what: str) -> None:
        for c, n in zip(self.caches, self.counts):
            if c.mutation_count != n:
                raise RuntimeError(f"{what}: a packed cache changed since the item table was built; call refresh()")


class KiviDecodeBatch:
    def __init__(self, caches, queries, *, out_dtype: torch.dtype | None = None):
        if not caches or len(caches) != len(queries):
            raise ValueError("KiviDecodeBatch needs one query per packed segment")
        first = caches[0]
        for c in caches:
            if not c.kernel_native_layout or c.k_bits != c.v_bits or c.k_bits not in (2, 4):
                raise ValueError("Batched decode needs native equal 2/4-bit packed segments")
            if (c.k_bits, c.group_size, c.num_kv_heads, c.head_dim) != (
                first.k_bits, first.group_size, first.num_kv_heads, first.head_dim
            ):
                raise ValueError("Batched decode segments must share bits, group size and head shapes")
        q0 = queries[0]
        self.device = nat.require_device(*queries, first.key_code, what="Batched KIVI decode")
        for q in queries:
            if q.shape != q0.shape or q.dtype != q0.dtype:
                raise ValueError("Batched decode queries must be of one shape/dtype")
            _check_rows(q, self.device, "Batched decode query")
        lq, hq, d = map(int, q0.shape)
        if hq % first.num_kv_heads:
            raise ValueError("Query heads must be divisible by KIVI KV heads")
        res_dtypes = {c.residual_key.dtype for c in caches if c.residual_tokens}
        if len(res_dtypes) > 1:
            raise ValueError("Batched decode residuals must share one dtype")
        self.res_dtype = res_dtypes.pop() if res_dtypes else q0.dtype
        self.out_dtype = out_dtype or q0.dtype
        self.caches = list(caches)
        self.queries = list(queries)
        self.outputs = [torch.empty((lq, hq, d), dtype=self.out_dtype, device=self.device) for _ in caches]
        self.lses = [torch.empty((hq, lq), dtype=torch.float32, device=self.device) for _ in caches]
        self.shape = (lq, hq, d)
        self.sm_scale = 1.0 / math.sqrt(d)
        self.workspace = None
        self.refresh()

    def refresh(self) -> None:
        """(Re)build the device item table from the caches' current tensors."""

        caches, queries = self.caches, self.queries
        first = caches[0]
        lq, hq, d = self.shape
        tensors = list(queries) + self.outputs + self.lses
        for c in caches:
            tensors += _check_cache(c, self.device, "Batched KIVI decode")
        items = (nat.KiviItem * len(caches))()
        for i, (c, q) in enumerate(zip(caches, queries)):
            tr = c.residual_tokens
            items[i] = c.native_item(q.data_ptr(), self.outputs[i].data_ptr(), self.lses[i].data_ptr(),
                                     residual_key_ptr=c.residual_key.data_ptr() if tr else None,
                                     residual_value_ptr=c.residual_value.data_ptr() if tr else None,
                                     residual_tokens=tr)
        raw = bytes(ctypes.string_at(ctypes.addressof(items), ctypes.sizeof(items)))
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)
        self.max_tq = max(c.quantized_tokens for c in caches)
        self.max_tr = max(c.residual_tokens for c in caches)
        self.ws_bytes = nat.decode_workspace_bytes(len(caches), first.k_bits, first.group_size, hq,
                                                   first.num_kv_heads, d, lq, self.max_tq, self.max_tr)
        if self.workspace is None or self.workspace.numel() < self.ws_bytes:
            self.workspace = nat.workspace(self.device, self.ws_bytes)
        self._guard = _TableGuard(caches, tensors)

    @property
    def algorithmic_bytes(self) -> int:
        """HBM bytes one run must move at least once: packed codes + stats,
        residual K/V, queries and outputs."""

        total = 0
        for c, q, o in zip(self.caches, self.queries, self.outputs):
            for t in (c.key_code, c.key_scale, c.key_minimum, c.value_code, c.value_scale, c.value_minimum):
                total += t.numel() * t.element_size()
            total += 2 * c.residual_key.numel() * c.residual_key.element_size()
            total += q.numel() * q.element_size() + o.numel() * o.element_size()
        return total

    def run(self, stream: int | None = None) -> None:
        self._guard.check("KiviDecodeBatch.run")
        lq, hq, d = self.shape
        first = self.caches[0]
        nat.call(
            "uc_kivi_attn_decode_batch", self.table.data_ptr(), len(self.caches), first.k_bits,
            first.group_size, hq, first.num_kv_heads, d, lq, nat.dtype_code(self.queries[0].dtype),
            nat.dtype_code(self.res_dtype), nat.dtype_code(self.out_dtype), self.sm_scale, self.max_tq,
            self.max_tr, self.workspace.data_ptr(), self.ws_bytes,
            nat.stream(self.device) if stream is None else stream,
        )


class MixedDecodeBatch:
    """Decode over groups of KV segments that share one query: each group is a
    list of PackedKIVICache segments and dense (key, value) [T, Hkv, D]
    segments (bf16 H2O / protected tokens) and is attended as one softmax over
    all of them by a single uc_kivi_attn_decode_segments launch for every
    group -- the decode form of _run_fused_mixed_attention
    (adapters/bagel.py:1598-1858) without concatenating the segments.

    Dense segments and residual windows must share one dtype (the kernel reads
    them as fp16 either way).  refresh() rebuilds the item table after
    segments change (a residual append or flush); run() allocates nothing."""

    def __init__(self, groups, queries, *, out_dtype: torch.dtype | None = None):
        if not groups or len(groups) != len(queries):
            raise ValueError("MixedDecodeBatch needs one query per segment group")
        packed = [s for g in groups for s in g if not isinstance(s, tuple)]
        if not packed:
            raise ValueError("MixedDecodeBatch needs at least one packed segment")
        first = packed[0]
        for c in packed:
            if not c.kernel_native_layout or c.k_bits != c.v_bits or c.k_bits not in (2, 4):
                raise ValueError("Mixed decode needs native equal 2/4-bit packed segments")
            if (c.k_bits, c.group_size, c.num_kv_heads, c.head_dim) != (
                first.k_bits, first.group_size, first.num_kv_heads, first.head_dim
            ):
                raise ValueError("Mixed decode packed segments must share bits, group size and head shapes")
        q0 = queries[0]
        self.device = nat.require_device(*queries, first.key_code, what="Mixed KIVI decode")
        for q in queries:
            if q.shape != q0.shape or q.dtype != q0.dtype:
                raise ValueError("Mixed decode queries must be of one shape/dtype")
            _check_rows(q, self.device, "Mixed decode query")
        lq, hq, d = map(int, q0.shape)
        dtypes = set()
        for g in groups:
            for s in g:
                if isinstance(s, tuple):
                    k, v = s
                    if k.shape != v.shape or k.dim() != 3 or tuple(k.shape[1:]) != (first.num_kv_heads, d):
                        raise ValueError("Dense segments must be matching [tokens, kv_heads, head_dim] tensors")
                    if k.dtype != v.dtype:
                        raise ValueError("Dense segment keys and values must share one dtype")
                    dtypes.add(k.dtype)
                elif s.residual_tokens:
                    dtypes.add(s.residual_key.dtype)
        if len(dtypes) > 1:
            raise ValueError("Dense segments and residual windows must share one dtype")
        self.res_dtype = dtypes.pop() if dtypes else q0.dtype
        self.out_dtype = out_dtype or q0.dtype
        self.bits, self.group_size, self.kv_heads = first.k_bits, first.group_size, first.num_kv_heads
        self.groups = [list(g) for g in groups]
        self.queries = list(queries)
        self.segs = max(len(g) for g in groups)
        self.outputs = [torch.empty((lq, hq, d), dtype=self.out_dtype, device=self.device) for _ in groups]
        self.lses = [torch.empty((hq, lq), dtype=torch.float32, device=self.device) for _ in groups]
        self.shape = (lq, hq, d)
        self.sm_scale = 1.0 / math.sqrt(d)
        self.refresh()

    def refresh(self) -> None:
        """(Re)build the device item table from the segments' current tensors."""

        tensors = list(self.queries) + self.outputs + self.lses
        caches = []
        for g in self.groups:
            for s in g:
                if isinstance(s, tuple):
                    if int(s[0].shape[0]):
                        _check_rows(s[0], self.device, "Mixed decode dense key segment")
                        _check_rows(s[1], self.device, "Mixed decode dense value segment")
                    tensors += list(s)
                else:
                    tensors += _check_cache(s, self.device, "Mixed KIVI decode")
                    caches.append(s)
        n = len(self.groups) * self.segs
        items = (nat.KiviItem * n)()
        max_tq = max_tr = 0
        for gi, (g, q) in enumerate(zip(self.groups, self.queries)):
            out, lse = self.outputs[gi], self.lses[gi]
            for j in range(self.segs):
                idx = gi * self.segs + j
                s = g[j] if j < len(g) else None
                if s is None:  # padding: an empty segment
                    items[idx] = nat.KiviItem(None, None, None, None, None, None, None, None, q.data_ptr(),
                                              out.data_ptr(), lse.data_ptr(), 0, 0, 0)
                elif isinstance(s, tuple):
                    k, v = s
                    tr = int(k.shape[0])
                    items[idx] = nat.KiviItem(None, None, None, None, None, None, k.data_ptr() if tr else None,
                                              v.data_ptr() if tr else None, q.data_ptr(), out.data_ptr(),
                                              lse.data_ptr(), 0, tr, 0)
                    max_tr = max(max_tr, tr)
                else:
                    tr = s.residual_tokens
                    items[idx] = s.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                               residual_key_ptr=s.residual_key.data_ptr() if tr else None,
                                               residual_value_ptr=s.residual_value.data_ptr() if tr else None,
                                               residual_tokens=tr)
                    max_tq, max_tr = max(max_tq, s.quantized_tokens), max(max_tr, tr)
        raw = bytes(ctypes.string_at(ctypes.addressof(items), ctypes.sizeof(items)))
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)
        self.n_items, self.max_tq, self.max_tr = n, max_tq, max_tr
        lq, hq, d = self.shape
        self.ws_bytes = nat.decode_workspace_bytes(n, self.bits, self.group_size, hq, self.kv_heads, d, lq,
                                                   max_tq, max_tr)
        if getattr(self, "workspace", None) is None or self.workspace.numel() < self.ws_bytes:
            self.workspace = nat.workspace(self.device, self.ws_bytes)
        self._guard = _TableGuard(caches, tensors)

    @property
    def algorithmic_bytes(self) -> int:
        """Packed codes + stats, residual and dense K/V, queries and outputs,
        each counted once."""

        total = 0
        for g, q, o in zip(self.groups, self.queries, self.outputs):
            for s in g:
                if isinstance(s, tuple):
                    total += sum(t.numel() * t.element_size() for t in s)
                    continue
                for t in (s.key_code, s.key_scale, s.key_minimum, s.value_code, s.value_scale, s.value_minimum):
                    total += t.numel() * t.element_size()
                total += 2 * s.residual_key.numel() * s.residual_key.element_size()
            total += q.numel() * q.element_size() + o.numel() * o.element_size()
        return total

    def run(self, stream: int | None = None) -> None:
        self._guard.check("MixedDecodeBatch.run")
        lq, hq, d = self.shape
        nat.call(
            "uc_kivi_attn_decode_segments", self.table.data_ptr(), self.n_items, self.segs, self.bits,
            self.group_size, hq, self.kv_heads, d, lq, nat.dtype_code(self.queries[0].dtype),
            nat.dtype_code(self.res_dtype), nat.dtype_code(self.out_dtype), self.sm_scale, self.max_tq,
            self.max_tr, self.workspace.data_ptr(), self.ws_bytes,
            nat.stream(self.device) if stream is None else stream,
        )
