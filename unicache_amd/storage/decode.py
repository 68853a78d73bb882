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
    segments change (a residual append or flush); run() allocates nothing.

    Streaming decode: reserve(tokens) gives every packed segment room for that
    many appended tokens; append() then adds a decode step's tokens to every
    packed segment's residual window with one launch that also updates the
    device item table (uc_kivi_residual_append), and flushes windows that
    reach `flush_at` into the packed prefix in place -- no refresh, no host
    copy of the table, no allocation until the reserve is used up."""

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
        self._room = 0  # tokens every packed segment can still take without allocating
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
        streams = self._attach_streams(caches) if self._room > 0 else {}
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
                    st = streams.get(id(s))
                    rk = s.residual_key.data_ptr() if tr else None
                    rv = s.residual_value.data_ptr() if tr else None
                    if st is not None:
                        # a streamed window is addressed even while empty
                        # (appends write there); an empty view has no address
                        buf, row = st[2].buf, s.num_kv_heads * s.head_dim * st[2].buf.element_size()
                        rk = buf.data_ptr() + st[2].off * row
                        rv = buf.data_ptr() + (int(buf.shape[1]) + st[2].off) * row
                        st[1].item = idx
                    items[idx] = s.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                               residual_key_ptr=rk, residual_value_ptr=rv, residual_tokens=tr)
                    max_tq, max_tr = max(max_tq, s.quantized_tokens), max(max_tr, tr)
        raw = bytes(ctypes.string_at(ctypes.addressof(items), ctypes.sizeof(items)))
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)
        self.n_items, self.max_tq, self.max_tr = n, max_tq, max_tr
        lq, hq, d = self.shape
        # sized for the longest window the reserve allows, so appends keep it
        self.ws_bytes = nat.decode_workspace_bytes(n, self.bits, self.group_size, hq, self.kv_heads, d, lq,
                                                   max_tq + self._room, max_tr + self._room)
        if getattr(self, "workspace", None) is None or self.workspace.numel() < self.ws_bytes:
            self.workspace = nat.workspace(self.device, self.ws_bytes)
        self._streams = [streams[id(c)] for c in caches if id(c) in streams]
        if self._streams:
            self._entries = (nat.AppendEntry * len(self._streams))(*(e for _, e, _ in self._streams))
            # the dense segments' lengths are fixed; the windows' longest grows with appends
            self._dense_max_tr = max((int(s[0].shape[0]) for g in self.groups for s in g if isinstance(s, tuple)),
                                     default=0)
            self._stream_max_tr = max(st.tr for _, _, st in self._streams)
        self._guard = _TableGuard(caches, tensors)

    # ------------------------------------------------------------ streaming --
    def _attach_streams(self, caches) -> dict:
        """Streaming state of every packed segment: {id(cache): (cache, append
        entry, _StreamState)}; the item index is filled in by refresh()."""

        from .physical import _StreamState

        streams = {}
        for c in caches:
            if id(c) in streams:
                raise ValueError("Streaming decode needs each packed segment in one group only")
            buf, off = c._residual_slot()
            ids = c.__dict__.get("_ids_capacity")
            if buf is None or ids is None or c.logical_token_ids.data_ptr() != ids.data_ptr():
                raise RuntimeError("Streaming decode: reserve() the packed segments first")
            old = c.__dict__.get("_stream")
            if old is not None and old is not getattr(self, "_owned_states", {}).get(id(c)):
                c._mutated()  # another batch streamed into this cache: its table is now stale
            state = _StreamState(buf, ids, off, c.residual_tokens, c.quantized_tokens)
            c.__dict__["_stream"] = state
            streams[id(c)] = (c, nat.AppendEntry(0, 0, ids.data_ptr()), state)
        self._owned_states = {k: v[2] for k, v in streams.items()}
        return streams

    def reserve(self, tokens: int) -> None:
        """Room for `tokens` more tokens appended to every packed segment (and
        for flushing them) without allocation; rebuilds the item table."""

        caches = [s for g in self.groups for s in g if not isinstance(s, tuple)]
        for c in caches:
            c.reserve(int(tokens))
            if c.logical_token_ids.device != self.device:
                raise RuntimeError("Streaming decode keeps the logical ids on the GPU")
        self._room = int(tokens)
        self.refresh()

    def append(self, keys: torch.Tensor, values: torch.Tensor, logical_token_ids: torch.Tensor, *,
               flush_at: int | None = None, keep: int = 0, stream: int | None = None) -> int:
        """Append n tokens to the residual window of every packed segment, in
        one launch: keys / values [S, n, Hkv, D] contiguous in the windows'
        dtype and logical_token_ids int64 [S, n], all on the batch's GPU, S =
        the packed segments in group order.  Segments whose window then holds
        at least `flush_at` tokens are flushed (all but `keep` of the window,
        in whole groups) into their packed prefix.  Returns the tokens packed,
        summed over the segments.  The segments' residual_key / residual_value
        / logical_token_ids views follow on their next read."""

        self._guard.check("MixedDecodeBatch.append")
        streams = self._streams if self._room > 0 else []
        n = int(keys.shape[1]) if keys.dim() == 4 else -1
        if not streams or n > self._room:
            self.reserve(max(n, 2 * self._room, 256))
            streams = self._streams
        if (keys.shape != values.shape or keys.dim() != 4 or int(keys.shape[0]) != len(streams)
                or tuple(keys.shape[2:]) != (self.kv_heads, self.shape[2])):
            raise ValueError("Streaming decode expects keys / values [packed segments, n, kv_heads, head_dim]")
        if keys.dtype != self.res_dtype or values.dtype != self.res_dtype:
            raise ValueError("Streaming decode: appended tokens must be in the residual dtype")
        if tuple(logical_token_ids.shape) != tuple(keys.shape[:2]) or logical_token_ids.dtype != torch.int64:
            raise ValueError("Streaming decode: logical_token_ids must be int64 [packed segments, n]")
        for t, what in ((keys, "keys"), (values, "values"), (logical_token_ids, "logical_token_ids")):
            if t.device != self.device or not t.is_contiguous():
                raise ValueError(f"Streaming decode: {what} must be contiguous on {self.device}")
        sid = nat.stream(self.device) if stream is None else stream
        nat.call("uc_kivi_residual_append", self.table.data_ptr(), ctypes.addressof(self._entries), len(streams),
                 keys.data_ptr(), values.data_ptr(), logical_token_ids.data_ptr(), n, self.kv_heads,
                 self.shape[2], nat.dtype_code(self.res_dtype), sid)
        for _, _, st in streams:
            st.tr += n
            st.dirty = True
        self._room -= n
        self._stream_max_tr += n
        self.max_tr = max(self._dense_max_tr, self._stream_max_tr)
        if flush_at is None or self._stream_max_tr < int(flush_at):
            return 0
        return self._flush(int(flush_at), int(keep), sid)

    def _flush(self, flush_at: int, keep: int, sid: int) -> int:
        """Flush every window holding >= flush_at tokens (the packing kernels
        write into the reserved packed storage in place), then move the
        device items past the packed rows with one launch."""

        moved = []
        for c, entry, st in self._streams:
            if st.tr < flush_at:
                continue
            count = c.flush_residual(keep)  # reads the pulled views; packs in place
            if count:
                st.tq += count
                st.tr -= count
                st.off += count
                moved.append((c, entry, count))
        if not moved:
            return 0
        adv = (nat.AppendEntry * len(moved))(*(nat.AppendEntry(e.item, count, None) for _, e, count in moved))
        nat.call("uc_kivi_residual_append", self.table.data_ptr(), ctypes.addressof(adv), len(moved), None, None,
                 None, 0, self.kv_heads, self.shape[2], nat.dtype_code(self.res_dtype), sid)
        guard = self._guard
        slot = {id(c): i for i, c in enumerate(guard.caches)}
        for c, _, _ in moved:  # the flushes changed these caches on purpose
            guard.counts[slot[id(c)]] = c.mutation_count
        self.max_tq = max(max(st.tq for _, _, st in self._streams), self.max_tq)
        self._stream_max_tr = max(st.tr for _, _, st in self._streams)
        self.max_tr = max(self._dense_max_tr, self._stream_max_tr)
        return sum(count for _, _, count in moved)

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
