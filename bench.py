"""Benchmark of the packed-KV decode hot path on one MI355X.

Workload: batched decode over 2-bit KIVI-packed KV,
GQA 28/4, head_dim 128, 28 layers, batch 8, 8192 tokens per sequence (8064
packed + 128 bf16 residual), one bf16 query token per sequence per step.
A step is one decode pass over all 28 layers x 8 sequences: a single
uc_kivi_attn_decode_batch launch (split-K partials + LSE combine) over 28
distinct layer buffers (755 MB, more than the 256 MB Infinity Cache).

Prints one JSON line: metric value = algorithmic bytes moved per step / step
time (GB/s), plus the roofline of the decode kernel and a CPU baseline (the
numpy oracle on a bounded sample of the same workload, rank 0, N=1).
"""

from __future__ import annotations

import argparse
import functools
import gc
import itertools
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0

LAYERS, BATCH, TOKENS, HKV, HQ, D = 28, 8, 8192, 4, 28, 128
BITS, GROUP, RESIDUAL = 2, 32, 128

# HBM bytes per step of the default workload from rocprofv3 PMC passes
# (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000 over both decode kernels, the factors
# from a 1 GiB device copy); profiles/decode_batch_c1.md has the commands.
MEASURED_TRAFFIC_BYTES = 773_993_882


def make_kv(tokens, *, seed, device, heads=HKV, head_dim=D):
    """N(0,1) K with 8 random channels per head scaled x10, N(0,1) V (bf16)."""

    g = torch.Generator(device=device).manual_seed(seed)
    key = torch.randn(tokens, heads, head_dim, generator=g, device=device, dtype=torch.float32)
    value = torch.randn(tokens, heads, head_dim, generator=g, device=device, dtype=torch.float32)
    for h in range(heads):
        ch = torch.randperm(head_dim, generator=g, device=device)[:8]
        key[:, h, ch] *= 10.0
    return key.to(torch.bfloat16), value.to(torch.bfloat16)


def build_workload(device, layers=LAYERS, batch=BATCH, tokens=TOKENS):
    from unicache_amd.storage import PackedKIVICache

    caches, queries = [], []
    pack_ms = 0.0
    pack_bytes = 0
    for layer in range(layers):
        for b in range(batch):
            key, value = make_kv(tokens, seed=1000 * layer + b, device=device)
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            cache = PackedKIVICache.from_dense(key, value, logical_token_ids=torch.arange(tokens, device=device),
                                               token_type_id=3, k_bits=BITS, v_bits=BITS, group_size=GROUP,
                                               residual_length=RESIDUAL, backend="cuda")
            stop.record()
            torch.cuda.synchronize()
            pack_ms += start.elapsed_time(stop)
            pack_bytes += key.numel() * 2 * 2 + cache.resident_bytes - cache.logical_token_ids.numel() * 8
            caches.append(cache)
            g = torch.Generator(device=device).manual_seed(7 + 1000 * layer + b)
            queries.append(torch.randn(1, HQ, D, generator=g, device=device).to(torch.bfloat16))
            del key, value
    return caches, queries, pack_ms, pack_bytes


def from_dense_throughput(device, rounds=28):
    """PackedKIVICache.from_dense as the materialisation loop runs it with the
    caching allocator warm (memory of the previous request reused): rounds of
    8 config-1 sequences (8192 tokens, 2-bit, R=128), each round replacing the
    previous round's caches, timed as a whole with HIP events."""

    from unicache_amd.storage import PackedKIVICache

    inputs = [make_kv(TOKENS, seed=27000 + b, device=device) for b in range(BATCH)]
    ids = torch.arange(TOKENS, device=device)

    def one_round():
        return [PackedKIVICache.from_dense(k, v, logical_token_ids=ids, token_type_id=3, k_bits=BITS, v_bits=BITS,
                                           group_size=GROUP, residual_length=RESIDUAL, backend="cuda")
                for k, v in inputs]

    held = one_round()
    nbytes = sum(k.numel() * 2 * 2 + c.resident_bytes - c.logical_token_ids.numel() * 8
                 for (k, _), c in zip(inputs, held))
    for _ in range(3):
        held = one_round()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gc.disable()
    try:
        start.record()
        for _ in range(rounds):
            held = one_round()
        stop.record()
        torch.cuda.synchronize()
    finally:
        gc.enable()
    ms = start.elapsed_time(stop) / rounds
    return nbytes / (ms * 1e-3) / 1e9, ms / BATCH


def pack_throughput(device, steps, tokens=TOKENS, residual=RESIDUAL):
    """uc_kivi_pack of one config-1 sequence (8064 packed tokens, 2-bit, G=32)
    into preallocated native-layout outputs, calls back to back: the C-ABI pack
    path without from_dense's per-cache allocations.  `tokens` / `residual`
    give other lengths (the 32k line of --only-pack)."""

    from unicache_amd.storage.physical import _native_storage, _pack_native_into

    tq = tokens - residual
    nbytes = 2 * tq * HKV * D * 2 + tq * 384
    calls = []
    for s in range(rotation(nbytes)):
        key, value = make_kv(tokens, seed=26000 + s, device=device)
        storage = _native_storage(tq, HKV, D, BITS, BITS, GROUP, device)
        calls.append(functools.partial(_pack_native_into, storage, 0, key[:tq], value[:tq], k_bits=BITS, v_bits=BITS,
                                       group_size=GROUP))
    stream = torch.cuda.current_stream(device)
    ms = time_steps(cycling(calls), steps, 3, stream, settle_ms=ROW_SETTLE_MS)
    return nbytes / (ms * 1e-3) / 1e9, ms


def time_steps(fn, steps, warmup, stream, settle_ms=0.0):
    """Mean ms per call of fn over `steps` calls timed back to back with HIP
    events, after `warmup` untimed calls (and, with settle_ms, after running fn
    for that much GPU time first, so the clocks have ramped up).  Python's
    cyclic garbage collector is paused over the timed calls, so a collection
    pass does not land inside a host-bound line.  It is not run just before
    them: a full collection here idled the GPU for ~45 ms between the clock
    settling and the timed calls, which then ran on re-ramping clocks."""

    if settle_ms:
        settle(fn, stream, settle_ms=settle_ms)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    gc.disable()
    try:
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        stop.record(stream)
        torch.cuda.synchronize()
    finally:
        gc.enable()
    return start.elapsed_time(stop) / steps


# The GPU's clocks ramp up over the first ~20-50 ms of sustained work after an
# idle spell; steps timed before that read 10-20 % slow.  settle() runs the
# step (untimed, before the W warm-up steps) until SETTLE_MS of GPU time has
# passed, so the K timed steps see the clocks a decode loop runs at.
SETTLE_MS = 200.0
# the same for each operator row (h2o_c3, rows): 30 ms of the operator first
ROW_SETTLE_MS = 30.0
# The MI355X's last-level cache holds 256 MB, so an operator timed back to back
# on one set of inputs would read part of them from it.  The HBM lines whose
# working set is smaller cycle through enough distinct input (and output) sets
# to exceed ROTATE_BYTES together, so the timed calls stream from HBM.
ROTATE_BYTES = 512 << 20


def rotation(footprint, cap=64):
    """Distinct sets a line with this many bytes per call cycles through."""

    return max(1, min(cap, -(-ROTATE_BYTES // max(1, int(footprint)))))


def cycling(calls):
    """One callable running calls[0], calls[1], ... in turn."""

    it = itertools.cycle(calls)
    return lambda: next(it)()


def settle(fn, stream, settle_ms=SETTLE_MS, max_steps=20000):
    """Run fn back to back until settle_ms of GPU time has elapsed (checked
    every 16 steps); returns (steps run, GPU ms)."""

    start = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    done, elapsed = 0, 0.0
    while done < max_steps and elapsed < settle_ms:
        for _ in range(16):
            fn()
        done += 16
        mark = torch.cuda.Event(enable_timing=True)
        mark.record(stream)
        mark.synchronize()
        elapsed = start.elapsed_time(mark)
    return done, elapsed


def time_steps_each(fn, steps, warmup, stream):
    """W warm-up steps, then K timed steps with an event after each: returns
    (mean ms per step over the K steps, [ms of each step]).  The mean is
    first-to-last event time / K, the same bracket as time_steps."""

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    gc.disable()
    try:
        events[0].record(stream)
        for i in range(steps):
            fn()
            events[i + 1].record(stream)
        torch.cuda.synchronize()
    finally:
        gc.enable()
    each = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]
    return events[0].elapsed_time(events[-1]) / steps, each


def long_context_decode(device, steps, layers=LAYERS, tokens=32768):
    """Config 4's packed segment as a pure-packed variant: batch 1, 28 layers x
    32768 tokens (32640 packed 2-bit + 128 residual), one decode step = one
    uc_kivi_attn_decode_batch over the 28 layers."""

    from unicache_amd.storage import PackedKIVICache
    from unicache_amd.storage.decode import KiviDecodeBatch

    caches, queries = [], []
    for layer in range(layers):
        key, value = make_kv(tokens, seed=7000 + layer, device=device)
        caches.append(PackedKIVICache.from_dense(key, value, logical_token_ids=torch.arange(tokens, device=device),
                                                 token_type_id=3, k_bits=BITS, v_bits=BITS, group_size=GROUP,
                                                 residual_length=RESIDUAL, backend="cuda"))
        g = torch.Generator(device=device).manual_seed(7500 + layer)
        queries.append(torch.randn(1, HQ, D, generator=g, device=device).to(torch.bfloat16))
        del key, value
    batch = KiviDecodeBatch(caches, queries)
    stream = torch.cuda.current_stream(device)
    sid = stream.cuda_stream
    settle(lambda: batch.run(sid), stream)
    ms = time_steps(lambda: batch.run(sid), steps, max(20, steps), stream)
    gbs = batch.algorithmic_bytes / (ms * 1e-3) / 1e9
    return {
        "workload": f"pure-packed 32k decode: batch 1, {layers} layers x {tokens} tokens "
                    f"({caches[0].quantized_tokens} packed 2-bit + {caches[0].residual_tokens} residual), Lq=1",
        "ms_per_step": round(ms, 5),
        "gbs": round(gbs, 1),
        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "bytes_per_step": batch.algorithmic_bytes,
    }


def editing_attention(device, steps, layers=LAYERS, bits=BITS):
    """Config 2, the whole editing attention of a layer: 1088 queries x 28 heads
    against 2304 keys -- the 1024 source-VAE tokens (896 packed at `bits` + 128
    residual) and the 256 instruction + 1024 ViT bf16 tokens -- in one
    uc_kivi_attn_mq_segments launch (the packed prefix dequantized inside the
    attention kernel, the residual and the two bf16 segments read where they
    lie: the call run_fused_mixed_attention makes); 28 layers of distinct
    caches.  TFLOP/s = 4*Lq*Hq*T*D per layer / time."""

    from unicache_amd import _native as nat
    from unicache_amd.storage import PackedKIVICache

    lq, vae, instr, vit = 1088, 1024, 256, 1024
    calls = []
    for layer in range(layers):
        key, value = make_kv(vae, seed=5000 + layer, device=device)
        cache = PackedKIVICache.from_dense(key, value, logical_token_ids=torch.arange(vae, device=device),
                                           token_type_id=3, k_bits=bits, v_bits=bits, group_size=GROUP,
                                           residual_length=RESIDUAL, backend="cuda")
        ik, iv = make_kv(instr, seed=5100 + layer, device=device)
        tk, tv = make_kv(vit, seed=5200 + layer, device=device)
        g = torch.Generator(device=device).manual_seed(9000 + layer)
        q = torch.randn(lq, HQ, D, generator=g, device=device).to(torch.bfloat16)
        out = torch.empty_like(q)
        lse = torch.empty(HQ, lq, dtype=torch.float32, device=device)
        item = (nat.KiviItem * 1)(cache.native_item(None, None, None, residual_key_ptr=cache.residual_key.data_ptr(),
                                                    residual_value_ptr=cache.residual_value.data_ptr(),
                                                    residual_tokens=cache.residual_tokens))
        dense = (nat.DenseSegment * 2)(
            nat.DenseSegment(ik.data_ptr(), iv.data_ptr(), instr, HKV * D, D),
            nat.DenseSegment(tk.data_ptr(), tv.data_ptr(), vit, HKV * D, D))
        calls.append((item, dense, cache, q, out, lse, ik, iv, tk, tv))
        del key, value
    keys = calls[0][2].quantized_tokens + calls[0][2].residual_tokens + instr + vit
    stream = torch.cuda.current_stream(device)
    sid = stream.cuda_stream
    bf16 = nat.dtype_code(torch.bfloat16)

    def step():
        for item, dense, cache, q, out, lse, *_ in calls:
            nat.call("uc_kivi_attn_mq_segments", item, 1, dense, 2, q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                     bits, GROUP, HQ, HKV, D, lq, bf16, bf16, bf16, 1.0 / math.sqrt(D), sid)

    settle(step, stream)
    ms = time_steps(step, steps, 2, stream)
    flop = 4 * lq * HQ * keys * D
    tflops = flop * layers / (ms * 1e-3) / 1e12
    return {
        "workload": f"config 2 editing attention: Lq=1088 x 28 heads over {keys} keys (VAE {vae} at {bits}-bit: "
                    f"896 packed + 128 residual; instruction {instr} + ViT {vit} bf16), {layers} layers, "
                    f"one uc_kivi_attn_mq_segments launch per layer",
        "ms_per_layer": round(ms / layers, 4),
        "tflops": round(tflops, 1),
        "frac_of_bf16_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4),
        "flop_per_layer": flop,
    }


def h2o_eviction(device, steps):
    """Config 3, one layer: bf16-probability attention mass of 512 queries over
    4096 keys summed per KV head (uc_h2o_scores, MFMA), then per segment
    (256 instruction, 3840 ViT tokens) the 20% budget top-k + recent window and
    the GQA gather into [4, 819, 128] (GQAH2OCache.from_dense), then the
    keep-mask compaction of the dense cache."""

    from unicache_amd.operators.physical import per_kv_head_scores_from_qk
    from unicache_amd.storage import GQAH2OCache
    from unicache_amd.storage.tensor_backend import TensorCacheStorageBackend, h2o_budget

    lq, tokens = 512, 4096
    key, value = make_kv(tokens, seed=3, device=device)
    g = torch.Generator(device=device).manual_seed(33)
    q = torch.randn(lq, HQ, D, generator=g, device=device).to(torch.bfloat16)
    scores = torch.empty(HKV, tokens, dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device)
    # the attention pass before the H2O update yields each row's LSE
    # (run_fused_mixed_attention returns it); the score pass then needs one
    # QK sweep: P = bf16(exp(logit - lse)) summed per KV head
    from unicache_amd.storage.kivi_cuda import dense_attention_summary

    _, lse = dense_attention_summary(q, key, value)
    ms_scores = time_steps(lambda: per_kv_head_scores_from_qk(q, key, out=scores, lse=lse), steps, 2, stream,
                           settle_ms=ROW_SETTLE_MS)
    ms_scores_stats = time_steps(lambda: per_kv_head_scores_from_qk(q, key, out=scores.zero_()), steps, 2, stream,
                                 settle_ms=ROW_SETTLE_MS)
    spans = [(0, 256), (256, 4096)]
    ids = [torch.arange(lo, hi, device=device) for lo, hi in spans]  # the caller's logical token ids

    budgets = [h2o_budget(hi - lo, {"target_budget_ratio": 0.2}) for lo, hi in spans]

    def select_gather():
        # both segments of the layer, as compact_and_materialize builds them:
        # one GQAH2OCache.from_dense_segments call, one launch
        return GQAH2OCache.from_dense_segments([
            dict(key=key[lo:hi], value=value[lo:hi], logical_token_ids=seg_ids, token_type_id=1,
                 per_kv_head_scores=scores[:, lo:hi], target_tokens=target, recent_tokens=recent,
                 selection_frozen=True)
            for (lo, hi), seg_ids, (target, recent) in zip(spans, ids, budgets)])

    ms_sel = time_steps(select_gather, steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    retained = sum(s.retained_tokens for s in select_gather())
    keep = torch.ones(tokens, dtype=torch.bool, device=device)
    keep[:256] = False
    keep[256:4096:2] = False
    lens = torch.tensor([tokens], device=device)
    ms_compact = time_steps(lambda: TensorCacheStorageBackend.compact(
        key=key, value=value, key_type_ids=None, sample_lens=lens, keep_masks=[keep], sample_lengths=[tokens]),
        steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    kept = int(keep.sum())
    flop = 2 * lq * HQ * tokens * D
    gather_bytes = 2 * (2 * HKV * retained * D * 2) + 2 * HKV * retained * (8 + 4) + HKV * tokens * 4
    compact_bytes = 2 * 2 * kept * HKV * D * 2
    return {
        "workload": "config 3, one layer: scores of Lq=512 x 28 heads over 4096 keys given the attention "
                    "pass's LSE (uc_h2o_scores_lse; without it uc_h2o_scores adds a max/sum pass), "
                    f"select + gather of 2 segments to {retained} tokens per head, keep-mask compaction "
                    f"keeping {kept} of {tokens} dense rows",
        "scores_ms": round(ms_scores, 4),
        "scores_tflops": round(flop / (ms_scores * 1e-3) / 1e12, 1),
        "scores_frac_of_bf16_mfma_peak": round(flop / (ms_scores * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
        "scores_without_lse_ms": round(ms_scores_stats, 4),
        "select_gather_ms": round(ms_sel, 4),
        "select_gather_gbs": round(gather_bytes / (ms_sel * 1e-3) / 1e9, 1),
        "compact_ms": round(ms_compact, 4),
        "compact_gbs": round(compact_bytes / (ms_compact * 1e-3) / 1e9, 1),
    }


def mixed_decode(device, steps, layers=LAYERS):
    """Config 4: per layer the VAE segment (20352 tokens:
    20224 packed 2-bit + 128 fp16 residual) and the bf16 tokens kept dense (128
    protected + instruction 4096 -> 819 and ViT 8192 -> 1638 after H2O at a 20%
    budget) attended as one softmax; all 28 layers in one
    uc_kivi_attn_decode_segments launch.

    Two figures: the decode step itself (the static table, timed back to
    back), and the 64-step decode loop of the configuration: each step runs
    the decode launch, then appends one new token to every layer's residual
    window (one uc_kivi_residual_append launch that also moves the device item
    table's lengths), and a window that reaches 160 tokens is flushed -- 128 of
    its tokens quantized into the packed prefix in place -- as the CPU row C4
    does after its 32nd step.  The loop's host time (enqueueing) is reported
    beside its GPU time."""

    from unicache_amd.storage import PackedKIVICache
    from unicache_amd.storage.decode import MixedDecodeBatch

    vae, dense_tokens = 20352, 128 + 819 + 1638
    groups, queries, caches = [], [], []
    for layer in range(layers):
        key, value = make_kv(vae, seed=11000 + layer, device=device)
        cache = PackedKIVICache.from_dense(key.half(), value.half(),
                                           logical_token_ids=torch.arange(vae, device=device), token_type_id=3,
                                           k_bits=BITS, v_bits=BITS, group_size=GROUP, residual_length=RESIDUAL,
                                           backend="cuda")
        dk, dv = make_kv(dense_tokens, seed=12000 + layer, device=device)
        groups.append([cache, (dk.half().contiguous(), dv.half().contiguous())])
        caches.append(cache)
        gq = torch.Generator(device=device).manual_seed(13000 + layer)
        queries.append(torch.randn(1, HQ, D, generator=gq, device=device).to(torch.bfloat16))
        del key, value, dk, dv
    batch = MixedDecodeBatch(groups, queries)
    stream = torch.cuda.current_stream(device)
    sid = stream.cuda_stream
    settle(lambda: batch.run(sid), stream)
    ms = time_steps(lambda: batch.run(sid), steps, max(20, steps), stream)
    step_bytes = batch.algorithmic_bytes
    gbs = step_bytes / (ms * 1e-3) / 1e9
    packed0, window0 = caches[1].quantized_tokens, caches[1].residual_tokens

    # the 64-step loop; the append kernel is loaded by a throwaway one-layer
    # batch first, and the reserve is taken outside the timed loop
    loop_steps, flush_at, keep = 64, 160, 32
    nk, nv = make_kv(loop_steps * layers, seed=14000, device=device)
    new_k = nk.half().view(loop_steps, layers, 1, HKV, D)
    new_v = nv.half().view(loop_steps, layers, 1, HKV, D)
    new_ids = (torch.arange(loop_steps, device=device).view(loop_steps, 1, 1) + vae).expand(
        loop_steps, layers, 1).contiguous()
    spare = PackedKIVICache.from_dense(nk[:256].half(), nv[:256].half(),
                                       logical_token_ids=torch.arange(256, device=device), token_type_id=3,
                                       k_bits=BITS, v_bits=BITS, group_size=GROUP, residual_length=RESIDUAL,
                                       backend="cuda")
    warm = MixedDecodeBatch([[spare]], [queries[0]])
    warm.append(new_k[0, :1], new_v[0, :1], new_ids[0, :1], stream=sid)
    warm.run(sid)
    batch.reserve(loop_steps)
    settle(lambda: batch.run(sid), stream, settle_ms=50.0)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    h0 = time.perf_counter()
    flushed = 0
    for t in range(loop_steps):
        batch.run(sid)
        flushed += batch.append(new_k[t], new_v[t], new_ids[t], flush_at=flush_at, keep=keep, stream=sid)
    h1 = time.perf_counter()
    t1.record(stream)
    torch.cuda.synchronize()
    loop_ms = t0.elapsed_time(t1)
    # attention bytes read over the loop: every step reads each layer's packed
    # prefix (384 B / token), window and dense tokens (2048 B / token), q and out
    # (codes of K and V, then fp16 scale + minimum of K (per channel, over a
    # group of tokens) and of V (per group of channels))
    per_tok_packed = HKV * (2 * D * BITS // 8 + 2 * 2 * D * 2 // GROUP)
    per_tok_dense = HKV * D * 2 * 2
    loop_bytes, tq, tr = 0, packed0, window0
    for t in range(loop_steps):
        loop_bytes += layers * (tq * per_tok_packed + (tr + dense_tokens) * per_tok_dense + 2 * HQ * D * 2)
        tr += 1
        if tr >= flush_at:
            moved = (tr - keep) // GROUP * GROUP
            tq, tr = tq + moved, tr - moved
    assert (tq, tr) == (caches[1].quantized_tokens, caches[1].residual_tokens)
    assert flushed == layers * (tq - packed0)
    return {
        "workload": f"config 4 decode step: {layers} layers x (VAE {vae} tokens: {packed0} packed "
                    f"2-bit + {window0} fp16 residual | {dense_tokens} dense tokens: 128 protected "
                    "+ 819 + 1638 H2O-retained), batch 1, Lq=1, one uc_kivi_attn_decode_segments launch",
        "ms_per_step": round(ms, 5),
        "gbs": round(gbs, 1),
        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "bytes_per_step": step_bytes,
        "loop_64": {
            "workload": f"configs[4] decode loop: {loop_steps} steps x {layers} layers; per step the decode "
                        "launch, then one token appended to every layer's window (one uc_kivi_residual_append "
                        f"launch), a window reaching {flush_at} tokens flushed ({flush_at - keep} tokens packed "
                        "in place), as the CPU row C4",
            "gpu_ms_per_step": round(loop_ms / loop_steps, 5),
            "host_us_per_step": round((h1 - h0) * 1e6 / loop_steps, 1),
            "attention_gbs": round(loop_bytes / (loop_ms * 1e-3) / 1e9, 1),
            "flushed_tokens_per_layer": tq - packed0,
        },
    }


def _hbm_line(workload, ms, nbytes, **extra):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": workload, "ms": round(ms, 5), "bytes": int(nbytes), "gbs": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), **extra}


def secondary_rows(device, steps):
    """The remaining operators of the path, each at a configuration's shapes,
    timed with HIP events on the current stream; bytes are the algorithmic
    reads + writes (each tensor once)."""

    from unicache_amd.adapters.bagel import merge_attention_summaries
    from unicache_amd.operators.builtin import kivi_fake_quant_key, kivi_fake_quant_value
    from unicache_amd.storage import GQAH2OCache, PackedKIVICache
    from unicache_amd.storage.kivi_cuda import dequantize_kivi_chunk, packed_kivi_attention_parts
    from unicache_amd.storage.physical import gqa_probability_value, gqa_query_key_logits

    stream = torch.cuda.current_stream(device)
    rows = {}

    # fake quantization (operators/builtin.py:31-65): K over 32-token groups, V over
    # 32-channel groups, bf16 in and out
    def fake_quant(k, v):
        return kivi_fake_quant_key(k, bits=BITS, group_size=GROUP), kivi_fake_quant_value(v, bits=BITS,
                                                                                          group_size=GROUP)

    for tokens, label in ((2048, "config 0"), (32768, "32k tokens")):
        nbytes = 2 * 2 * tokens * HKV * D * 2
        sets = [make_kv(tokens, seed=21000 + tokens + s, device=device) for s in range(rotation(nbytes))]
        ms = time_steps(cycling([functools.partial(fake_quant, k, v) for k, v in sets]), steps, 2, stream,
                        settle_ms=ROW_SETTLE_MS)
        rows[f"fake_quant_{tokens}"] = _hbm_line(
            f"{label}: kivi_fake_quant_key + kivi_fake_quant_value on [{tokens}, 4, 128] bf16, 2-bit, G=32 "
            f"({len(sets)} input sets in turn)", ms, nbytes)
        del sets

    # the fake-quant segment operator (operators/builtin.py:281-476) at config 0:
    # a 2048-token segment, the last 128 tokens and 16 protected ones kept
    from types import SimpleNamespace

    from unicache_amd.core.registry import OperatorExecutionContext
    from unicache_amd.operators import KIVIQuantizationOperator

    k0, v0 = make_kv(2048, seed=21900, device=device)
    seg = torch.ones(2048, dtype=torch.bool, device=device)
    prot = torch.zeros(2048, dtype=torch.bool, device=device)
    prot[:16] = True
    op = KIVIQuantizationOperator()
    params = op.build_params({"bits": BITS, "group_size": GROUP, "residual_length": RESIDUAL})

    def fq_operator():
        ctx = OperatorExecutionContext(runtime=SimpleNamespace(kv_metadata={}), step=SimpleNamespace(segment_id=0),
                                       params=params, q=None, k=k0, v=v0, attn_mask=None, key_type_ids=None,
                                       segment_mask=seg, protected_mask=prot, state={}, record=lambda r: None,
                                       set_storage_snapshot=lambda r: None, storage_num_kv_heads=HKV)
        return op.execute(ctx)

    ms = time_steps(fq_operator, steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    rows["fake_quant_operator_c0"] = _hbm_line(
        "config 0: KIVIQuantizationOperator.execute on a 2048-token segment (last 128 and 16 protected tokens "
        "kept), 2-bit, G=32: masks, row gather, fake quant, write-back into copies of K and V",
        ms, 2 * (2048 * HKV * D * 2 * 2 + 1904 * HKV * D * 2 * 2))

    # native pack (kivi_cuda.py:157-190) of a 32k-token K/V in one call
    from unicache_amd.storage.kivi_cuda import quantize_kivi_native

    nbytes = 2 * 32768 * HKV * D * 2 + 32768 * 384
    sets = [make_kv(32768, seed=21500 + s, device=device) for s in range(rotation(nbytes))]
    ms = time_steps(cycling([functools.partial(quantize_kivi_native, k, v, k_bits=BITS, v_bits=BITS, group_size=GROUP)
                             for k, v in sets]), steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    rows["pack_32k"] = _hbm_line(
        "quantize_kivi_native of [32768, 4, 128] bf16 K and V, 2-bit, G=32 (codes + fp16 stats out; "
        f"{len(sets)} input sets in turn)", ms, nbytes)
    del sets

    # chunked dequantization (kivi_cuda.py:58-93) of a 32k-token packed cache
    tokens = 32768
    tq = tokens - RESIDUAL
    nbytes = tq * 384 + 2 * tq * HKV * D * 2
    calls = []
    for s in range(rotation(nbytes)):
        k, v = make_kv(tokens, seed=22000 + s, device=device)
        cache = PackedKIVICache.from_dense(k, v, logical_token_ids=torch.arange(tokens, device=device),
                                           token_type_id=3, k_bits=BITS, v_bits=BITS, group_size=GROUP,
                                           residual_length=RESIDUAL, backend="cuda")
        assert cache.quantized_tokens == tq
        out_k = torch.empty(tq, HKV, D, dtype=torch.bfloat16, device=device)
        calls.append(functools.partial(dequantize_kivi_chunk, cache, start=0, stop=tq, dtype=torch.bfloat16,
                                       output_key=out_k, output_value=torch.empty_like(out_k)))
        del k, v
    ms = time_steps(cycling(calls), steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    rows["dequantize_chunk_32k"] = _hbm_line(
        f"dequantize_kivi_chunk of {tq} packed 2-bit tokens into bf16 K/V workspaces (GQA 4 x 128; "
        f"{len(calls)} caches in turn)", ms, nbytes)
    del calls

    # packed attention parts (kivi_cuda.py:238-329): logits then P.V at config 0
    tokens = 2048
    k, v = make_kv(tokens, seed=23000, device=device)
    c0 = PackedKIVICache.from_dense(k, v, logical_token_ids=torch.arange(tokens, device=device), token_type_id=3,
                                    k_bits=BITS, v_bits=BITS, group_size=GROUP, residual_length=RESIDUAL,
                                    backend="cuda")
    q1 = torch.randn(1, HQ, D, device=device).to(torch.bfloat16)

    def parts():
        logits, apply_value = packed_kivi_attention_parts(c0, q1)
        return apply_value(torch.softmax(logits, -1))

    ms = time_steps(parts, steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    t_all = c0.quantized_tokens + c0.residual_tokens
    rows["attention_parts_c0"] = _hbm_line(
        f"config 0: packed_kivi_attention_parts ({c0.quantized_tokens} packed + {c0.residual_tokens} residual, "
        "Lq=1) + torch softmax + the AV closure",
        ms, 2 * (c0.quantized_tokens * 384 // 2 + c0.residual_tokens * 1024) + 2 * HQ * t_all * 4 * 2)

    # GQA logits and P.V over dense keys (physical.py:20-63) at config 3's shapes
    lq, tokens = 512, 4096
    k, v = make_kv(tokens, seed=24000, device=device)
    q = torch.randn(lq, HQ, D, device=device).to(torch.bfloat16)
    ms = time_steps(lambda: gqa_query_key_logits(q, k), max(3, steps // 4), 1, stream, settle_ms=ROW_SETTLE_MS)
    rows["gqa_logits_c3"] = _hbm_line(
        "config 3 shapes: gqa_query_key_logits, q [512, 28, 128] bf16 x k [4096, 4, 128] -> fp32 [28, 512, 4096]",
        ms, q.numel() * 2 + k.numel() * 2 + HQ * lq * tokens * 4,
        tflops=round(2 * lq * HQ * tokens * D / (ms * 1e-3) / 1e12, 1))
    p_bytes = HQ * lq * tokens * 2
    prob_sets = []
    for s in range(rotation(p_bytes)):
        qs = q if s == 0 else torch.randn(lq, HQ, D, device=device).to(torch.bfloat16)
        prob_sets.append(torch.softmax(gqa_query_key_logits(qs, k) / math.sqrt(D), -1).to(torch.bfloat16))
    probs = prob_sets[0]
    ms = time_steps(cycling([functools.partial(gqa_probability_value, p, v) for p in prob_sets]), max(3, steps // 4),
                    1, stream, settle_ms=ROW_SETTLE_MS)
    rows["gqa_pv_c3"] = _hbm_line(
        "config 3 shapes: gqa_probability_value, p [28, 512, 4096] bf16 x v [4096, 4, 128] -> [28, 512, 128] "
        f"({len(prob_sets)} probability sets in turn)",
        ms, probs.numel() * 2 + v.numel() * 2 + HQ * lq * D * 2,
        tflops=round(2 * lq * HQ * tokens * D / (ms * 1e-3) / 1e12, 1))

    # H2O score update from materialised probabilities (physical.py:598-610)
    seg = GQAH2OCache.from_dense(k, v, logical_token_ids=torch.arange(tokens, device=device), token_type_id=1,
                                 per_kv_head_scores=torch.rand(HKV, tokens, device=device), target_tokens=tokens,
                                 recent_tokens=0, selection_frozen=True)
    ms = time_steps(cycling([functools.partial(seg.update_scores, p) for p in prob_sets]), steps, 2, stream,
                    settle_ms=ROW_SETTLE_MS)
    rows["h2o_update_scores_c3"] = _hbm_line(
        "config 3 shapes: GQAH2OCache.update_scores, bf16 probabilities [28, 512, 4096] summed per KV head "
        f"({len(prob_sets)} probability sets in turn)",
        ms, probs.numel() * 2 + 2 * HKV * tokens * 4)
    del probs, prob_sets

    # batched physical attention (adapters/bagel.py:773-980): three CFG samples of
    # config 2's queries over the packed VAE segment plus their own bf16 keys
    from unicache_amd.adapters import run_batched_physical_attention

    lq, vae, current = 1088, 1024, (1280, 1024, 256)
    vk, vv = make_kv(vae, seed=25000, device=device)
    vae_cache = PackedKIVICache.from_dense(vk, vv, logical_token_ids=torch.arange(vae, device=device),
                                           token_type_id=3, k_bits=BITS, v_bits=BITS, group_size=GROUP,
                                           residual_length=RESIDUAL, backend="cuda")
    ck, cv = make_kv(sum(current), seed=25001, device=device)
    cq = torch.randn(3 * lq, HQ, D, device=device).to(torch.bfloat16)
    cu_q = torch.tensor([0, lq, 2 * lq, 3 * lq], dtype=torch.int32)
    cu_k = torch.tensor([0, current[0], current[0] + current[1], sum(current)], dtype=torch.int32)
    ms = time_steps(lambda: run_batched_physical_attention(cq, ck, cv, cu_q, cu_k, [[vae_cache]] * 3), steps, 2,
                    stream, settle_ms=ROW_SETTLE_MS)
    flop = sum(4 * lq * HQ * (vae + c) * D for c in current)
    rows["batched_cfg_c2"] = {
        "workload": "three CFG samples of config 2 (1088 queries x 28 heads each) over the 2-bit VAE segment "
                    "(896 packed + 128 residual) plus 1280 / 1024 / 256 current bf16 keys: "
                    "run_batched_physical_attention: one segment-table attention launch for the three samples "
                    "(uc_kivi_attn_mq_table), host-side preparation included",
        "ms": round(ms, 5), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
        "frac_of_bf16_mfma_peak": round(flop / (ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4)}

    # LSE merge of config 2's three segment summaries (adapters/bagel.py:57-72)
    lq = 1088
    summaries = [(torch.randn(lq, HQ, D, device=device).to(torch.bfloat16), torch.randn(HQ, lq, device=device))
                 for _ in range(3)]
    ms = time_steps(lambda: merge_attention_summaries(summaries), steps, 2, stream, settle_ms=ROW_SETTLE_MS)
    rows["lse_merge_c2"] = _hbm_line(
        "config 2: merge_attention_summaries of 3 segment summaries ([1088, 28, 128] bf16 + LSE [28, 1088])",
        ms, (3 + 1) * (lq * HQ * D * 2 + HQ * lq * 4))
    return rows


def _host_cores():
    """(threads, CPU model): the cores this process may use (affinity and a
    cgroup CPU quota both bound it) and /proc/cpuinfo's model name."""

    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return n, model


def _median_ms(fn, runs=5):
    fn()  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return sorted(times)[len(times) // 2]


def cpu_baseline(c1_layer_bytes, c4_layer_bytes):
    """the torch-CPU restatement of the path
    (oracle/torch_cpu.py) timed on this host's cores, 1 warm-up and the
    median of 5 runs per row, at each configuration's shapes.  Whole-step
    figures for 28 layers are per-layer times x 28 (marked extrapolated)."""

    from oracle import torch_cpu as T

    threads, model = _host_cores()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)

    def kv(tokens):
        key = torch.randn(tokens, HKV, D, generator=g)
        for h in range(HKV):
            key[:, h, torch.randperm(D, generator=g)[:8]] *= 10.0
        return key.to(torch.bfloat16), torch.randn(tokens, HKV, D, generator=g).to(torch.bfloat16)

    def q(lq):
        return torch.randn(lq, HQ, D, generator=g).to(torch.bfloat16)

    rows = {}
    try:
        # C0: pack 2048 tokens (R=128), then one decode over packed + residual
        k0, v0 = kv(2048)
        rows["c0_pack_ms"] = _median_ms(lambda: T.from_dense(k0, v0, bits=BITS, group_size=GROUP,
                                                             residual_length=RESIDUAL))
        s0, q0 = T.from_dense(k0, v0, bits=BITS, group_size=GROUP, residual_length=RESIDUAL), q(1)
        rows["c0_decode_ms"] = _median_ms(lambda: T.packed_decode(s0, q0))
        # C1: one layer = 8 sequences of 8064 packed + 128 residual tokens, Lq=1
        segs = [T.from_dense(*kv(TOKENS), bits=BITS, group_size=GROUP, residual_length=RESIDUAL)
                for _ in range(BATCH)]
        qs = [q(1) for _ in range(BATCH)]
        c1 = _median_ms(lambda: [T.packed_decode(s, x) for s, x in zip(segs, qs)])
        rows["c1_layer_ms"] = c1
        rows["c1_all_layers_ms_extrapolated"] = c1 * LAYERS
        rows["c1_gbs"] = c1_layer_bytes / (c1 * 1e-3) / 1e9
        del segs
        # C2: one layer of the editing pass, 1088 queries over the 2-bit VAE
        # segment (896 packed + 128 residual) and 1280 bf16 tokens
        s2 = T.from_dense(*kv(1024), bits=BITS, group_size=GROUP, residual_length=RESIDUAL)
        dk, dv = kv(1280)
        q2 = q(1088)

        def editing():
            pk, pv = T.dequantize(s2)
            return T.attention_summary(q2, torch.cat([dk, pk]), torch.cat([dv, pv]))

        c2 = _median_ms(editing)
        rows["c2_layer_ms"] = c2
        rows["c2_all_layers_ms_extrapolated"] = c2 * LAYERS
        rows["c2_gflops"] = 4 * 1088 * HQ * 2304 * D / (c2 * 1e-3) / 1e9
        # C3: H2O scores of 512 queries over 4096 keys; top-k + gather of the
        # instruction (256 -> 51) and ViT (3840 -> 768) history at 20 %
        k3, v3 = kv(4096)
        q3 = q(512)
        rows["c3_scores_ms"] = _median_ms(lambda: T.h2o_scores(q3, k3))
        sc = T.h2o_scores(q3, k3)

        def select_gather():
            for lo, hi in ((0, 256), (256, 4096)):
                n = hi - lo
                target = max(1, int(round(n * 0.2)))
                recent = int(round(target * 0.25))
                T.h2o_select_gather(sc[:, lo:hi], k3[lo:hi], v3[lo:hi], heavy_k=target - recent, recent=recent)

        rows["c3_topk_gather_ms"] = _median_ms(select_gather)
        # C4: 64 decode steps of one layer over the VAE segment (20224 packed
        # + 128 residual) and 2585 dense tokens, each appending one token to
        # the residual; after step 32 one 128-token flush packs its head
        s4 = T.from_dense(*kv(20352), bits=BITS, group_size=GROUP, residual_length=RESIDUAL)
        dk4, dv4 = kv(2585)
        nk, nv = kv(64)
        q4 = q(1)

        def steps64():
            seg = dict(s4)
            for t in range(64):
                pk, pv = T.dequantize(seg)
                T.attention_summary(q4, torch.cat([pk, dk4]), torch.cat([pv, dv4]))
                seg["residual_key"] = torch.cat([seg["residual_key"], nk[t:t + 1]])
                seg["residual_value"] = torch.cat([seg["residual_value"], nv[t:t + 1]])
                if t == 31:
                    seg = T.flush(seg, 128)

        c4 = _median_ms(steps64) / 64
        rows["c4_step_layer_ms"] = c4
        rows["c4_step_all_layers_ms_extrapolated"] = c4 * LAYERS
        rows["c4_gbs"] = c4_layer_bytes / (c4 * 1e-3) / 1e9
    finally:
        torch.set_num_threads(prev)
    rows = {k: round(v, 4) for k, v in rows.items()}
    return {
        "value": rows["c1_gbs"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": model,
        "sample": "oracle/torch_cpu.py (torch-CPU restatement: dequantize + fp32 GQA attention with bf16 "
                  "probabilities) on one config-1 layer (8 sequences x 8064 packed 2-bit + 128 bf16 tokens, "
                  f"Lq=1), {threads} threads, median of 5 after 1 warm-up; value = the layer's algorithmic "
                  "bytes / its time.  rows: C0-C4 at their shapes, 28-layer figures extrapolated x28",
        "rows": rows,
    }


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=100)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--layers", type=int, default=LAYERS)
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="only run a 1 GiB device copy (PMC traffic calibration)")
    parser.add_argument("--only-decode", action="store_true",
                        help="only build the config-1 workload and run its decode step (for counter passes)")
    parser.add_argument("--only-editing", type=int, choices=(2, 4), default=None,
                        help="only run the config-2 editing attention at this bit width (for counter passes)")
    parser.add_argument("--only-h2o", action="store_true",
                        help="only run the config-3 H2O line (for counter passes)")
    parser.add_argument("--only-pack", action="store_true",
                        help="only run the pack lines (for counter passes)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decode hot path shards by sequence / KV head with no "
              "exchange, and this build runs on a single MI355X (use --gpus 1)", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": 1 << 30}))
        return

    if args.only_editing:
        print(json.dumps(editing_attention(device, args.steps, layers=args.layers, bits=args.only_editing)))
        return
    if args.only_h2o:
        print(json.dumps(h2o_eviction(device, args.steps)))
        return
    if args.only_pack:
        gbs, ms = pack_throughput(device, args.steps)
        gbs32, ms32 = pack_throughput(device, args.steps, tokens=32768, residual=0)
        print(json.dumps({"pack_gbs": round(gbs, 2), "pack_ms_per_sequence": round(ms, 5),
                          "pack_32k_into_gbs": round(gbs32, 2), "pack_32k_into_ms": round(ms32, 5)}))
        return

    from unicache_amd.storage.decode import KiviDecodeBatch

    caches, queries, pack_ms, pack_bytes = build_workload(device, layers=args.layers)
    batch = KiviDecodeBatch(caches, queries)
    stream = torch.cuda.current_stream(device)
    sid = stream.cuda_stream
    run = lambda: batch.run(sid)  # noqa: E731
    settle_steps, settle_ms = settle(run, stream)
    ms, step_ms = time_steps_each(run, args.steps, args.warmup, stream)
    if args.only_decode:
        print(json.dumps({"config1_decode_ms": round(ms, 5),
                          "gbs": round(batch.algorithmic_bytes / (ms * 1e-3) / 1e9, 2)}))
        return
    step_bytes = batch.algorithmic_bytes
    value = step_bytes / (ms * 1e-3) / 1e9

    # per-layer launches (28 launches of 8 sequences each) for comparison
    per_layer = [KiviDecodeBatch(caches[i * BATCH:(i + 1) * BATCH], queries[i * BATCH:(i + 1) * BATCH])
                 for i in range(args.layers)]
    ms_layers = time_steps(lambda: [p.run(sid) for p in per_layer], max(5, args.steps // 5), 2, stream)

    seq_layer_bytes = step_bytes // (args.layers * BATCH)
    result = {
        "metric": "packed-KV decode attention GB/s (2-bit KIVI, config 1: 28 layers x batch 8 x 8192 ctx)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u2 codes + fp16 stats, bf16 q/residual, fp32 accumulate",
        "data": "synthetic (seeded N(0,1), 8 K outlier channels x10 per head)",
        "config": {
            "workload": "config 1: batched decode, 2-bit packed KV, GQA 28/4, head_dim 128, "
                        f"{args.layers} layers, batch {BATCH}, 8192 tokens (8064 packed + 128 residual), Lq=1",
            "layers": args.layers, "batch": BATCH, "context": TOKENS, "bits": BITS, "group_size": GROUP,
            "residual": RESIDUAL,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": MEASURED_TRAFFIC_BYTES if args.layers == LAYERS else None,
            "kernel": "uc_kivi_attn_decode_batch = decode_mfma_kernel + decode_mfma_combine, one call per step",
            "bytes_per_launch": step_bytes,
        },
        "per_layer_launches_gbs": round(step_bytes / (ms_layers * 1e-3) / 1e9, 2),
        # untimed clock settling before the W warm-up steps, and each timed
        # step's own event time (their mean is ms_per_step)
        "clock_settle": {"steps": settle_steps, "gpu_ms": round(settle_ms, 1)},
        "step_ms": [round(t, 5) for t in step_ms],
    }
    pack_gbs, pack_call_ms = pack_throughput(device, max(20, args.steps))
    result["pack_gbs"] = round(pack_gbs, 2)
    result["pack_ms_per_sequence"] = round(pack_call_ms, 5)
    # from_dense in a materialisation loop with the allocator warm, and (cold)
    # the 224 first-time builds above, each paying for new device memory
    fd_gbs, fd_ms = from_dense_throughput(device)
    result["pack_from_dense_gbs"] = round(fd_gbs, 2)
    result["pack_from_dense_ms_per_sequence"] = round(fd_ms, 5)
    result["pack_from_dense_cold_gbs"] = round(pack_bytes / (pack_ms * 1e-3) / 1e9, 2)
    del batch, per_layer, caches, queries
    torch.cuda.empty_cache()
    result["decode_32k"] = long_context_decode(device, max(5, args.steps // 2))
    torch.cuda.empty_cache()
    result["mixed_decode_c4"] = mixed_decode(device, max(5, args.steps // 2))
    torch.cuda.empty_cache()
    result["editing_c2"] = {f"{b}bit": editing_attention(device, max(3, args.steps // 5), bits=b) for b in (2, 4)}
    torch.cuda.empty_cache()
    result["h2o_c3"] = h2o_eviction(device, max(5, args.steps // 5))
    torch.cuda.empty_cache()
    result["rows"] = secondary_rows(device, max(5, args.steps // 5))
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(seq_layer_bytes * BATCH,
                                              result["mixed_decode_c4"]["bytes_per_step"] // LAYERS)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
