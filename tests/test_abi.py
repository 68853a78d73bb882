"""The C-ABI library loads on a machine without a GPU and exports every
entry point declared in include/unicache_hip.h; argument validation runs on
the host before any launch."""

import ctypes
import os
import re
import subprocess

import pytest

from unicache_amd import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "unicache_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(uc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert declared_functions() == nat.exported_symbols()


def test_library_exports_every_declared_symbol():
    lib = nat.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", nat.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (uc_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported


def test_abi_version_and_error_state():
    lib = nat.load_library()
    assert lib.uc_abi_version() == nat.ABI_VERSION
    rc = lib.uc_kivi_pack(None, 0, 0, 0, None, 0, 0, 0, nat.UC_BF16, 64, 4, 128, 3, 2, 32, nat.UC_FP16,
                          None, 0, 0, 0, None, None, 0, 0, 0, None, 0, 0, 0, None, None, 0, 0, 0, None)
    assert rc == nat.UC_EINVAL
    assert b"2, 4, or 8" in lib.uc_last_error()
    with pytest.raises(ValueError, match="group_size"):
        nat.call("uc_kivi_pack", None, 0, 0, 0, None, 0, 0, 0, nat.UC_BF16, 64, 4, 128, 2, 2, 48, nat.UC_FP16,
                 None, 0, 0, 0, None, None, 0, 0, 0, None, 0, 0, 0, None, None, 0, 0, 0, None)
    with pytest.raises(ValueError, match="multiple of group_size"):
        nat.call("uc_kivi_pack", None, 0, 0, 0, None, 0, 0, 0, nat.UC_BF16, 70, 4, 128, 2, 2, 32, nat.UC_FP16,
                 None, 0, 0, 0, None, None, 0, 0, 0, None, 0, 0, 0, None, None, 0, 0, 0, None)


def test_select_rejects_oversized_window():
    with pytest.raises(ValueError, match="exceeds"):
        nat.call("uc_h2o_select", None, 10, 1, 4, 10, 8, 3, None, None)


def test_decode_validation():
    item = nat.KiviItem()
    item.quantized_tokens = 64
    with pytest.raises(ValueError, match="<= 16"):
        nat.call("uc_kivi_attn_decode", ctypes.byref(item), 2, 32, 28, 4, 128, 3, nat.UC_BF16, nat.UC_BF16,
                 nat.UC_BF16, 0.1, None, 0, None)
    with pytest.raises(ValueError, match="workspace"):
        nat.call("uc_kivi_attn_decode", ctypes.byref(item), 2, 32, 28, 4, 128, 1, nat.UC_BF16, nat.UC_BF16,
                 nat.UC_BF16, 0.1, None, 0, None)


def test_workspace_bytes():
    # AV: per (q head, row, split) D + 2 floats; splits = ceil(T/512) + 1
    # decode-like AV (28 x 1 query rows) splits every 64 keys: 8192 / 64 + 1 splits
    assert nat.workspace_bytes(nat.UC_OP_KIVI_AV, 1, 28, 1, 128, 8192) == 28 * 1 * 129 * 130 * 4
    # longer calls split every 512 keys and also fit V^T staged for the MFMA path
    assert nat.workspace_bytes(nat.UC_OP_KIVI_AV, 1, 28, 512, 128, 4096) == max(28 * 512 * 9 * 130 * 4,
                                                                               28 * 128 * 4096 * 2)
    # MFMA decode (head_dim 128, 2-bit): per (item, KV head, split) 16x128 fp16 + 16x2 fp32;
    # MFMA path: packed splits of 8 super-tiles of 256 tokens (2-bit), residual splits of
    # 2 waves x 128 tokens: 8064 packed tokens -> 4 splits, 128 residual tokens -> 1 split
    splits = -(-8064 // (4 * 2 * 256)) + 1
    assert nat.decode_workspace_bytes(2, 2, 32, 28, 4, 128, 1, 8064, 128) == 2 * 4 * splits * (16 * 128 * 2 + 16 * 2 * 4)
    # other shapes: generic split-K, per (item, q head, row, split) D + 2 floats
    assert nat.decode_workspace_bytes(1, 2, 32, 28, 4, 64, 1, 1024, 0) == 28 * 2 * 66 * 4
    # MFMA score path: (max, sum) per (row block of 256, key chunk, row), at most
    # (blocks + 768) * 256 of them, then one fp32 partial per (row block, KV head,
    # key), with at most ceil(Hq * Lq / 256) + Hq row blocks; this also covers the
    # generic path's (max, sum) per (query head, row)
    blocks = -(-28 * 512 // 256) + 28
    assert nat.workspace_bytes(nat.UC_OP_H2O_SCORES, 1, 28, 512, 128, 4096) == (
        (blocks + 768) * 256 * 8 + blocks * 4096 * 4)
    with pytest.raises(ValueError):
        nat.workspace_bytes(99, 1, 1, 1, 1, 1)


def test_editing_validation():
    item = nat.KiviItem()
    item.quantized_tokens = 64
    args = (28, 4, 128, 512, nat.UC_BF16, nat.UC_BF16, nat.UC_BF16, 0.1, None, 0, None)
    with pytest.raises(ValueError, match="bits must be 2 or 4"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 3, 32, *args)
    with pytest.raises(ValueError, match="group_size must be 32, 64 or 128"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 2, 16, *args)
    with pytest.raises(ValueError, match="head_dim must be 128"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 2, 32, 28, 4, 64, 512, nat.UC_BF16, nat.UC_BF16,
                 nat.UC_BF16, 0.1, None, 0, None)
    with pytest.raises(ValueError, match="multiple of KV heads"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 2, 32, 28, 3, 128, 512, nat.UC_BF16, nat.UC_BF16,
                 nat.UC_BF16, 0.1, None, 0, None)
    # the multi-query kernel dequantizes inside the attention pass: no workspace
    assert nat.mq_workspace_bytes(4, 128, 64, 128) == 0
    assert nat.mq_workspace_bytes(4, 128, 0, 128) == 0
    with pytest.raises(ValueError):
        nat.mq_workspace_bytes(0, 128, 64, 128)
    # aligned placeholders (never dereferenced on the host); each case below
    # breaks one check, so no call reaches a launch
    item.residual_tokens = 128
    for name in ("query", "out", "residual_key", "residual_value", "key_code", "key_scale", "key_min",
                 "value_code", "value_scale", "value_min"):
        setattr(item, name, 0x1000)
    item.out = 0x1008
    with pytest.raises(ValueError, match="16-byte aligned"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 2, 32, *args)
    item.out = 0x1000
    item.residual_value = 0x1004
    with pytest.raises(ValueError, match="dense keys and values must be 16-byte aligned"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 2, 32, *args)
    item.residual_value = 0x1000
    with pytest.raises(ValueError, match="sm_scale must be positive"):
        nat.call("uc_kivi_attn_mq", ctypes.byref(item), 2, 32, 28, 4, 128, 512, nat.UC_BF16, nat.UC_BF16,
                 nat.UC_BF16, 0.0, None, 0, None)


def test_merge_and_fake_quant_validation():
    with pytest.raises(ValueError, match="At least one attention summary"):
        nat.call("uc_lse_merge", None, None, 0, nat.UC_BF16, 4, 28, 128, None, None, None)
    with pytest.raises(ValueError, match="at most 16 segments"):
        nat.call("uc_lse_merge", None, None, 17, nat.UC_BF16, 4, 28, 128, None, None, None)
    with pytest.raises(ValueError, match="Unsupported fake quant bits: 5"):
        nat.call("uc_kivi_fake_quant", None, 512, 128, 1, nat.UC_BF16, 4, 4, 128, 5, 0, 32, None, None)
    with pytest.raises(ValueError, match="dim must be 0"):
        nat.call("uc_kivi_fake_quant", None, 512, 128, 1, nat.UC_BF16, 4, 4, 128, 2, 1, 32, None, None)
    with pytest.raises(ValueError, match="divisible by KV heads for GQA H2O"):
        nat.call("uc_h2o_colsum", None, nat.UC_BF16, 0, 0, 1, 28, 1, 64, 3, 0, None, None)
    with pytest.raises(ValueError, match="divisible by KIVI KV heads"):
        nat.call("uc_kivi_qk", None, nat.UC_BF16, 1, 28, None, None, None, nat.UC_FP16, 0, 0, 2, 32,
                 None, nat.UC_BF16, 16, 0, 0, 3, 128, 0.1, None, None)
    with pytest.raises(ValueError, match="packed_capacity must be 0 or a multiple of group_size"):
        nat.call("uc_kivi_qk", None, nat.UC_BF16, 1, 28, None, None, None, nat.UC_FP16, 64, 48, 2, 32,
                 None, nat.UC_BF16, 16, 0, 0, 4, 128, 0.1, None, None)


def test_editing_batch_validation():
    items = (nat.KiviItem * 9)()
    lens = (ctypes.c_int64 * 9)(*([512] * 9))
    tail = (2, 32, 28, 4, 128, nat.UC_BF16, nat.UC_BF16, nat.UC_BF16, 0.1, None, 0, None)
    with pytest.raises(ValueError, match="n_items must be 1..8"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 0, *tail)
    with pytest.raises(ValueError, match="n_items must be 1..8"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 9, *tail)
    with pytest.raises(ValueError, match="query/out are NULL"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 2, *tail)
    for it in items[:2]:
        it.query = it.out = 0x1000
    with pytest.raises(ValueError, match="empty segment"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 2, *tail)
    # aligned placeholders (never dereferenced on the host); each case below
    # breaks one check, so no call reaches a launch
    for it in items[:2]:
        it.residual_tokens = 100
        it.quantized_tokens = 64
        for name in ("query", "out", "residual_key", "residual_value", "key_code", "key_scale", "key_min",
                     "value_code", "value_scale", "value_min"):
            setattr(it, name, 0x1000)
    items[1].residual_key = 0x1008
    with pytest.raises(ValueError, match="16-byte aligned"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 2, *tail)
    items[1].residual_key = 0x1000
    items[1].quantized_tokens = 48
    with pytest.raises(ValueError, match="multiple of group_size"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 2, *tail)
    items[1].quantized_tokens = 64
    lens[1] = 0
    with pytest.raises(ValueError, match="query_len must be positive"):
        nat.call("uc_kivi_attn_mq_batch", items, lens, 2, *tail)


def test_editing_segments_validation():
    q = 0x1000
    packed = (nat.KiviItem * 9)()
    for it in packed:
        it.quantized_tokens = 64
        for name in ("key_code", "key_scale", "key_min", "value_code", "value_scale", "value_min"):
            setattr(it, name, 0x2000)
    dense = (nat.DenseSegment * 17)()
    for d in dense:
        d.key, d.value, d.tokens, d.token_stride, d.head_stride = 0x3000, 0x3000, 100, 512, 128
    tail = (2, 32, 28, 4, 128, 512, nat.UC_BF16, nat.UC_BF16, nat.UC_BF16, 0.1, None)

    def call(n_packed, n_dense, query=q):
        nat.call("uc_kivi_attn_mq_segments", packed, n_packed, dense, n_dense, query, q, None, *tail)

    with pytest.raises(ValueError, match="more than 8 packed segments"):
        call(9, 0)
    with pytest.raises(ValueError, match="more than 16 dense segments"):
        call(1, 17)
    with pytest.raises(ValueError, match="16-byte aligned"):
        call(1, 1, query=0x1004)
    dense[0].token_stride = 130  # not a multiple of 8 elements
    with pytest.raises(ValueError, match="16-byte token and head strides"):
        call(1, 1)
    dense[0].token_stride = 512
    dense[0].value = 0x3008
    with pytest.raises(ValueError, match="16-byte aligned"):
        call(0, 1)
    dense[0].value = 0x3000
    dense[0].tokens = 1 << 22  # 2^22 rows of 1 KiB: past 32-bit offsets
    with pytest.raises(ValueError, match="too long for 32-bit offsets"):
        call(0, 1)
    dense[0].tokens = 100
    packed[0].packed_capacity = 32
    with pytest.raises(ValueError, match="packed_capacity"):
        call(1, 0)
    packed[0].packed_capacity = 0
    with pytest.raises(ValueError, match="empty segment"):
        call(0, 0)
    with pytest.raises(ValueError, match="bad segment arrays"):
        nat.call("uc_kivi_attn_mq_segments", None, 1, dense, 0, q, q, None, *tail)


def test_editing_table_validation():
    q = 0x1000
    packed = (nat.KiviItem * 2)()
    for it in packed:
        it.quantized_tokens = 64
        for name in ("key_code", "key_scale", "key_min", "value_code", "value_scale", "value_min"):
            setattr(it, name, 0x2000)
    dense = (nat.DenseSegment * 2)()
    for d in dense:
        d.key, d.value, d.tokens, d.token_stride, d.head_stride = 0x3000, 0x3000, 100, 512, 128
    queries = (nat.MqQuery * 9)()
    for qq in queries:
        qq.query, qq.out, qq.query_len = q, q, 512
    tail = (2, 32, 28, 4, 128, nat.UC_BF16, nat.UC_BF16, nat.UC_BF16, 0.1, None)

    def call(n_queries):
        nat.call("uc_kivi_attn_mq_table", queries, n_queries, packed, 2, dense, 2, *tail)

    with pytest.raises(ValueError, match="n_queries must be 1..8"):
        call(0)
    with pytest.raises(ValueError, match="n_queries must be 1..8"):
        call(9)
    queries[0].packed_begin, queries[0].n_packed = 1, 2  # past the 2 packed items
    with pytest.raises(ValueError, match="outside the arrays"):
        call(1)
    queries[0].packed_begin, queries[0].n_packed = 0, 1
    queries[0].dense_begin, queries[0].n_dense = -1, 1
    with pytest.raises(ValueError, match="outside the arrays"):
        call(1)
    queries[0].dense_begin, queries[0].n_dense = 0, 0
    queries[1].out = q + 8  # the second query's output misaligned: refused before any launch
    with pytest.raises(ValueError, match="16-byte aligned"):
        call(2)


def test_copy_spans_validation():
    with pytest.raises(ValueError, match="0..8 spans per call"):
        nat.call("uc_copy_spans", None, 9, None)
    table = (ctypes.c_int64 * 3)(0, 0, -1)
    with pytest.raises(ValueError, match="negative size"):
        nat.call("uc_copy_spans", ctypes.addressof(table), 1, None)
    table = (ctypes.c_int64 * 3)(0, 0x1000, 16)
    with pytest.raises(ValueError, match="null pointer"):
        nat.call("uc_copy_spans", ctypes.addressof(table), 1, None)
    nat.call("uc_copy_spans", None, 0, None)  # nothing to copy, nothing launched
