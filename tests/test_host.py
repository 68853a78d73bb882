"""Host-side behaviour of the drop-in API that needs no GPU: dispatch rules,
budget arithmetic and the fail-closed error contract (no CPU fallback)."""

import pytest
import torch

from oracle import h2o as H
from unicache_amd.core.decisions import PhysicalCacheRequest
from unicache_amd.operators import KIVIPackedQuantizationOperator, H2OPhysicalGQAOperator
from unicache_amd.storage import GQAH2OCache, PackedKIVICache
from unicache_amd.storage import kivi_cuda
from unicache_amd.storage.tensor_backend import h2o_budget


def test_kernel_backend_selection(monkeypatch):
    # kivi_cuda.py:26-34, test_physical.py:505-508
    monkeypatch.delenv("UNICACHE_KIVI_MULTI_QUERY_BACKEND", raising=False)
    assert kivi_cuda.select_kivi_kernel_backend(1) == "official_gemv"
    assert kivi_cuda.select_kivi_kernel_backend(2) == "triton_tiled"
    assert kivi_cuda.select_kivi_kernel_backend(802) == "triton_tiled"
    monkeypatch.setenv("UNICACHE_KIVI_MULTI_QUERY_BACKEND", "official_gemv")
    assert kivi_cuda.select_kivi_kernel_backend(802) == "official_gemv"
    monkeypatch.setenv("UNICACHE_KIVI_MULTI_QUERY_BACKEND", "bogus")
    with pytest.raises(ValueError):
        kivi_cuda.select_kivi_kernel_backend(1)


@pytest.mark.parametrize("n", [12, 256, 3840, 4096, 8192, 10, 1])
def test_budget_matches_oracle(n):
    for params in ({"target_budget_ratio": 0.2, "recent_budget_fraction": 0.25},
                   {"target_budget_ratio": 0.5}, {"budget": 7, "recent_size": 3}, {"keep_k": 5}):
        assert h2o_budget(n, params) == H.budget(n, params)


def test_cpu_tensors_fail_closed():
    key = torch.randn(64, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA"):
        PackedKIVICache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=3, k_bits=2,
                                   v_bits=2, group_size=32, residual_length=0, backend="cuda")
    for backend in ("reference", "cuda"):  # both backends run on the HIP kernels only
        with pytest.raises(RuntimeError, match="GPU|CUDA"):
            PackedKIVICache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=3, k_bits=2,
                                       v_bits=2, group_size=32, residual_length=0, backend=backend)
    with pytest.raises(ValueError, match="Unknown KIVI physical backend"):
        PackedKIVICache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=3, k_bits=2,
                                   v_bits=2, group_size=32, residual_length=0, backend="triton")
    with pytest.raises(RuntimeError):
        GQAH2OCache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=1,
                               per_kv_head_scores=torch.rand(4, 64), target_tokens=8, recent_tokens=2)


def test_argument_errors_are_value_errors():
    key = torch.randn(64, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        PackedKIVICache.from_dense(key, key[:, :2], logical_token_ids=torch.arange(64), token_type_id=3,
                                   k_bits=2, v_bits=2, group_size=32, residual_length=0)
    with pytest.raises(ValueError):
        PackedKIVICache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=3,
                                   k_bits=3, v_bits=2, group_size=32, residual_length=0)
    # the kernel-native layout (backend "cuda", 2/4-bit) keeps its group sizes;
    # every backend refuses a group size below 1 (physical.py:247-256)
    with pytest.raises(ValueError):
        PackedKIVICache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=3,
                                   k_bits=2, v_bits=2, group_size=48, residual_length=0, backend="cuda")
    with pytest.raises(ValueError):
        PackedKIVICache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=3,
                                   k_bits=2, v_bits=2, group_size=0, residual_length=0)
    with pytest.raises(ValueError):
        GQAH2OCache.from_dense(key, key, logical_token_ids=torch.arange(64), token_type_id=1,
                               per_kv_head_scores=torch.rand(3, 64), target_tokens=8, recent_tokens=2)


def test_operator_params_and_requests():
    op = KIVIPackedQuantizationOperator()
    params = op.build_params({"bits": 2, "group_size": 32, "residual_length": 128})
    assert params["k_bits"] == 2 and params["backend"] == "cuda" and params["residual_length"] == 128
    with pytest.raises(ValueError):
        op.build_params({"bits": 3})
    h2o = H2OPhysicalGQAOperator()
    assert h2o.build_params({})["target_budget_ratio"] == 0.2
    with pytest.raises(ValueError):
        h2o.build_params({"target_budget_ratio": 0.0})
    mask = torch.ones(5, dtype=torch.bool)
    with pytest.raises(ValueError):
        PhysicalCacheRequest(operator="x", segment_id="s", token_count=4, segment_mask=mask)
    with pytest.raises(ValueError):
        PhysicalCacheRequest(operator="x", segment_id="s", token_count=5, segment_mask=mask,
                             per_kv_head_scores=torch.zeros(2, 4))


def test_batched_attention_argument_checks():
    # run_batched_physical_attention (apply_static_physical_attention_batch,
    # adapters/bagel.py:773-980) checks its varlen table on the host before any
    # launch; the batch launcher rejects an empty or mixed item list the same way
    from unicache_amd.adapters import run_batched_physical_attention

    q = torch.zeros(6, 28, 128, dtype=torch.bfloat16)
    k = torch.zeros(5, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="one more entry"):
        run_batched_physical_attention(q, k, k, [0, 6], [0, 5], [[], []])
    with pytest.raises(ValueError, match="must cover q and k"):
        run_batched_physical_attention(q, k, k, [0, 3, 5], [0, 2, 5], [[], []])
    with pytest.raises(ValueError, match="no physical segments"):
        run_batched_physical_attention(q, k, k, [0, 3, 6], [0, 2, 5], [[], []])
    kivi_cuda.packed_batch_with_dense([])  # nothing to launch


def _native_cpu_cache(tokens, capacity, *, bits=2, group=32, heads=4, head_dim=128):
    # layout checks only: CPU tensors never reach a kernel here
    from unicache_amd.storage.physical import _native_storage, _native_views

    store = _native_storage(capacity, heads, head_dim, bits, bits, group, "cpu")
    kc, ks, km, vc, vs, vm = _native_views(store, tokens, bits, group)
    res = torch.zeros(0, heads, head_dim, dtype=torch.bfloat16)
    return PackedKIVICache(kc, ks, km, vc, vs, vm, res, res, torch.arange(tokens), 3, bits, bits, group, tokens,
                           head_dim, heads, backend="cuda", kernel_native_layout=True)


@pytest.mark.parametrize("bits", [2, 4])
def test_token_major_views_and_capacity(bits):
    c = _native_cpu_cache(256, 416, bits=bits)
    # reference shapes (kivi_cuda.py:177-182) over token-major storage
    assert tuple(c.key_code.shape) == (4, 128, 256 * bits // 32) and tuple(c.key_scale.shape) == (4, 128, 8)
    assert tuple(c.value_code.shape) == (4, 256, 128 * bits // 32) and tuple(c.value_minimum.shape) == (4, 256, 4)
    assert c.key_code.stride() == (416 * bits // 32 * 128, 1, 128) and c.key_scale.stride() == (13 * 128, 1, 128)
    assert c.packed_capacity == 416
    *ptrs, cap = c.native_packed_pointers()
    assert cap == 416 and ptrs[0] == c.key_code.data_ptr()
    # code word (h, d, w) sits at h*(C*b/32)*D + w*D + d of the storage
    flat = c.key_code.as_strided((4 * 416 * bits // 32 * 128,), (1,))
    flat.zero_()
    c.key_code[2, 5, 3] = 77
    assert int(flat[2 * (416 * bits // 32) * 128 + 3 * 128 + 5]) == 77


def test_token_major_layout_is_enforced():
    c = _native_cpu_cache(256, 256)
    assert c.packed_capacity == 256
    c.native_packed_pointers()
    # UniCache's word-major contiguous tensors of the same shapes are refused
    c.key_code = c.key_code.contiguous()
    with pytest.raises(ValueError, match="token-major"):
        c.native_packed_pointers()
    c = _native_cpu_cache(256, 256)
    c.value_scale = c.value_scale.float()
    with pytest.raises(ValueError, match="value_scale"):
        c.native_packed_pointers()
    c = _native_cpu_cache(256, 256)
    c.kernel_native_layout = False
    with pytest.raises(RuntimeError, match="kernel-native"):
        c.native_packed_pointers()


def test_fake_quant_operator_params():
    from unicache_amd.operators import KIVIQuantizationOperator

    op = KIVIQuantizationOperator()
    assert op.build_params({"bits": 2})["working_set_mode"] == "attention_view"
    with pytest.raises(ValueError, match="k_bits=5 is unsupported"):
        op.build_params({"bits": 4, "k_bits": 5})
    with pytest.raises(ValueError, match="working_set_mode must be"):
        op.build_params({"working_set_mode": "disk"})
    with pytest.raises(ValueError, match="host_backed"):
        op.build_params({"working_set_mode": "host_backed"})


@pytest.mark.parametrize("bits,group", [(2, 32), (4, 128)])
def test_native_block_matches_storage_views(bits, group):
    # from_dense's one-allocation block: the same native shapes and strides as
    # views of token-major storage, addresses on 256-byte boundaries, an ids slot
    from unicache_amd.storage.physical import _native_block, _native_storage, _native_views

    views, ptrs, ids = _native_block(512, 4, 128, bits, bits, group, "cpu", torch.int64, 512)
    ref = _native_views(_native_storage(512, 4, 128, bits, bits, group, "cpu"), 512, bits, group)
    for v, r, p in zip(views, ref, ptrs):
        assert v.dtype == r.dtype and v.shape == r.shape and v.stride() == r.stride()
        assert v.data_ptr() == p and (p - ptrs[0]) % 256 == 0  # 256-byte steps within the allocation
    assert ids.shape == (512,) and ids.dtype == torch.int64 and (ids.data_ptr() - ptrs[0]) % 256 == 0
    # the tensors do not overlap: each one starts past the previous one's last byte
    firsts = sorted(v.data_ptr() for v in [*views, ids])
    sizes = {v.data_ptr(): v.numel() * v.element_size() for v in [*views, ids]}
    for a, b in zip(firsts, firsts[1:]):
        assert a + sizes[a] <= b
