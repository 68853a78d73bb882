"""uc_kivi_attn_decode_static (no workspace argument, library-held scratch)
against uc_kivi_attn_decode with a caller workspace: bit-identical outputs
and LSEs on two calls in a row, the second over a shorter segment."""

import ctypes
import math

import pytest
import torch

from tests.helpers import kv_pair, queries
from unicache_amd import _native as nat
from unicache_amd.storage import PackedKIVICache

pytestmark = pytest.mark.gpu


def _summaries(cache, q, *, static):
    lq, hq, d = map(int, q.shape)
    out = torch.full((lq, hq, d), float("nan"), dtype=q.dtype, device=q.device)
    lse = torch.full((hq, lq), float("nan"), dtype=torch.float32, device=q.device)
    tr = cache.residual_tokens
    item = cache.native_item(q.data_ptr(), out.data_ptr(), lse.data_ptr(),
                             residual_key_ptr=cache.residual_key.data_ptr() if tr else None,
                             residual_value_ptr=cache.residual_value.data_ptr() if tr else None, residual_tokens=tr)
    args = (cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq, nat.dtype_code(q.dtype),
            nat.dtype_code(cache.residual_key.dtype), nat.dtype_code(q.dtype), 1.0 / math.sqrt(d))
    if static:
        nat.call("uc_kivi_attn_decode_static", ctypes.byref(item), *args, nat.stream(q.device))
    else:
        ws_bytes = nat.decode_workspace_bytes(1, cache.k_bits, cache.group_size, hq, cache.num_kv_heads, d, lq,
                                              cache.quantized_tokens, tr)
        ws = nat.workspace(q.device, ws_bytes)
        nat.call("uc_kivi_attn_decode", ctypes.byref(item), *args, ws.data_ptr(), ws_bytes, nat.stream(q.device))
    torch.cuda.synchronize()
    return out, lse


# (bits, group, query_len, [tokens of call 1, tokens of call 2]); group 16 runs
# the generic split-K kernel, the others the MFMA kernel
CASES = [(2, 32, 1, [32768, 4096]), (4, 64, 2, [8192, 1000]), (2, 16, 1, [6000, 700])]


@pytest.mark.parametrize("bits,group,lq,sizes", CASES)
def test_static_decode_equals_workspace_decode(device, bits, group, lq, sizes):
    for call, tokens in enumerate(sizes):
        print(f"static decode bits={bits} group={group} lq={lq} tokens={tokens} call={call}", flush=True)
        key, value = kv_pair(tokens, seed=40 + call)
        cache = PackedKIVICache.from_dense(key.to(device), value.to(device), logical_token_ids=torch.arange(tokens),
                                           token_type_id=3, k_bits=bits, v_bits=bits, group_size=group,
                                           residual_length=128, backend="cuda")
        q = queries(lq, seed=50 + call).to(device)
        out_ws, lse_ws = _summaries(cache, q, static=False)
        out_st, lse_st = _summaries(cache, q, static=True)
        assert torch.isfinite(out_ws.float()).all() and torch.isfinite(lse_ws).all()
        assert torch.equal(out_st, out_ws), f"call {call}: outputs differ"
        assert torch.equal(lse_st, lse_ws), f"call {call}: LSEs differ"


def test_static_decode_rejects_oversized_segment(device):
    # 4M packed tokens need ~34 MB of split scratch: refused before any launch
    item = nat.KiviItem()
    item.quantized_tokens = 1 << 22
    with pytest.raises(ValueError, match="scratch"):
        nat.call("uc_kivi_attn_decode_static", ctypes.byref(item), 2, 32, 28, 4, 128, 1, nat.UC_BF16, nat.UC_BF16,
                 nat.UC_BF16, 0.088, nat.stream(device))
    assert nat.lib().uc_kivi_decode_scratch_bytes() == 8 << 20
