"""KIVIQuantizationOperator (operators/builtin.py:281-476) on the GPU: the
quantized rows are the segment minus its last residual_length tokens minus
the protected ones, fake-quantized as one key block (groups along the selected
tokens) and one value block (groups along channels) and written back in place
-- bit-exact against the numpy oracle, with UniCache's record values."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kivi as K
from tests.helpers import f32, kv_pair
from unicache_amd.core.registry import OperatorExecutionContext
from unicache_amd.operators import KIVIQuantizationOperator

pytestmark = pytest.mark.gpu


def _ctx(k, v, seg, prot, params):
    records, snaps = [], []
    ctx = OperatorExecutionContext(
        runtime=SimpleNamespace(kv_metadata={}), step=SimpleNamespace(segment_id="vae"), params=params, q=None,
        k=k, v=v, attn_mask=None, key_type_ids=None, segment_mask=seg, protected_mask=prot, state={},
        record=records.append, set_storage_snapshot=snaps.append, storage_num_kv_heads=4)
    return ctx, records, snaps


def _expected(k, v, seg, prot, *, bits, group, residual, preserve=True):
    seg_idx = np.flatnonzero(seg)
    quant = seg.copy()
    if residual > 0 and seg_idx.size:
        quant[seg_idx[-residual:]] = False
    if preserve:
        quant &= ~prot
    ek, ev = f32(k).copy(), f32(v).copy()
    if quant.any():
        ek[quant] = K.fake_quant(ek[quant], bits=bits, dim=0, group_size=group)
        ev[quant] = K.fake_quant(ev[quant], bits=bits, dim=-1, group_size=group)
    return ek, ev, int(quant.sum())


@pytest.mark.parametrize("bits,group,residual", [(2, 32, 32), (4, 32, 128), (4, 64, 0), (8, 32, 17)])
def test_segment_masking_matches_oracle(device, bits, group, residual):
    key, value = kv_pair(512, seed=40 + bits)
    seg = np.zeros(512, dtype=bool)
    seg[40:460] = True
    prot = np.zeros(512, dtype=bool)
    prot[[10, 41, 42, 100, 250, 455]] = True  # inside and outside the segment
    ctx, records, snaps = _ctx(key.to(device), value.to(device), torch.from_numpy(seg).to(device),
                               torch.from_numpy(prot).to(device), {"bits": bits, "group_size": group,
                                                                   "residual_length": residual})
    op = KIVIQuantizationOperator()
    op.build_params(ctx.params)
    op.execute(ctx)
    ek, ev, n = _expected(key, value, seg, prot, bits=bits, group=group, residual=residual)
    assert np.array_equal(f32(ctx.k), ek) and np.array_equal(f32(ctx.v), ev)
    assert records[0]["quantized_tokens"] == n
    assert records[0]["protected_tokens_preserved"] == 5
    snap = snaps[0]
    assert snap["segment_tokens"] == 420 and snap["full_precision_tokens"] == 420 - n
    assert snap["original_storage_bytes"] == 420 * 4 * 128 * 2 * 2


def test_bypass_and_whole_segment_residual(device):
    key, value = kv_pair(128, seed=3)
    seg = torch.zeros(128, dtype=torch.bool)
    seg[:64] = True
    prot = torch.zeros(128, dtype=torch.bool)
    for params in ({"bits": 2, "bypass_quantization": True}, {"bits": 2, "residual_length": 64}):
        ctx, records, _ = _ctx(key.to(device), value.to(device), seg.to(device), prot.to(device), params)
        KIVIQuantizationOperator().execute(ctx)
        assert records[0]["quantized_tokens"] == 0
        assert torch.equal(ctx.k.cpu(), key) and torch.equal(ctx.v.cpu(), value)
    # protected tokens quantized too when preserve_protected is off
    prot[5] = True
    ctx, records, _ = _ctx(key.to(device), value.to(device), seg.to(device), prot.to(device),
                           {"bits": 4, "residual_length": 0, "preserve_protected": False})
    KIVIQuantizationOperator().execute(ctx)
    ek, ev, n = _expected(key, value, seg.numpy(), prot.numpy(), bits=4, group=32, residual=0, preserve=False)
    assert n == 64 and records[0]["protected_tokens_preserved"] == 0
    assert np.array_equal(f32(ctx.k), ek) and np.array_equal(f32(ctx.v), ev)


@pytest.mark.parametrize("n,residual,preserve,bypass", [(0, 4, 1, 0), (1, 0, 1, 0), (33, 5, 0, 0), (2048, 128, 1, 0),
                                                        (2048, 128, 1, 1), (70001, 5000, 1, 0), (5000, 0, 0, 0)])
def test_fake_quant_mask_kernel(device, n, residual, preserve, bypass):
    # uc_fake_quant_mask on scattered segment and protected masks: the selected
    # rows (segment minus its last `residual` tokens minus protected ones),
    # their compact order both ways and the three counts
    from unicache_amd import _native as nat

    rng = np.random.default_rng(n + residual)
    seg = rng.random(n) < 0.7
    prot = rng.random(n) < 0.05
    quant = seg.copy()
    idx = np.flatnonzero(seg)
    if residual > 0 and idx.size:
        quant[idx[-residual:]] = False
    if preserve:
        quant &= ~prot
    if bypass:
        quant[:] = False
    sd, pd = torch.from_numpy(seg).to(device), torch.from_numpy(prot).to(device)
    dst = torch.empty(max(n, 1), dtype=torch.int32, device=device)
    src = torch.empty(max(n, 1), dtype=torch.int32, device=device)
    counts = torch.empty(3, dtype=torch.int64, device=device)
    nat.call("uc_fake_quant_mask", sd.data_ptr(), pd.data_ptr(), n, residual, preserve, bypass, dst.data_ptr(),
             src.data_ptr(), counts.data_ptr(), nat.stream(device))
    sel = np.flatnonzero(quant)
    exp_dst = np.full(n, -1, dtype=np.int32)
    exp_dst[sel] = np.arange(sel.size)
    assert counts.cpu().tolist() == [int(seg.sum()), int(sel.size), int((seg & prot).sum())]
    assert np.array_equal(dst[:n].cpu().numpy(), exp_dst)
    assert np.array_equal(src[:sel.size].cpu().numpy(), sel)


def test_segment_masking_scattered_segment(device):
    # a segment of scattered tokens through the whole operator
    key, value = kv_pair(700, seed=9)
    rng = np.random.default_rng(9)
    seg = rng.random(700) < 0.6
    prot = rng.random(700) < 0.03
    ctx, records, _ = _ctx(key.to(device), value.to(device), torch.from_numpy(seg).to(device),
                           torch.from_numpy(prot).to(device), {"bits": 2, "group_size": 32, "residual_length": 40})
    KIVIQuantizationOperator().execute(ctx)
    ek, ev, n = _expected(key, value, seg, prot, bits=2, group=32, residual=40)
    assert records[0]["quantized_tokens"] == n
    assert np.array_equal(f32(ctx.k), ek) and np.array_equal(f32(ctx.v), ev)
