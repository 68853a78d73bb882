"""GPU parity of the dense keep-mask compaction (tensor_backend.py:54-77):
bit-exact rows, order and per-sample counts against the oracle."""

import numpy as np
import pytest
import torch

from oracle import h2o as H
from tests.helpers import kv_pair
from unicache_amd.storage.tensor_backend import TensorCacheStorageBackend, compact_rows

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lens,keep_frac,seed", [([4096], 0.2, 0), ([256, 3840], 0.2, 1), ([5, 0, 17, 1000], 0.5, 2),
                                                   ([300], 1.0, 3), ([300], 0.0, 4), ([33333], 0.9, 5)])
def test_compact_matches_oracle(device, lens, keep_frac, seed):
    total = sum(lens)
    key, value = kv_pair(total, seed=seed)
    ids = torch.arange(1000, 1000 + total, dtype=torch.int64)
    rng = np.random.default_rng(seed)
    masks = [torch.from_numpy(rng.random(n) < keep_frac) for n in lens]
    res = TensorCacheStorageBackend.compact(key=key.to(device), value=value.to(device),
                                            key_type_ids=ids.to(device),
                                            sample_lens=torch.tensor(lens, device=device),
                                            keep_masks=[m.to(device) for m in masks])
    ek, ev, ei, elens = H.compact(key.view(torch.int16).numpy(), value.view(torch.int16).numpy(), ids.numpy(),
                                  lens, [m.numpy() for m in masks])
    assert np.array_equal(res.key.cpu().view(torch.int16).numpy(), ek)
    assert np.array_equal(res.value.cpu().view(torch.int16).numpy(), ev)
    assert np.array_equal(res.key_type_ids.cpu().numpy(), ei)
    assert res.sample_lens.cpu().tolist() == elens
    assert res.compacted_bytes == 2 * ek.size * 2 and res.original_bytes == 2 * key.numel() * 2


@pytest.mark.parametrize("shape,dtype", [((257, 3, 5), torch.float16), ((64, 7), torch.float32),
                                         ((1000,), torch.int64), ((99, 1), torch.uint8)])
def test_compact_rows_any_row_width(device, shape, dtype):
    g = torch.Generator().manual_seed(7)
    t = (torch.randn(shape, generator=g) * 100).to(dtype)
    keep = torch.rand(shape[0], generator=g) < 0.6
    (out,) = compact_rows([t.to(device)], keep.to(device))
    assert torch.equal(out.cpu(), t[keep])


def test_compact_strided_rows(device):
    # rows of a [T, H, D] view whose row stride exceeds the row size
    base = torch.randn(50, 4, 128, dtype=torch.float32).to(torch.bfloat16)
    view = base.to(device)[:, 1:3]
    keep = torch.arange(50) % 3 == 0
    (out,) = compact_rows([view], keep.to(device))
    assert torch.equal(out.cpu(), base[:, 1:3][keep])


def test_compact_many_tensors_one_call(device):
    # six tensors of one mask: four 16-byte-aligned ones share one launch, the
    # fifth aligned one and the 12-byte rows take the per-tensor kernels
    g = torch.Generator().manual_seed(11)
    n = 1500
    tensors = [torch.randn(n, 4, 128, generator=g).to(torch.bfloat16), torch.randn(n, 2, 64, generator=g).half(),
               torch.randn(n, 8, generator=g), torch.randint(0, 99, (n, 2), generator=g, dtype=torch.int64),
               torch.randn(n, 16, generator=g).to(torch.bfloat16), torch.randn(n, 3, generator=g)]
    keep = torch.rand(n, generator=g) < 0.4
    outs = compact_rows([t.to(device) for t in tensors] + [None], keep.to(device))
    assert outs[-1] is None
    for t, o in zip(tensors, outs):
        assert torch.equal(o.cpu(), t[keep])


def test_compact_empty_cache(device):
    key = torch.zeros(0, 4, 128, dtype=torch.bfloat16, device=device)
    res = TensorCacheStorageBackend.compact(key=key, value=key.clone(), key_type_ids=None,
                                            sample_lens=torch.zeros(0, dtype=torch.long, device=device),
                                            keep_masks=[])
    assert res.key.shape == (0, 4, 128) and res.sample_lens.numel() == 0


def test_copy_spans_bit_exact(device):
    # one launch for several copies: 16-byte aligned spans, an odd-sized one
    # and an unaligned one, each equal to its source; bytes around the
    # destinations stay untouched
    import ctypes

    from unicache_amd import _native as nat

    g = torch.Generator().manual_seed(3)
    srcs = [torch.randint(0, 256, (n,), generator=g, dtype=torch.uint8).to(device) for n in (4096, 1000, 77, 0)]
    outs = [torch.full((n + 32,), 0xAB, dtype=torch.uint8, device=device) for n in (4096, 1000, 77, 0)]
    offsets = (16, 16, 3, 0)  # destination offsets inside the padded outputs
    spans = []
    for s, o, off in zip(srcs, outs, offsets):
        spans += [s.data_ptr(), o.data_ptr() + off, s.numel()]
    table = (ctypes.c_int64 * len(spans))(*spans)
    nat.call("uc_copy_spans", ctypes.addressof(table), len(srcs), nat.stream(device))
    for s, o, off in zip(srcs, outs, offsets):
        o = o.cpu()
        assert torch.equal(o[off:off + s.numel()], s.cpu())
        assert (o[:off] == 0xAB).all() and (o[off + s.numel():] == 0xAB).all()
