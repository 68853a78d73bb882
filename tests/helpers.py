"""Seeded synthetic inputs shared by the GPU tests (BAGEL-7B-MoT shapes)."""

import numpy as np
import torch


def kv_pair(tokens, heads=4, head_dim=128, *, seed=0, outliers=8, dtype=torch.bfloat16):
    """K with `outliers` random channels per head scaled x10 (config 0), V N(0,1)."""

    g = torch.Generator().manual_seed(seed)
    key = torch.randn(tokens, heads, head_dim, generator=g, dtype=torch.float32)
    value = torch.randn(tokens, heads, head_dim, generator=g, dtype=torch.float32)
    for h in range(heads):
        ch = torch.randperm(head_dim, generator=g)[:outliers]
        key[:, h, ch] *= 10.0
    return key.to(dtype), value.to(dtype)


def queries(length, heads=28, head_dim=128, *, seed=1, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(length, heads, head_dim, generator=g, dtype=torch.float32).to(dtype)


def f32(t):
    return t.detach().float().cpu().numpy()


def assert_close(actual, expected, *, max_abs=2e-2, mean_abs=1e-3, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    err = np.abs(a - e)
    assert np.isfinite(a).all(), what
    assert err.max() <= max_abs, f"{what}: max abs err {err.max():.3g} > {max_abs}"
    assert err.mean() <= mean_abs, f"{what}: mean abs err {err.mean():.3g} > {mean_abs}"
