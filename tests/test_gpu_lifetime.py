"""Object lifetimes of the C ABI (include/dr_attn.h dr_ctx_destroy): passes,
caches and RoPE tables hold their context, so destroying the context first
and the objects afterwards is safe, as a garbage collector may do.  Needs an
MI355X."""
from __future__ import annotations

import math

import numpy as np
import pytest

import dr_attn as dr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    if not t.cuda.is_available() or dr.device_count() == 0:
        pytest.skip("no GPU visible")
    dr.load()
    return t


def test_context_destroyed_before_its_objects(torch):
    ctx = dr.Context(0)
    h, hd, n = 4, 128, 96
    cache = dr.StepCache(ctx, n, [h], [hd])
    p = dr.Pass(ctx, range(n))
    rope = dr.Rope(ctx, n, hd, 10000.0)
    k = torch.randn(n, h * hd, device="cuda")
    cache.store(0, p, k, k)
    ctx.close()  # the caller's hold only: the cache, pass and table keep it
    q = torch.randn(n, h * hd, device="cuda")
    out = torch.empty(n * h * hd, device="cuda")
    cache.attention(0, [(q, out, p)], h, scale=1 / math.sqrt(hd))
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()
    rope.close()
    p.close()
    cache.close()  # the last hold: the context is freed here
