"""dr_attention_cached_noalloc (include/dr_attn.h) against dr_attention_cached:
the same plan and kernels, with the key-split partials in the library's fixed
device scratch instead of the context's workspace, so the outputs must be
bit-identical.  Two calls in a row on each shape, the second with fewer
query rows (the scratch keeps the first call's contents).  Needs an MI355X.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import dr_attn as dr

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available() or dr.device_count() == 0:
        pytest.skip("no GPU visible")
    dr.load()

    class Dev:
        def __init__(self):
            self.t = torch
            self.stream = torch.cuda.Stream()
            self.ctx = dr.Context(0)
            self.ctx.set_stream(self.stream.cuda_stream)

        def put(self, a):
            with torch.cuda.stream(self.stream):
                return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")

        def empty(self, n):
            with torch.cuda.stream(self.stream):
                return torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")

        def get(self, x):
            self.stream.synchronize()
            return x.cpu().numpy()

    return Dev()


# (h, hkv, hd, n_prompt, n_canvas first call, n_canvas second call, window, forced splits)
SHAPES = {
    "hd128_split3": (8, 8, 128, 1400, 200, 70, None, 3),
    # a window above 1024 keeps hd 256 on the staged kernel, which splits the keys by itself
    "hd256_window_auto_split": (16, 8, 256, 2048, 256, 100, 1500, 0),
    # the per-wave-stream kernel (hd 256, window <= 1024) with forced splits
    "hd256_streams_split2": (16, 8, 256, 2048, 256, 100, 700, 2),
}


@pytest.mark.parametrize("name", list(SHAPES))
def test_noalloc_matches_cached_twice(dev, name):
    h, hkv, hd, n_p, n_c1, n_c2, window, n_split = SHAPES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    n_t = n_p + n_c1
    kvs = hkv * hd
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    K = rng.standard_normal((n_t, kvs), dtype=np.float32)
    V = rng.standard_normal((n_t, kvs), dtype=np.float32)
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    dev.ctx.set_split(n_split)
    try:
        for call, n_c in enumerate((n_c1, n_c2)):
            pc = dr.Pass(dev.ctx, range(n_t - n_c, n_t))
            Q = dev.put(rng.standard_normal((n_c, h * hd), dtype=np.float32))
            outs = {}
            for noalloc in (False, True):
                out = dev.empty(n_c * h * hd)
                cache.attention(0, [(Q, out, pc)], h, sliding_window=window, scale=1 / math.sqrt(hd),
                                noalloc=noalloc)
                info = dev.ctx.last_launch()
                outs[noalloc] = dev.get(out)
            say(f"{name} call {call} (n_c {n_c}): launch {info}")
            assert info["n_split"] > 1, "the shape must use the split workspace"
            if name == "hd256_window_auto_split":
                assert info["kernel"] == dr.KERNEL_STAGED
            if name == "hd256_streams_split2":
                assert info["kernel"] == dr.KERNEL_STREAMS
            assert not np.any(np.isnan(outs[False]))
            assert np.array_equal(outs[False], outs[True]), name
    finally:
        dev.ctx.set_split(0)


def test_noalloc_rejects_workspace_beyond_scratch(dev):
    """A plan whose partials exceed the fixed 64 MiB is an error, not an
    allocation: 32 heads x 2048 queries at hd 128 in 2 splits need 68 MB."""
    h, hd, n_t, n_c = 32, 128, 2560, 2048
    cache = dr.StepCache(dev.ctx, n_t, [h], [hd])
    pc = dr.Pass(dev.ctx, range(n_t - n_c, n_t))
    q = dev.empty(n_c * h * hd)
    out = dev.empty(n_c * h * hd)
    dev.ctx.set_split(2)
    try:
        with pytest.raises(dr.DrError) as ei:
            cache.attention(0, [(q, out, pc)], h, scale=0.1, noalloc=True)
    finally:
        dev.ctx.set_split(0)
    assert ei.value.status == dr.DR_ERR_INVALID
    say(f"rejected: {ei.value.message}")
