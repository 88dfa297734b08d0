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
    # a key band above 4608 (window 5000 from the last 256 or 100 of 6256
    # positions: 5255 or 5099 keys) keeps hd 256 on the staged kernel, which
    # splits the keys by itself
    "hd256_window_auto_split": (16, 8, 256, 6000, 256, 100, 5000, 0),
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


def test_noalloc_first_call_allocates_nothing(dev):
    """On a fresh context, dr_attention_cached_noalloc as the first call that
    needs a split workspace makes no allocation (the library's counter of its
    hipMalloc / hipHostMalloc calls stands still over two calls, the second
    smaller), while dr_attention_cached on the same problem then does (the
    counter sees allocations), with bit-identical results."""
    h, hd, n_p, n_c1, n_c2 = 8, 128, 1400, 200, 70
    rng = np.random.default_rng(11)
    n_t = n_p + n_c1
    ctx = dr.Context(0)
    ctx.set_stream(dev.stream.cuda_stream)
    ctx.set_split(3)
    cache = dr.StepCache(ctx, n_t, [h], [hd])
    K = rng.standard_normal((n_t, h * hd), dtype=np.float32)
    V = rng.standard_normal((n_t, h * hd), dtype=np.float32)
    cache.store(0, dr.Pass(ctx, range(n_t)), dev.put(K), dev.put(V))
    calls = []
    for n_c in (n_c1, n_c2):
        calls.append((dr.Pass(ctx, range(n_t - n_c, n_t)), dev.put(rng.standard_normal((n_c, h * hd),
                                                                                        dtype=np.float32)),
                      dev.empty(n_c * h * hd), dev.empty(n_c * h * hd)))
    dev.get(calls[-1][3])
    before = dr.alloc_count()
    for pc, Q, out, _ in calls:
        cache.attention(0, [(Q, out, pc)], h, scale=1 / math.sqrt(hd), noalloc=True)
        assert ctx.last_launch()["n_split"] == 3
    dev.get(calls[-1][2])
    assert dr.alloc_count() == before, "dr_attention_cached_noalloc allocated"
    for pc, Q, _, out in calls:
        cache.attention(0, [(Q, out, pc)], h, scale=1 / math.sqrt(hd))
    dev.get(calls[-1][3])
    assert dr.alloc_count() > before, "dr_attention_cached grows the context's split workspace"
    for _, _, a, b in calls:
        ga, gb = dev.get(a), dev.get(b)
        assert not np.any(np.isnan(ga))
        assert np.array_equal(ga, gb)
    ctx.close()


def test_noalloc_hilo_layer_with_q_norm_below_the_tile(dev):
    """A hi/lo layer with a QK-norm at a head dim below its tile (96) runs the
    Q epilogue into a Q workspace first; the allocation-free entry point puts
    that workspace in the fixed scratch too: same bits as
    dr_attention_cached, no allocation."""
    h, hkv, hd, n_t, n_c = 4, 2, 96, 320, 64
    rng = np.random.default_rng(12)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.set_precision(0, dr.PRECISION_HILO)
    K = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    V = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    pc = dr.Pass(dev.ctx, range(n_t - n_c, n_t))
    Q = dev.put(rng.standard_normal((n_c, h * hd), dtype=np.float32))
    w = dev.put(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    outs = [dev.empty(n_c * h * hd) for _ in range(2)]
    dev.get(outs[1])
    before = dr.alloc_count()
    cache.attention(0, [(Q, outs[0], pc)], h, scale=1.0, q_norm_w=w, noalloc=True)
    assert dev.ctx.last_launch()["kernel"] == dr.KERNEL_HILO
    dev.get(outs[0])
    assert dr.alloc_count() == before
    cache.attention(0, [(Q, outs[1], pc)], h, scale=1.0, q_norm_w=w)
    a, b = dev.get(outs[0]), dev.get(outs[1])
    assert not np.any(np.isnan(a))
    assert np.array_equal(a, b)
