"""A StepCache of several layers on the device (StepCache holds one K and one
V array per layer, src/model/cache.rs:25-54; per-layer geometry from
build_layer_attn, src/model/loader.rs:318-379): every layer is stored and
attended with its own data, in interleaved order, and checked against the
oracle; afterwards every layer's K/V is read back and must still be the bf16
of what was stored into it, so no layer's store or attention touched
another's.  Needs an MI355X.

Two caches:
- BASELINE.json's C5 as stated: DiffusionGemma shape, 16 query / 8 KV heads
  at head dim 256, 4096 cached + 256 canvas, layers S,S,S,S,S,G (sliding
  layers: symmetric window 1024; global: full), scale 1/sqrt(256);
- DiffusionGemma's real mixed geometry (docs/diffusiongemma.md:8-14,
  loader.rs:339-377): sliding layers 8 KV heads at head dim 256, the global
  layer 2 KV heads at head dim 512, one cache holding both.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import TOL_MAX, TOL_MEAN, RowsSpec, Shape, as_kernel_sees, bf16_round, err_stats

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


# per layer: (n_head_kv, head_dim, sliding window or None)
GEOMETRIES = {
    "c5_six_layers": dict(n_head=16, n_prompt=4096, n_canvas=256,
                          layers=[(8, 256, 1024)] * 5 + [(8, 256, None)]),
    "gemma_mixed_hd256_hd512": dict(n_head=16, n_prompt=1536, n_canvas=256,
                                    layers=[(8, 256, 1024)] * 5 + [(2, 512, None)]),
}
ORDER = [3, 0, 5, 1, 4, 2]  # stores and attentions interleaved across layers


@pytest.mark.parametrize("name", list(GEOMETRIES))
def test_multi_layer_cache_vs_oracle(dev, name):
    geo = GEOMETRIES[name]
    h, n_p, n_c = geo["n_head"], geo["n_prompt"], geo["n_canvas"]
    n_t = n_p + n_c
    layers = geo["layers"]
    cache = dr.StepCache(dev.ctx, n_t, [g[0] for g in layers], [g[1] for g in layers])
    p_all = dr.Pass(dev.ctx, range(n_t))
    p_can = dr.Pass(dev.ctx, range(n_p, n_t))
    rng = np.random.default_rng(sum(map(ord, name)))
    data = {}
    for layer in ORDER:
        hkv, hd, window = layers[layer]
        K = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
        V = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
        Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
        data[layer] = (Q, K, V)
        cache.store(layer, p_all, dev.put(K), dev.put(V))
        out = dev.empty(n_c * h * hd)
        scale = 1 / math.sqrt(hd)
        cache.attention(layer, [(dev.put(Q), out, p_can)], h, sliding_window=window, scale=scale)
        info = dev.ctx.last_launch()
        got = dev.get(out)
        s = Shape(n_c, n_t, h, hkv, hd, sliding_window=window, scale=scale)
        qr, kr = RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t)))
        want = np.zeros(n_c * h * hd, np.float32)
        orc.attention(want, Q.reshape(-1).copy(), K.reshape(-1).copy(), V.reshape(-1).copy(), s, qr, kr,
                      threads=0)
        mx, mean = err_stats(got, want)
        say(f"{name} layer {layer} (hkv {hkv}, hd {hd}, window {window}): max-abs {mx:.3e} "
            f"mean-abs {mean:.3e}; launch hd tile {info['head_dim_tile']} split {info['n_split']}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (layer, mx, mean)
    # every layer still holds the bf16 of its own rows
    for layer, (hkv, hd, _) in enumerate(layers):
        _, K, V = data[layer]
        ok, ov = dev.empty(n_t * hkv * hd), dev.empty(n_t * hkv * hd)
        cache.gather(layer, range(n_t), ok, ov)
        gk, gv = dev.get(ok), dev.get(ov)
        assert np.array_equal(gk, bf16_round(K).reshape(-1)), f"layer {layer} K changed"
        assert np.array_equal(gv, bf16_round(V).reshape(-1)), f"layer {layer} V changed"
    say(f"{name}: all {len(layers)} layers intact after the interleaved stores and attentions")


def test_layer_index_out_of_range_is_an_error(dev):
    cache = dr.StepCache(dev.ctx, 64, [2, 2], [128, 128])
    p = dr.Pass(dev.ctx, range(64))
    z = dev.put(np.zeros((64, 256), np.float32))
    with pytest.raises(dr.DrError) as ei:
        cache.store(2, p, z, z)
    assert ei.value.status == dr.DR_ERR_INVALID
