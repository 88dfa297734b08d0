"""Seeded random problems through every attention kernel family against the
oracle of attention() (src/model/attention.rs:101-186).

Each case draws a shape and the options a caller can combine: head dims
that fill their tile or not (multiples of 4 or not), GQA groups, sliding
windows, causal prefixes, batch slots, QK-norm, contiguous or scattered
query positions, a forced kernel family, forced key splits merged in-kernel
or by the merge kernel, bf16 Q rows where the stream kernel runs, key
counts that fill whole 32-key tiles (the cache store's tile kernel), and
hi/lo-precision layers (checked against the oracle on the unrounded f32
inputs, since that kernel is f32-accurate).  The seeds are fixed, so every
run draws the same cases.  A second set forces the stream kernel's 16-row
waves at head dim 256 over bands of up to ~1850 keys and grids of up to
three rounds of workgroups.  Needs an MI355X.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import check_raw, TOL_MAX, TOL_MEAN, RowsSpec, Shape, as_kernel_sees, err_stats

from test_gpu_kernels import dev, say  # noqa: F401

pytestmark = pytest.mark.gpu

N_CASES = 128


def _draw(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    kernel = [dr.KERNEL_AUTO, dr.KERNEL_STAGED, dr.KERNEL_STREAMS][seed % 3]
    hd_choices = [128, 256] if kernel == dr.KERNEL_STREAMS else [40, 64, 66, 96, 128, 130, 200, 256, 260, 384, 512]
    hd = int(rng.choice(hd_choices))
    hkv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 3, 7]))
    if hd > 256:
        hkv, group = min(hkv, 2), min(group, 3)
    n_p = int(rng.integers(0, 500))
    n_c = int(rng.integers(1, 180))
    batch = int(rng.choice([1, 1, 2]))
    window = int(rng.integers(16, 400)) if rng.random() < 0.4 else None
    prefix = int(rng.integers(0, n_p + n_c)) if rng.random() < 0.3 else None
    scattered = rng.random() < 0.3
    split = int(rng.choice([0, 0, 2, 3, 4]))
    in_kernel = bool(rng.random() < 0.7)
    qk_norm = bool(rng.random() < 0.4)
    bf16_q = kernel == dr.KERNEL_STREAMS and rng.random() < 0.5
    hilo = kernel == dr.KERNEL_AUTO and rng.random() < 0.35
    if seed % 4 == 0:
        # whole 32-key tiles from position 0: the cache store's tile kernel
        n_p = (n_p + n_c + 31) // 32 * 32 - n_c
        if prefix is not None:
            prefix = min(prefix, n_p + n_c - 1)
    return dict(kernel=kernel, hd=hd, hkv=hkv, h=hkv * group, n_p=n_p, n_c=n_c, batch=batch,
                window=window, prefix=prefix, scattered=scattered, split=split, in_kernel=in_kernel,
                qk_norm=qk_norm, bf16_q=bf16_q, hilo=hilo, seed=seed)


def _draw16(seed: int) -> dict:
    """A case for the stream kernel's 16-row waves at head dim 256
    (attn_ring16_kernel), forced so that bands longer than the planner's
    limit and grids of several rounds run on it too."""
    rng = np.random.default_rng(5000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 7]))
    n_p = int(rng.integers(0, 1600))
    n_c = int(rng.integers(1, 260))
    window = int(rng.integers(16, 1100)) if rng.random() < 0.5 else None
    prefix = int(rng.integers(0, n_p + n_c)) if rng.random() < 0.3 else None
    if seed % 4 == 0:
        n_p = (n_p + n_c + 31) // 32 * 32 - n_c
        if prefix is not None:
            prefix = min(prefix, n_p + n_c - 1)
    return dict(kernel=dr.KERNEL_STREAMS, hd=256, hkv=hkv, h=hkv * group, n_p=n_p, n_c=n_c,
                batch=int(rng.choice([1, 1, 2])), window=window, prefix=prefix,
                scattered=bool(rng.random() < 0.3), split=0, in_kernel=True,
                qk_norm=bool(rng.random() < 0.4), bf16_q=bool(rng.random() < 0.5), hilo=False,
                wave_rows=16, seed=seed)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_shape_vs_oracle(dev, seed):
    _check_case(dev, _draw(seed))


@pytest.mark.parametrize("seed", range(32))
def test_random_shape_16_row_waves_vs_oracle(dev, seed):
    _check_case(dev, _draw16(seed))


def _check_case(dev, c):
    seed = c["seed"]
    say(f"case {seed}: {c}")
    t = dev.t
    rng = np.random.default_rng(7000 + seed)
    h, hkv, hd, n_p, n_c, batch = c["h"], c["hkv"], c["hd"], c["n_p"], c["n_c"], c["batch"]
    n_t = n_p + n_c
    kvs = hkv * hd
    # query rows: the canvas (contiguous), or a sorted random subset
    if c["scattered"]:
        qpos = sorted(rng.choice(n_t, size=n_c, replace=False).tolist())
    else:
        qpos = list(range(n_p, n_t))
    qn = kn = None
    if c["qk_norm"]:
        qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    scale = 1 / math.sqrt(hd)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd], n_batch=batch)
    if c["hilo"]:
        cache.set_precision(0, dr.PRECISION_HILO)
    p_all = dr.Pass(dev.ctx, range(n_t))
    pq = dr.Pass(dev.ctx, qpos)
    items, outs, ins = [], [], []
    for b in range(batch):
        K = rng.standard_normal((n_t, kvs), dtype=np.float32)
        V = rng.standard_normal((n_t, kvs), dtype=np.float32)
        Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
        cache.store(0, p_all, dev.put(K), dev.put(V), dev.put(kn) if kn is not None else None, 1e-6, batch=b)
        if c["bf16_q"]:
            with t.cuda.stream(dev.stream):
                qd = t.from_numpy(Q).to("cuda").to(t.bfloat16)
            dev.stream.synchronize()
            Q = qd.float().cpu().numpy()  # the values the kernel reads
        else:
            qd = dev.put(Q)
        out = dev.empty(n_c * h * hd)
        items.append((qd, out, pq))
        outs.append(out)
        ins.append((Q, K, V))
    ctx = dev.ctx
    ctx.set_kernel(c["kernel"])
    ctx.set_split(c["split"])
    ctx.set_split_merge(c["in_kernel"])
    ctx.set_q_dtype(dr.DTYPE_BF16 if c["bf16_q"] else dr.DTYPE_F32)
    ctx.set_wave_rows(c.get("wave_rows", 0))
    try:
        cache.attention(0, items, h, sliding_window=c["window"], causal_prefix=c["prefix"], scale=scale,
                        q_norm_w=dev.put(qn) if qn is not None else None, q_norm_eps=1e-6)
        info = ctx.last_launch()
    finally:
        ctx.set_kernel(dr.KERNEL_AUTO)
        ctx.set_split(0)
        ctx.set_split_merge(True)
        ctx.set_q_dtype(dr.DTYPE_F32)
        ctx.set_wave_rows(0)
    say(f"  launch {info}")
    if c.get("wave_rows") == 16:
        assert info["kernel"] == dr.KERNEL_STREAMS and info["rows_per_wave"] == 16 and info["n_split"] == 1, info
    if c["kernel"] != dr.KERNEL_AUTO:
        assert info["kernel"] in (c["kernel"], dr.KERNEL_STAGED)  # STREAMS falls back where it does not apply
    if c["bf16_q"]:
        assert info["kernel"] == dr.KERNEL_STREAMS
    if c["hilo"]:
        assert info["kernel"] == dr.KERNEL_HILO
    if c["split"]:
        assert info["n_split"] == c["split"]
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=c["window"], causal_prefix=c["prefix"], scale=scale)
    qr, kr = RowsSpec(qpos), RowsSpec(list(range(n_t)))
    for b, ((Q, K, V), o) in enumerate(zip(ins, outs)):
        got = dev.get(o)
        q, k = Q.reshape(-1).copy(), K.reshape(-1).copy()
        if qn is not None:
            orc.norm_heads(q, qn, 1e-6)
            orc.norm_heads(k, kn, 1e-6)
        want = np.zeros(n_c * h * hd, np.float32)
        if c["hilo"]:
            orc.attention(want, q, k, V.reshape(-1).copy(), s, qr, kr, threads=0)
        else:
            orc.attention(want, *as_kernel_sees(q, k, V.reshape(-1).copy(), scale), s, qr, kr, threads=0)
            check_raw(orc, got, q, k, V.reshape(-1).copy(), s, qr, kr, f"seed {seed} batch {b}", say)
        # rows with no visible key are NaN in both
        assert np.array_equal(np.isnan(got), np.isnan(want)), (seed, b)
        mx, mean = err_stats(got, want)
        say(f"  batch {b}: max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (seed, b, mx, mean)
