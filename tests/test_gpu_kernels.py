"""The two attention kernel families (include/dr_attn.h DR_KERNEL_STAGED /
DR_KERNEL_STREAMS) on the same problems, each against the oracle of
attention() (src/model/attention.rs:101-186): MHA and GQA, several batch
slots, ragged key and row tails, sliding window, causal prefix, QK-norm and
key splits.  Also: the per-wave-stream kernel gives bit-identical results
from call to call (fixed summation order), and the planner picks it where it
is the faster one.  Needs an MI355X.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import check_raw, TOL_MAX, TOL_MEAN, RowsSpec, Shape, as_kernel_sees, err_stats

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


# (h, hkv, n_prompt, n_canvas, batch, window, prefix, qk_norm, n_split)
CASES = {
    "mha": (8, 8, 600, 256, 1, None, None, False, 0),
    "mha_ragged": (4, 4, 203, 77, 1, None, None, False, 0),
    "gqa_batch2": (14, 2, 300, 100, 2, None, None, False, 0),
    "window": (8, 4, 700, 160, 1, 150, None, False, 0),
    "prefix": (8, 8, 300, 130, 1, None, 360, False, 0),
    "window_prefix": (6, 3, 500, 111, 2, 90, 540, False, 0),
    "qk_norm": (8, 8, 400, 96, 1, None, None, True, 0),
    "split2": (4, 4, 900, 64, 1, None, None, False, 2),
    "split3_window": (4, 2, 1500, 64, 1, 400, None, False, 3),
    # 256 one-block workgroups streaming 36 key tiles each: the 8-wave build
    # of the per-wave-stream kernel (test_planner_hd128_waves)
    "long_stream": (8, 8, 100, 1024, 1, None, None, False, 0),
}
# head dim 256 (DiffusionGemma's sliding and global layers): the same kinds
# of problem for the 4-wave build of the per-wave-stream kernel
CASES_256 = {
    "mha": (4, 4, 600, 200, 1, None, None, False, 0),
    "ragged": (2, 2, 203, 77, 1, None, None, False, 0),
    "gqa_batch2": (8, 4, 300, 100, 2, None, None, False, 0),
    "window": (8, 4, 1100, 160, 1, 300, None, False, 0),
    "window_prefix": (4, 2, 500, 111, 2, 90, 540, False, 0),
    "qk_norm": (4, 4, 400, 96, 1, None, None, True, 0),
    "split2": (4, 4, 900, 64, 1, None, None, False, 2),
    "split3_window": (4, 2, 1500, 64, 1, 400, None, False, 3),
    # no window, 1256 keys, 64 one-block workgroups: the planner's choice
    # (run under DR_KERNEL_AUTO by test_planner_hd256_key_band)
    "global_auto": (8, 4, 1000, 256, 1, None, None, False, 0),
}


def _run(dev, name, kernel, hd=128, wave_rows=0):
    h, hkv, n_p, n_c, batch, window, prefix, qk_norm, n_split = (CASES if hd == 128 else CASES_256)[name]
    n_t = n_p + n_c
    kvs = hkv * hd
    rng = np.random.default_rng(sum(map(ord, name)) + hd)
    qn = kn = None
    if qk_norm:
        qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd], n_batch=batch)
    p_all = dr.Pass(dev.ctx, range(n_t))
    pc = dr.Pass(dev.ctx, range(n_p, n_t))
    ins, items, outs = [], [], []
    for b in range(batch):
        K = rng.standard_normal((n_t, kvs), dtype=np.float32)
        V = rng.standard_normal((n_t, kvs), dtype=np.float32)
        Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
        cache.store(0, p_all, dev.put(K), dev.put(V), dev.put(kn) if qk_norm else None, 1e-6, batch=b)
        out = dev.empty(n_c * h * hd)
        items.append((dev.put(Q), out, pc))
        outs.append(out)
        ins.append((Q, K, V))
    dev.ctx.set_kernel(kernel)
    dev.ctx.set_split(n_split)
    dev.ctx.set_wave_rows(wave_rows)
    try:
        cache.attention(0, items, h, sliding_window=window, causal_prefix=prefix,
                        scale=1 / math.sqrt(hd), q_norm_w=dev.put(qn) if qk_norm else None,
                        q_norm_eps=1e-6)
        info = dev.ctx.last_launch()
    finally:
        dev.ctx.set_kernel(dr.KERNEL_AUTO)
        dev.ctx.set_split(0)
        dev.ctx.set_wave_rows(0)
    got = [dev.get(o) for o in outs]
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=window, causal_prefix=prefix, scale=1 / math.sqrt(hd))
    qr, kr = RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t)))
    wants, raws = [], []
    for Q, K, V in ins:
        q, k = Q.reshape(-1).copy(), K.reshape(-1).copy()
        if qk_norm:
            orc.norm_heads(q, qn, 1e-6)
            orc.norm_heads(k, kn, 1e-6)
        want = np.zeros(n_c * h * hd, np.float32)
        # the oracle on the operands as the kernel rounds them: the kernel's
        # own arithmetic at the standard bar on every row
        orc.attention(want, *as_kernel_sees(q, k, V.reshape(-1).copy(), 1 / math.sqrt(hd)), s, qr, kr,
                      threads=0)
        wants.append(want)
        raws.append((q, k, V.reshape(-1).copy()))
    for b, (g, (q, k, v)) in enumerate(zip(got, raws)):  # and the raw f32 inputs
        check_raw(orc, g, q, k, v, s, qr, kr, f"{name} batch {b}", say)
    return got, wants, info


@pytest.mark.parametrize("kernel", [dr.KERNEL_STAGED, dr.KERNEL_STREAMS], ids=["staged", "streams"])
@pytest.mark.parametrize("name", list(CASES))
def test_kernel_family_vs_oracle(dev, name, kernel):
    got, wants, info = _run(dev, name, kernel)
    say(f"{name} kernel {kernel}: launch {info}")
    assert info["kernel"] == kernel
    if CASES[name][8]:
        assert info["n_split"] == CASES[name][8]
    for b, (g, w) in enumerate(zip(got, wants)):
        mx, mean = err_stats(g, w)
        say(f"  batch {b}: max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (name, b, mx, mean)


@pytest.mark.parametrize("kernel", [dr.KERNEL_STAGED, dr.KERNEL_STREAMS], ids=["staged", "streams"])
@pytest.mark.parametrize("name", [n for n in CASES_256 if n != "global_auto"])
def test_kernel_family_hd256_vs_oracle(dev, name, kernel):
    got, wants, info = _run(dev, name, kernel, hd=256)
    say(f"hd 256 {name} kernel {kernel}: launch {info}")
    assert info["kernel"] == kernel
    if kernel == dr.KERNEL_STREAMS:
        assert info["waves_per_wg"] == 4
    if CASES_256[name][8]:
        assert info["n_split"] == CASES_256[name][8]
    for b, (g, w) in enumerate(zip(got, wants)):
        mx, mean = err_stats(g, w)
        say(f"  batch {b}: max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (name, b, mx, mean)


@pytest.mark.parametrize("name", [n for n in CASES_256 if not CASES_256[n][8]])
def test_streams_16_row_waves_hd256_vs_oracle(dev, name):
    """The per-wave-stream kernel with 16-row waves at head dim 256
    (attn_ring16_kernel: one 16-row block per workgroup, no key split)."""
    got, wants, info = _run(dev, name, dr.KERNEL_STREAMS, hd=256, wave_rows=16)
    say(f"hd 256 {name} 16-row waves: launch {info}")
    assert info["kernel"] == dr.KERNEL_STREAMS and info["rows_per_wave"] == 16 and info["n_split"] == 1, info
    for b, (g, w) in enumerate(zip(got, wants)):
        mx, mean = err_stats(g, w)
        say(f"  batch {b}: max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (name, b, mx, mean)


@pytest.mark.parametrize("name", ["mha", "gqa_batch2", "window_prefix", "qk_norm"])
def test_kernel_families_agree(dev, name):
    """The two families compute the same function: they differ only in the
    order of the f32 sums (and where the running max moves)."""
    a, _, _ = _run(dev, name, dr.KERNEL_STAGED)
    b, _, _ = _run(dev, name, dr.KERNEL_STREAMS)
    for x, y in zip(a, b):
        assert np.max(np.abs(x - y)) < 2e-3


def test_streams_kernel_is_deterministic(dev):
    """Each wave owns a fixed set of key tiles, so every call sums each
    row's keys in the same order: repeated calls are bit-identical."""
    for hd in (128, 256):
        first, _, _ = _run(dev, "window_prefix", dr.KERNEL_STREAMS, hd)
        for _ in range(3):
            again, _, _ = _run(dev, "window_prefix", dr.KERNEL_STREAMS, hd)
            for x, y in zip(first, again):
                assert np.array_equal(x, y)


def test_planner_picks_streams_for_one_round(dev):
    """C2's shape (32 heads x 8 row blocks = 256 one-block workgroups) runs
    the per-wave-stream kernel; C3's GQA rows (448 blocks) keep the staged
    kernel's 64-row workgroups."""
    hd = 128
    for h, hkv, n_c, want in ((32, 32, 256, dr.KERNEL_STREAMS), (28, 4, 256, dr.KERNEL_STAGED)):
        n_t = 512 + n_c
        cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd], n_batch=2)
        pc = dr.Pass(dev.ctx, range(512, n_t))
        z = dev.put(np.zeros((n_t, hkv * hd), np.float32))
        for b in range(2):
            cache.store(0, dr.Pass(dev.ctx, range(n_t)), z, z, batch=b)
        q = dev.put(np.zeros((n_c, h * hd), np.float32))
        items = [(q, dev.empty(n_c * h * hd), pc) for _ in range(2 if hkv == 4 else 1)]
        cache.attention(0, items, h, scale=0.1)
        assert dev.ctx.last_launch()["kernel"] == want, (h, hkv)


def test_planner_hd128_waves(dev):
    """Head dim 128: the per-wave-stream kernel runs 4 waves per workgroup
    when a workgroup streams at most 32 key tiles (after any key split) and 8
    above, whose loads keep twice the bytes in flight; both builds against
    the oracle at the planner's choice."""
    for name, waves in (("mha", 4), ("split2", 4), ("long_stream", 8)):
        got, wants, info = _run(dev, name, dr.KERNEL_AUTO)
        say(f"{name}: launch {info}")
        assert info["kernel"] == dr.KERNEL_STREAMS and info["waves_per_wg"] == waves, (name, info)
        for g, w in zip(got, wants):
            mx, mean = err_stats(g, w)
            say(f"  max-abs {mx:.3e} mean-abs {mean:.3e}")
            assert mx <= TOL_MAX and mean <= TOL_MEAN, (name, mx, mean)


def test_planner_hd256_16_row_waves(dev):
    """Head dim 256 with a short key band: 16-row waves (one 16-row block per
    workgroup, no key split) where their workgroups fill more than half the
    CUs in one round; longer bands keep the 32-row kernel's two splits."""
    hd = 256
    # (h, hkv, n_prompt, n_canvas, window, rows per wave, n_split)
    cases = (
        (16, 8, 4096, 256, 1024, 16, 1),   # C5 sliding: band of 1279 keys
        (16, 8, 4096, 256, 256, 16, 1),
        (16, 8, 4096, 256, 1536, 32, 2),   # band of 1791 keys
        (16, 8, 1024, 256, None, 16, 1),   # 1280 keys
        (16, 8, 2048, 256, None, 32, 2),   # 2304 keys
        (8, 4, 1000, 256, None, 32, 2),    # 128 16-row workgroups: half the CUs
    )
    for h, hkv, n_p, n_c, window, rows, n_split in cases:
        n_t = n_p + n_c
        cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
        z = dev.put(np.zeros((n_t, hkv * hd), np.float32))
        cache.store(0, dr.Pass(dev.ctx, range(n_t)), z, z)
        q = dev.put(np.zeros((n_c, h * hd), np.float32))
        cache.attention(0, [(q, dev.empty(n_c * h * hd), dr.Pass(dev.ctx, range(n_p, n_t)))], h,
                        sliding_window=window, scale=1 / math.sqrt(hd))
        info = dev.ctx.last_launch()
        say(f"h {h}/{hkv} keys {n_t} window {window}: launch {info}")
        assert info["kernel"] == dr.KERNEL_STREAMS, info
        assert info["rows_per_wave"] == rows and info["n_split"] == n_split, (h, hkv, n_t, window, info)
        del cache


def test_planner_hd256_key_band(dev):
    """Head dim 256: the per-wave-stream kernel with two in-kernel-merged key
    splits where those splits fill the chip in one round and every row
    block's key band (the union of the rows' windows, from the passes'
    positions) holds at most 4608 keys; the staged kernel's 64-row split
    blocks otherwise.  Then the planner's choice on one such shape against
    the oracle."""
    hd = 256
    # (h, hkv, n_prompt, n_canvas, window, kernel, n_split or 0 for any)
    cases = (
        (16, 8, 4096, 256, None, dr.KERNEL_STREAMS, 2),   # C5 global: 4352 keys
        (16, 8, 8192, 256, None, dr.KERNEL_STAGED, 0),    # 8448 keys
        (16, 8, 6000, 256, 2500, dr.KERNEL_STREAMS, 2),   # band [3501, 6256): 2755 keys
        (16, 8, 6000, 256, 5000, dr.KERNEL_STAGED, 0),    # band [1001, 6256): 5255 keys
        (32, 16, 4096, 256, None, dr.KERNEL_STAGED, 0),   # 256 one-block workgroups: no room to split
    )
    for h, hkv, n_p, n_c, window, want, n_split in cases:
        n_t = n_p + n_c
        cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
        z = dev.put(np.zeros((n_t, hkv * hd), np.float32))
        cache.store(0, dr.Pass(dev.ctx, range(n_t)), z, z)
        q = dev.put(np.zeros((n_c, h * hd), np.float32))
        cache.attention(0, [(q, dev.empty(n_c * h * hd), dr.Pass(dev.ctx, range(n_p, n_t)))], h,
                        sliding_window=window, scale=1 / math.sqrt(hd))
        info = dev.ctx.last_launch()
        say(f"h {h}/{hkv} keys {n_t} window {window}: launch {info}")
        assert info["kernel"] == want, (h, hkv, n_t, window)
        if n_split:
            assert info["n_split"] == n_split and info["split_merge"] == 2
        del cache
    got, wants, info = _run(dev, "global_auto", dr.KERNEL_AUTO, hd=256)
    say(f"global_auto: launch {info}")
    assert info["kernel"] == dr.KERNEL_STREAMS and info["n_split"] == 2 and info["split_merge"] == 2
    for g, w in zip(got, wants):
        mx, mean = err_stats(g, w)
        say(f"  max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (mx, mean)
