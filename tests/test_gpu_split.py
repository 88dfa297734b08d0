"""StepCache::split_active (src/model/cache.rs:85-114) on the device
(dr_cache_split_active_dev), against the oracle's or_split_active, which
tests/test_oracle.py pins to the reference's own test case (tests.rs:39-68)
and to its vicinity and decay rules: the same active / cached lists, bit for
bit, step after step; host and device calls mixed on one slot; and passes
that drive the cached attention exactly as host-built ones do.  Needs an
MI355X.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc

from test_gpu_parity import check, dev, say, torch  # noqa: F401

pytestmark = pytest.mark.gpu

MASK = 4  # mask_token_id (docs/diffusiongemma.md:19); any token id works


def _next_seq(rng, seq, n_prompt):
    """One denoise step of a sampler: commit some masked canvas tokens, re-mask
    a few committed ones (remasking samplers) and change a few others."""
    s = seq.copy()
    canvas = np.arange(n_prompt, s.size)
    masked = canvas[s[canvas] == MASK]
    if masked.size:
        commit = rng.choice(masked, max(1, masked.size // 4), replace=False)
        s[commit] = rng.integers(5, 30000, commit.size)
    done = canvas[s[canvas] != MASK]
    if done.size > 8:
        s[rng.choice(done, 2, replace=False)] = MASK
        s[rng.choice(done, 2, replace=False)] = rng.integers(5, 30000, 2)
    return s.astype(np.int32)


@pytest.mark.parametrize("n_total,n,vicinity", [(768, 768, 0), (3000, 3000, 5),
                                                (4352, 4000, 64), (100, 37, 1000), (2048, 2048, 1)])
def test_split_active_dev_matches_oracle(dev, n_total, n, vicinity):
    rng = np.random.default_rng(n_total + vicinity)
    n_prompt = n // 3
    cache = dr.StepCache(dev.ctx, n_total, [1], [64])
    cache.set_vicinity(vicinity)
    prev = np.full(n, -1, np.int32)
    lc = np.full(n, -1, np.int32)
    seq = rng.integers(5, 30000, n).astype(np.int32)
    seq[n_prompt:] = MASK
    pa, pc = dr.Pass(dev.ctx, []), dr.Pass(dev.ctx, [])
    for step in range(10):
        is_masked = (seq == MASK).astype(np.uint8)
        want_a, want_c = orc.split_active(prev, lc, seq, is_masked, step, vicinity)
        na, nc = cache.split_active_dev(dev.put(seq), dev.put(is_masked), n, step, pa, pc)
        say(f"n {n} vicinity {vicinity} step {step}: {na} active, {nc} cached")
        assert (na, nc) == (len(want_a), len(want_c))
        assert pa.positions() == want_a
        assert pc.positions() == want_c
        # update_seq after the pass (sampler order); the slot holds n_total tokens
        full = np.full(n_total, 7, np.int32)
        full[:n] = seq
        cache.update_seq_dev(dev.put(full))
        prev = seq.copy()
        seq = _next_seq(rng, seq, n_prompt)


def test_split_state_moves_between_host_and_device(dev):
    """Host and device calls mixed on one slot give the oracle's sequence of
    splits: the state (prev_seq, last_changed) follows the call."""
    rng = np.random.default_rng(77)
    n = 1500
    cache = dr.StepCache(dev.ctx, n, [1], [64])
    cache.set_vicinity(3)
    prev = np.full(n, -1, np.int32)
    lc = np.full(n, -1, np.int32)
    seq = rng.integers(5, 30000, n).astype(np.int32)
    seq[500:] = MASK
    pa, pc = dr.Pass(dev.ctx, []), dr.Pass(dev.ctx, [])
    for step in range(12):
        is_masked = (seq == MASK).astype(np.uint8)
        want = orc.split_active(prev, lc, seq, is_masked, step, 3)
        if step % 3 == 0:
            got = cache.split_active(seq, is_masked, step)
        else:
            cache.split_active_dev(dev.put(seq), dev.put(is_masked), n, step, pa, pc)
            got = (pa.positions(), pc.positions())
        assert got == want, step
        if step % 2 == 0:
            cache.update_seq(seq)
        else:
            cache.update_seq_dev(dev.put(seq))
        prev = seq.copy()
        seq = _next_seq(rng, seq, 500)


def test_split_active_dev_passes_drive_the_step(dev):
    """A denoise step whose split comes from the device: the active pass
    stores the fresh rows and queries the cache, with the same outputs, bit
    for bit, as the host-built pass of the same positions."""
    rng = np.random.default_rng(78)
    h, hkv, hd, n_p, n_c = 8, 2, 128, 400, 200
    n_t = n_p + n_c
    kvs = hkv * hd
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    K = rng.standard_normal((n_t, kvs), dtype=np.float32)
    V = rng.standard_normal((n_t, kvs), dtype=np.float32)
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    seq = rng.integers(5, 30000, n_t).astype(np.int32)
    seq[n_p:] = MASK
    cache.update_seq_dev(dev.put(seq))
    seq = _next_seq(rng, seq, n_p)
    is_masked = (seq == MASK).astype(np.uint8)
    pa, pc = dr.Pass(dev.ctx, []), dr.Pass(dev.ctx, [])
    na, _ = cache.split_active_dev(dev.put(seq), dev.put(is_masked), n_t, 1, pa, pc)
    act = pa.positions()
    say(f"device split: {na} active of {n_t}")
    host_pass = dr.Pass(dev.ctx, act)
    Q = rng.standard_normal((na, h * hd), dtype=np.float32)
    Ka = rng.standard_normal((na, kvs), dtype=np.float32)
    Va = rng.standard_normal((na, kvs), dtype=np.float32)
    outs = []
    for p in (pa, host_pass):
        out = dev.empty(na * h * hd)
        cache.step(0, [(dev.put(Q), out, p, dev.put(Ka), dev.put(Va))], h, scale=1 / math.sqrt(hd))
        outs.append(dev.get(out))
    assert np.array_equal(outs[0], outs[1])
