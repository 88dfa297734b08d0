"""Calls that could overlap on the device, and the guards that keep them
apart (include/dr_attn.h: dr_ctx_set_stream, dr_attention_cached_noalloc,
DR_ERR_BUSY):

- a context that switches streams: the new stream waits for the work queued
  on the old one, so the context's split tickets and workspace are never in
  use on both;
- dr_attention_cached_noalloc from two contexts on two streams: the GPU's one
  scratch array is used by one call at a time;
- two host threads on one context: each call either runs alone or returns
  DR_ERR_BUSY.

Every output is compared bit for bit with the same call made alone (same
plan, same summation order).  Needs an MI355X.
"""
from __future__ import annotations

import math
import sys
import threading

import numpy as np
import pytest

import dr_attn as dr

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    if not torch.cuda.is_available() or dr.device_count() == 0:
        pytest.skip("no GPU visible")
    dr.load()
    return torch


def _problem(torch, ctx, stream, seed, h=16, hkv=8, hd=256, n_p=1500, n_c=128):
    """A cache with random K/V and n_sets query sets; returns (cache, pass, Qs)."""
    rng = np.random.default_rng(seed)
    n_t = n_p + n_c
    kvs = hkv * hd
    cache = dr.StepCache(ctx, n_t, [hkv], [hd])
    with torch.cuda.stream(stream):
        K = torch.from_numpy(rng.standard_normal((n_t, kvs), dtype=np.float32)).cuda()
        V = torch.from_numpy(rng.standard_normal((n_t, kvs), dtype=np.float32)).cuda()
        Qs = [torch.from_numpy(rng.standard_normal((n_c, h * hd), dtype=np.float32)).cuda() for _ in range(3)]
    cache.store(0, dr.Pass(ctx, range(n_t)), K, V)
    stream.synchronize()
    return cache, dr.Pass(ctx, range(n_p, n_t)), Qs, (h, hd, n_c)


def _empty(torch, stream, n):
    with torch.cuda.stream(stream):
        return torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")


def test_stream_switch_orders_the_contexts_work(torch_mod):
    """Split attention (in-kernel merge: the context's tickets and split
    workspace) on stream A, then at once on stream B after a switch, with
    only B synchronised: every output equals the same call made alone."""
    torch = torch_mod
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ctx = dr.Context(0)
    ctx.set_stream(sa.cuda_stream)
    ctx.set_split(2)
    try:
        cache, pc, Qs, (h, hd, n_c) = _problem(torch, ctx, sa, 11)
        scale = 1 / math.sqrt(hd)
        want = []
        for q in Qs:
            o = _empty(torch, sa, n_c * h * hd)
            cache.attention(0, [(q, o, pc)], h, scale=scale)
            sa.synchronize()
            want.append(o.cpu().numpy())
        info = ctx.last_launch()
        say(f"launch {info}")
        assert info["n_split"] == 2 and info["split_merge"] == 2
        for rep in range(3):
            outs = []
            for i, q in enumerate(Qs):
                s = (sa, sb)[(i + rep) % 2]
                ctx.set_stream(s.cuda_stream)
                o = _empty(torch, s, n_c * h * hd)
                cache.attention(0, [(q, o, pc)], h, scale=scale)
                outs.append(o)
            last = (sa, sb)[(len(Qs) - 1 + rep) % 2]
            last.synchronize()  # the other stream's calls are ordered before it
            for i, o in enumerate(outs):
                got = o.cpu().numpy()
                assert np.array_equal(got, want[i]), (rep, i)
    finally:
        ctx.set_stream(0)
        ctx.set_split(0)


def test_noalloc_calls_on_two_streams_take_turns(torch_mod):
    """Two contexts on two streams alternate dr_attention_cached_noalloc
    calls (forced key splits: the partials live in the GPU's one scratch
    array) with no host synchronisation between them."""
    torch = torch_mod
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ca, cb = dr.Context(0), dr.Context(0)
    ca.set_stream(sa.cuda_stream)
    cb.set_stream(sb.cuda_stream)
    for c in (ca, cb):
        c.set_split(4)
        c.set_split_merge(False)  # partials through split_merge_kernel: the whole scratch round trip
    pa = _problem(torch, ca, sa, 21)
    pb = _problem(torch, cb, sb, 22, h=8, hkv=8, hd=128, n_p=3000, n_c=200)
    want = {}
    for name, c, s, (cache, pc, Qs, (h, hd, n_c)) in (("a", ca, sa, pa), ("b", cb, sb, pb)):
        for i, q in enumerate(Qs):
            o = _empty(torch, s, n_c * h * hd)
            cache.attention(0, [(q, o, pc)], h, scale=1 / math.sqrt(hd))
            s.synchronize()
            want[name, i] = o.cpu().numpy()
        say(f"{name}: launch {c.last_launch()}")
        assert c.last_launch()["n_split"] == 4
    outs = {}
    for rep in range(4):
        for i in range(3):
            for name, s, (cache, pc, Qs, (h, hd, n_c)) in (("a", sa, pa), ("b", sb, pb)):
                o = _empty(torch, s, n_c * h * hd)
                cache.attention(0, [(Qs[i], o, pc)], h, scale=1 / math.sqrt(hd), noalloc=True)
                outs[rep, name, i] = o
    sa.synchronize()
    sb.synchronize()
    for (rep, name, i), o in outs.items():
        assert np.array_equal(o.cpu().numpy(), want[name, i]), (rep, name, i)


def test_two_threads_on_one_context(torch_mod):
    """Two host threads call into one context: each call runs alone and is
    right, or is refused with DR_ERR_BUSY; nothing in between."""
    torch = torch_mod
    st = torch.cuda.Stream()
    ctx = dr.Context(0)
    ctx.set_stream(st.cuda_stream)
    cache, pc, Qs, (h, hd, n_c) = _problem(torch, ctx, st, 31, h=8, hkv=4, hd=128, n_p=700, n_c=64)
    scale = 1 / math.sqrt(hd)
    o = _empty(torch, st, n_c * h * hd)
    cache.attention(0, [(Qs[0], o, pc)], h, scale=scale)
    st.synchronize()
    want = o.cpu().numpy()
    outs = [[_empty(torch, st, n_c * h * hd) for _ in range(40)] for _ in range(2)]
    done = [[False] * 40 for _ in range(2)]
    busy = [0, 0]
    errors = []

    def run(t):
        try:
            for i in range(40):
                try:
                    cache.attention(0, [(Qs[0], outs[t][i], pc)], h, scale=scale)
                    done[t][i] = True
                except dr.DrError as e:
                    if "DR_ERR_BUSY" not in str(e):
                        raise
                    busy[t] += 1
        except Exception as e:  # reported below
            errors.append(repr(e))

    th = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    st.synchronize()
    say(f"refused as busy: {busy}")
    assert not errors, errors
    for t in range(2):
        for i in range(40):
            if done[t][i]:
                assert np.array_equal(outs[t][i].cpu().numpy(), want), (t, i)
    assert sum(sum(d) for d in done) + sum(busy) == 80
